/*
 * CPU oracle for the quantized MatVec hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's scalar (and AVX2)
 * kernels, giving the expected values to tests/ and __graft_entry__.smoke() and serving as the timed CPU
 * baseline leg of bench.py. The product (satori_amd/libsatori_hip.so) never links, loads or
 * calls anything in this directory.
 *
 * Each function cites the reference file:line it restates (paths relative to the reference
 * repository root). Evaluation order follows the C# source term by term; the file is compiled
 * with -ffp-contract=off so no multiply-add is fused that the C# JIT would not fuse (RyuJIT
 * fuses only explicit Fma.MultiplyAdd calls).
 *
 * Every function is pinned by tests/test_oracle.py against the reference's golden fixtures, its tests'
 * known answers, FP64 brute force or an exact integer identity; none is "parity unpinned".
 */
#ifndef SATORI_ORACLE_H
#define SATORI_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: 0 ok; 1 ArgumentException; 2 ArgumentOutOfRangeException; 3 InvalidDataException;
 * 9 OverflowException. They mirror the exceptions the reference throws. */
enum { OR_OK = 0, OR_ARGUMENT = 1, OR_OUT_OF_RANGE = 2, OR_INVALID_DATA = 3, OR_OVERFLOW = 9 };

/* Formats: values of BlockQuantization (src/Satori.Core/BlockQuantization.cs:3). */
enum { OR_Q8_0 = 0, OR_Q4_0 = 1, OR_Q4_K = 2, OR_Q6_K = 3 };

float or_half_to_float(uint16_t bits);

/* ---- Ternary2 ---- */
int64_t or_t2_byte_length(int rows, int columns, int block_size);
int or_t2_quantize(const float* weights, int rows, int columns, int block_size, uint8_t* out, size_t out_len);
int or_t2_validate(const uint8_t* data, size_t len, int rows, int columns, int block_size);
void or_t2_dequantize(const uint8_t* data, int rows, int columns, int block_size, float* out);
void or_t2_matvec_scalar(const uint8_t* data, int rows, int columns, int block_size, const float* x, float* y);
void or_t2_matvec_avx2(const uint8_t* data, int rows, int columns, int block_size, const float* x, float* y);
void or_stq2_write_header(uint8_t header[32], int rows, int columns, int block_size);
int or_stq2_read_header(const uint8_t header[32], int* rows, int* columns, int* block_size);

/* Ternary bitplane layout (src/Satori.Core/TernaryBitplaneMatrix.cs, TernaryBitplaneMatVec.cs): each
 * block is the FP32 scale, then B/8 bytes of positive-plane bits, then B/8 bytes of negative-plane bits
 * (bit i % 8 of byte i / 8 is weight i). */
int or_tb_validate(const uint8_t* data, size_t len, int rows, int columns, int block_size);
void or_tb_from_t2(const uint8_t* t2, int rows, int columns, int block_size, uint8_t* out);
void or_tb_to_t2(const uint8_t* tb, int rows, int columns, int block_size, uint8_t* out);
void or_tb_matvec_scalar(const uint8_t* data, int rows, int columns, int block_size, const float* x, float* y);

/* ---- GGUF block formats ---- */
int64_t or_q_byte_length(int rows, int columns, int format);
int or_q_validate(const uint8_t* data, size_t len, int rows, int columns, int format);
void or_q_matvec_scalar(const uint8_t* data, int rows, int columns, int format, const float* x, float* y);
void or_q_matvec_avx2(const uint8_t* data, int rows, int columns, int format, const float* x, float* y);
void or_q_decode_block(const uint8_t* block, int format, float* out);

void or_q4k_get_scale_min(int j, const uint8_t* scales, int* scale, int* min);
float or_q4k_dot_block(const uint8_t* block, const float* x);
void or_q4k_decode_block(const uint8_t* block, float* w);
int32_t or_q4k_dot_product(const uint8_t* block, const uint8_t* activation);
int32_t or_q4k_min_product(const uint8_t* block, const uint8_t* activation);
float or_q4k_dot_block_quantized(const uint8_t* block, const uint8_t* activation);

float or_q6k_dot_block(const uint8_t* block, const float* x);
void or_q6k_decode_block(const uint8_t* block, float* w);
int32_t or_q6k_dot_product(const uint8_t* block, const uint8_t* activation);
float or_q6k_dot_block_quantized(const uint8_t* block, const uint8_t* activation);

void or_q8k_quantize_block(const float* x, uint8_t* block);
int or_q8k_quantize_row(const float* x, int columns, uint8_t* out, size_t out_len);

/* Batched projection (QuantizedMatVec.ExecuteBatch): x [P][C] -> y [P][R]. */
int or_q_matvec_batch(const uint8_t* data, int rows, int columns, int format, const float* x, int positions,
                      float* y);

/* K formats at one position against a Q8_K row, AVX2 integer kernel (the decode hot loop). */
void or_qk_matvec_quantized_avx2(const uint8_t* weights, int rows, int columns, int format,
                                 const uint8_t* activations, float* y);
/* ExecuteQuantizedTiled over 1..256 positions: activations [positions][columns / 256 * 292], output
 * [positions][rows] (QuantizedKAvx2Kernel.cs:47-99). */
void or_qk_matvec_quantized_tiled_avx2(const uint8_t* weights, int rows, int columns, int format,
                                       const uint8_t* activations, int positions, float* output);

/* NumericalCorpus.RandomMatrix: xorshift32 seed 1729 corpus (weights then input). */
/* TransformerOps (src/Satori.Core/TransformerOps.cs): FP64 arithmetic in the reference's order, FP32 out. */
void or_rms_norm(const float* input, const float* weights, float epsilon, int length, float* output);
void or_rms_norm_heads(float* vector, const float* weights, float epsilon, int head_dim, int length);
void or_rope(float* vector, int length, int head_dim, int position);
void or_rope_half(float* vector, int length, int head_dim, int position, double base, int rotary);
void or_swiglu(const float* gate, const float* up, int length, float* output);
void or_add(const float* left, const float* right, int length, float* output);
void or_grouped_attention(const float* query, const float* keys, const float* values, int query_heads,
                          int kv_heads, int head_dim, int tokens, double* scores, float* output);
/* QuantizedRow.DecodeRow (src/Satori.Core/QuantizedRow.cs:59-70). */
void or_q_decode_row(const uint8_t* row, int columns, int format, float* output);

void or_corpus_random_matrix(int rows, int columns, float* weights, float* input);

#ifdef __cplusplus
}
#endif
#endif
