/*
 * CPU oracle, AVX2 half: restatement of the reference's AVX2 kernels with the same intrinsic
 * sequence, so that bench.py can time the reference's vector path on the host beside the GPU
 * ("restated reference AVX2"), and tests can check it against the scalar restatement.
 *
 * TEST INFRASTRUCTURE ONLY (see satori_oracle.h). Built with -O3 -mavx2 -mfma -ffp-contract=off.
 */
#include <immintrin.h>
#include <string.h>

#include "satori_oracle.h"

static float rdf32(const uint8_t* p) { float f; memcpy(&f, p, 4); return f; }
static uint16_t rd16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }
static uint64_t rd64u(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

/* The three-step horizontal float sum used by every AVX2 kernel
 * (Ternary2Avx2Kernel.cs:42-45, QuantizedAvx2Kernel.cs:46-48, QuantizedKAvx2Kernel.cs:341-347). */
static inline float hsum(__m256 v) {
    __m128 halves = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    halves = _mm_add_ps(halves, _mm_shuffle_ps(halves, halves, 0x4E));
    halves = _mm_add_ss(halves, _mm_shuffle_ps(halves, halves, 0xB1));
    return _mm_cvtss_f32(halves);
}

/* Integer horizontal sum (QuantizedKAvx2Kernel.cs:130-136). */
static inline int hsum_i32(__m256i v) {
    __m128i halves = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    halves = _mm_add_epi32(halves, _mm_shuffle_epi32(halves, 0x4E));
    halves = _mm_add_epi32(halves, _mm_shuffle_epi32(halves, 0xB1));
    return _mm_cvtsi128_si32(halves);
}

/* Ternary2Avx2Kernel.Execute (src/Satori.Core/Ternary2Avx2Kernel.cs:10-56). */
void or_t2_matvec_avx2(const uint8_t* data, int rows, int columns, int block_size, const float* input, float* output) {
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4;
    const __m256i shifts = _mm256_setr_epi32(0, 2, 4, 6, 8, 10, 12, 14);
    const __m256i mask = _mm256_set1_epi32(3);
    const __m256i negative_code = _mm256_set1_epi32(2);
    const __m256i sign_bit = _mm256_set1_epi32((int)0x80000000u);
    for (int row = 0; row < rows; row++) {
        float sum = 0;
        for (int block = 0; block < blocks; block++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks + block) * stride;
            float scale = rdf32(bytes);
            int column = block * block_size;
            int count = block_size < columns - column ? block_size : columns - column;
            __m256 accumulator = _mm256_setzero_ps();
            int i = 0;
            for (; i <= count - 8; i += 8) {
                unsigned packed = rd16(bytes + 4 + i / 4);
                __m256i codes = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32((int)packed), shifts), mask);
                __m256i zero = _mm256_cmpeq_epi32(codes, _mm256_setzero_si256());
                __m256i negative = _mm256_and_si256(_mm256_cmpeq_epi32(codes, negative_code), sign_bit);
                __m256 activations = _mm256_loadu_ps(input + column + i);
                __m256 signed_ = _mm256_xor_ps(activations, _mm256_castsi256_ps(negative));
                accumulator = _mm256_add_ps(accumulator, _mm256_andnot_ps(_mm256_castsi256_ps(zero), signed_));
            }
            float partial = hsum(accumulator);
            for (; i < count; i++) {
                int code = (bytes[4 + i / 4] >> (2 * (i % 4))) & 3;
                if (code == 1) partial += input[column + i];
                else if (code == 2) partial -= input[column + i];
            }
            sum += partial * scale;
        }
        output[row] = sum;
    }
}

/* QuantizedAvx2Kernel.Execute (src/Satori.Core/QuantizedAvx2Kernel.cs:10-53): Q8_0 and Q4_0. */
static void q_legacy_avx2(const uint8_t* data, int rows, int columns, int format, int block_bytes,
                          const float* source, float* output) {
    const __m256i nibble_mask = _mm256_set1_epi32(15);
    const __m256i bias = _mm256_set1_epi32(8);
    int blocks_per_row = columns / 32;
    for (int row = 0; row < rows; row++) {
        float total = 0;
        for (int b = 0; b < blocks_per_row; b++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks_per_row + b) * block_bytes;
            __m256 accumulator = _mm256_setzero_ps();
            if (format == OR_Q8_0) {
                for (int j = 0; j < 32; j += 8) {
                    __m128i packed = _mm_cvtsi64_si128((long long)rd64u(bytes + 2 + j));
                    __m256 codes = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(packed));
                    __m256 values = _mm256_loadu_ps(source + b * 32 + j);
                    accumulator = _mm256_add_ps(accumulator, _mm256_mul_ps(codes, values));
                }
            } else {
                for (int j = 0; j < 16; j += 8) {
                    __m128i packed = _mm_cvtsi64_si128((long long)rd64u(bytes + 2 + j));
                    __m256i codes = _mm256_cvtepu8_epi32(packed);
                    __m256 low = _mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_and_si256(codes, nibble_mask), bias));
                    __m256 high = _mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_srli_epi32(codes, 4), bias));
                    accumulator = _mm256_add_ps(accumulator, _mm256_mul_ps(low, _mm256_loadu_ps(source + b * 32 + j)));
                    accumulator = _mm256_add_ps(accumulator, _mm256_mul_ps(high, _mm256_loadu_ps(source + b * 32 + j + 16)));
                }
            }
            total += or_half_to_float(rd16(bytes)) * hsum(accumulator);
        }
        output[row] = total;
    }
}

/* QuantizedKAvx2Kernel.ExecuteQ4K (src/Satori.Core/QuantizedKAvx2Kernel.cs:225-269). */
static void q4k_float_avx2(const uint8_t* data, int rows, int columns, const float* source, float* output) {
    const __m256i low_mask = _mm256_set1_epi32(15);
    int blocks_per_row = columns / 256;
    for (int row = 0; row < rows; row++) {
        float total = 0;
        for (int b = 0; b < blocks_per_row; b++) {
            const uint8_t* block = data + ((int64_t)row * blocks_per_row + b) * 144;
            float d = or_half_to_float(rd16(block));
            float dmin = or_half_to_float(rd16(block + 2));
            const uint8_t* scales = block + 4;
            const uint8_t* qs = block + 16;
            int column_base = b * 256;
            for (int g = 0; g < 4; g++) {
                const uint8_t* q = qs + g * 32;
                int sm[4];
                or_q4k_get_scale_min(g * 2, scales, &sm[0], &sm[2]);
                or_q4k_get_scale_min(g * 2 + 1, scales, &sm[1], &sm[3]);
                __m256 low_scale = _mm256_set1_ps(d * (float)sm[0]);
                __m256 low_bias = _mm256_set1_ps(dmin * (float)sm[2]);
                __m256 high_scale = _mm256_set1_ps(d * (float)sm[1]);
                __m256 high_bias = _mm256_set1_ps(dmin * (float)sm[3]);
                __m256 accumulator = _mm256_setzero_ps();
                for (int j = 0; j < 32; j += 8) {
                    __m128i packed = _mm_cvtsi64_si128((long long)rd64u(q + j));
                    __m256i codes = _mm256_cvtepu8_epi32(packed);
                    __m256 low = _mm256_cvtepi32_ps(_mm256_and_si256(codes, low_mask));
                    __m256 high = _mm256_cvtepi32_ps(_mm256_srli_epi32(codes, 4));
                    __m256 low_w = _mm256_sub_ps(_mm256_mul_ps(low, low_scale), low_bias);
                    __m256 high_w = _mm256_sub_ps(_mm256_mul_ps(high, high_scale), high_bias);
                    accumulator = _mm256_add_ps(accumulator, _mm256_mul_ps(low_w, _mm256_loadu_ps(source + column_base + g * 64 + j)));
                    accumulator = _mm256_add_ps(accumulator, _mm256_mul_ps(high_w, _mm256_loadu_ps(source + column_base + g * 64 + 32 + j)));
                }
                total += hsum(accumulator);
            }
        }
        output[row] = total;
    }
}

/* QuantizedKAvx2Kernel.Build (src/Satori.Core/QuantizedKAvx2Kernel.cs:333-339). */
static inline __m256 q6_build(__m256i ql, int nibble, __m256i qh_field) {
    __m256i q = nibble == 0 ? _mm256_and_si256(ql, _mm256_set1_epi32(15)) : _mm256_srli_epi32(ql, 4);
    __m256i code = _mm256_or_si256(_mm256_slli_epi32(qh_field, 4), q);
    return _mm256_cvtepi32_ps(_mm256_sub_epi32(code, _mm256_set1_epi32(32)));
}

/* QuantizedKAvx2Kernel.ExecuteQ6K (src/Satori.Core/QuantizedKAvx2Kernel.cs:271-328). */
static void q6k_float_avx2(const uint8_t* data, int rows, int columns, const float* source, float* output) {
    const __m256i three = _mm256_set1_epi32(3);
    int blocks_per_row = columns / 256;
    for (int row = 0; row < rows; row++) {
        float total = 0;
        for (int b = 0; b < blocks_per_row; b++) {
            const uint8_t* block = data + ((int64_t)row * blocks_per_row + b) * 210;
            float d = or_half_to_float(rd16(block + 208));
            const uint8_t* ql = block;
            const uint8_t* qh = block + 128;
            const int8_t* scales = (const int8_t*)(block + 192);
            int column_base = b * 256;
            for (int half = 0; half < 2; half++) {
                const uint8_t* lql = ql + half * 64;
                const uint8_t* lqh = qh + half * 32;
                const int8_t* lsc = scales + half * 8;
                int base = column_base + half * 128;
                for (int l = 0; l < 32; l += 8) {
                    int sub = l / 16;
                    __m256i a1i = _mm256_cvtepu8_epi32(_mm_cvtsi64_si128((long long)rd64u(lql + l)));
                    __m256i a2i = _mm256_cvtepu8_epi32(_mm_cvtsi64_si128((long long)rd64u(lql + l + 32)));
                    __m256i bx = _mm256_cvtepu8_epi32(_mm_cvtsi64_si128((long long)rd64u(lqh + l)));
                    __m256i qh0 = _mm256_and_si256(bx, three);
                    __m256i qh1 = _mm256_and_si256(_mm256_srli_epi32(bx, 2), three);
                    __m256i qh2 = _mm256_and_si256(_mm256_srli_epi32(bx, 4), three);
                    __m256i qh3 = _mm256_and_si256(_mm256_srli_epi32(bx, 6), three);
                    __m256 c1 = q6_build(a1i, 0, qh0), c2 = q6_build(a2i, 0, qh1);
                    __m256 c3 = q6_build(a1i, 4, qh2), c4 = q6_build(a2i, 4, qh3);
                    __m256 w1 = _mm256_mul_ps(c1, _mm256_set1_ps(d * (float)lsc[sub + 0]));
                    __m256 w2 = _mm256_mul_ps(c2, _mm256_set1_ps(d * (float)lsc[sub + 2]));
                    __m256 w3 = _mm256_mul_ps(c3, _mm256_set1_ps(d * (float)lsc[sub + 4]));
                    __m256 w4 = _mm256_mul_ps(c4, _mm256_set1_ps(d * (float)lsc[sub + 6]));
                    __m256 acc = _mm256_setzero_ps();
                    acc = _mm256_add_ps(acc, _mm256_mul_ps(w1, _mm256_loadu_ps(source + base + l)));
                    acc = _mm256_add_ps(acc, _mm256_mul_ps(w2, _mm256_loadu_ps(source + base + l + 32)));
                    acc = _mm256_add_ps(acc, _mm256_mul_ps(w3, _mm256_loadu_ps(source + base + l + 64)));
                    acc = _mm256_add_ps(acc, _mm256_mul_ps(w4, _mm256_loadu_ps(source + base + l + 96)));
                    total += hsum(acc);
                }
            }
        }
        output[row] = total;
    }
}

/* QuantizedMatVec.ExecuteAvx2 dispatch (src/Satori.Core/QuantizedMatVec.cs:18-26). */
void or_q_matvec_avx2(const uint8_t* data, int rows, int columns, int format, const float* x, float* y) {
    switch (format) {
        case OR_Q8_0: q_legacy_avx2(data, rows, columns, format, 34, x, y); break;
        case OR_Q4_0: q_legacy_avx2(data, rows, columns, format, 18, x, y); break;
        case OR_Q4_K: q4k_float_avx2(data, rows, columns, x, y); break;
        case OR_Q6_K: q6k_float_avx2(data, rows, columns, x, y); break;
    }
}

/* QuantizedKAvx2Kernel.DotQuantizedQ4K (src/Satori.Core/QuantizedKAvx2Kernel.cs:108-128). */
static float q4k_dot_quantized_avx2(const uint8_t* weights, const uint8_t* activation, const int* scales,
                                    const int* mins, float d, float dmin) {
    const uint8_t* quants = weights + 16;
    const int8_t* codes = (const int8_t*)(activation + 4);
    const int16_t* sums = (const int16_t*)(activation + 260);
    const __m256i low_mask = _mm256_set1_epi8(15);
    __m256i accumulator = _mm256_setzero_si256();
    int min_total = 0;
    for (int sub = 0; sub < 8; sub++) {
        __m256i packed = _mm256_loadu_si256((const __m256i*)(quants + sub / 2 * 32));
        __m256i nibbles = (sub & 1) == 0 ? _mm256_and_si256(packed, low_mask)
                                         : _mm256_and_si256(_mm256_srli_epi16(packed, 4), low_mask);
        __m256i group_codes = _mm256_loadu_si256((const __m256i*)(codes + sub * 32));
        __m256i pairs = _mm256_maddubs_epi16(nibbles, group_codes);
        accumulator = _mm256_add_epi32(accumulator, _mm256_madd_epi16(pairs, _mm256_set1_epi16((short)scales[sub])));
        min_total += mins[sub] * (sums[sub * 2] + sums[sub * 2 + 1]);
    }
    return d * (float)hsum_i32(accumulator) - dmin * (float)min_total;
}

/* QuantizedKAvx2Kernel.DotProductQ6K (src/Satori.Core/QuantizedKAvx2Kernel.cs:163-202). */
static int q6k_dot_product_avx2(const uint8_t* block, const uint8_t* activation) {
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* scales = (const int8_t*)(block + 192);
    const int8_t* codes = (const int8_t*)(activation + 4);
    const int16_t* sums = (const int16_t*)(activation + 260);
    const __m256i low_nibble = _mm256_set1_epi8(0x0F);
    const __m256i two_bits = _mm256_set1_epi8(0x03);
    const __m256i upper_half = _mm256_set1_epi8(0x30);
    __m256i accumulator = _mm256_setzero_si256();
    int centring = 0;
    for (int group = 0; group < 8; group++) {
        int half = group / 4, quarter = group % 4;
        __m256i packed = _mm256_loadu_si256((const __m256i*)(ql + half * 64 + (quarter % 2) * 32));
        __m256i nibbles = quarter >= 2 ? _mm256_and_si256(_mm256_srli_epi16(packed, 4), low_nibble)
                                       : _mm256_and_si256(packed, low_nibble);
        __m256i hword = _mm256_loadu_si256((const __m256i*)(qh + half * 32));
        __m256i field = quarter == 0 ? hword
                      : quarter == 1 ? _mm256_srli_epi16(hword, 2)
                      : quarter == 2 ? _mm256_srli_epi16(hword, 4)
                                     : _mm256_srli_epi16(hword, 6);
        __m256i high = _mm256_and_si256(field, two_bits);
        __m256i quants = _mm256_or_si256(nibbles, _mm256_and_si256(_mm256_slli_epi16(high, 4), upper_half));
        __m256i group_codes = _mm256_loadu_si256((const __m256i*)(codes + group * 32));
        __m256i pairs = _mm256_maddubs_epi16(quants, group_codes);
        int8_t low = scales[group * 2], high_scale = scales[group * 2 + 1];
        __m256i lane_scales = _mm256_setr_m128i(_mm_set1_epi16(low), _mm_set1_epi16(high_scale));
        accumulator = _mm256_add_epi32(accumulator, _mm256_madd_epi16(pairs, lane_scales));
        centring += 32 * (low * sums[group * 2] + high_scale * sums[group * 2 + 1]);
    }
    return hsum_i32(accumulator) - centring;
}

/* QuantizedKAvx2Kernel.ExecuteQuantizedTiled at one position over all rows, with the activation
 * already quantized by Q8KCodec.QuantizeRow (QuantizedKAvx2Kernel.cs:47-99). */
void or_qk_matvec_quantized_avx2(const uint8_t* weights, int rows, int columns, int format,
                                 const uint8_t* activations, float* output) {
    int blocks_per_row = columns / 256;
    int block_bytes = format == OR_Q4_K ? 144 : 210;
    int q4 = format == OR_Q4_K;
    int sub_scales[8], sub_mins[8];
    for (int row = 0; row < rows; row++) {
        float accumulator = 0;
        const uint8_t* weight_row = weights + (int64_t)row * blocks_per_row * block_bytes;
        for (int block = 0; block < blocks_per_row; block++) {
            const uint8_t* bw = weight_row + block * block_bytes;
            float d, dmin = 0;
            if (q4) {
                for (int sub = 0; sub < 8; sub++) or_q4k_get_scale_min(sub, bw + 4, &sub_scales[sub], &sub_mins[sub]);
                d = or_half_to_float(rd16(bw));
                dmin = or_half_to_float(rd16(bw + 2));
            } else {
                d = or_half_to_float(rd16(bw + 208));
            }
            const uint8_t* activation = activations + (int64_t)block * 292;
            float activation_scale = rdf32(activation);
            if (activation_scale == 0) continue;
            accumulator += q4 ? q4k_dot_quantized_avx2(bw, activation, sub_scales, sub_mins, d * activation_scale,
                                                       dmin * activation_scale)
                              : activation_scale * d * (float)q6k_dot_product_avx2(bw, activation);
        }
        output[row] = accumulator;
    }
}

/* QuantizedKAvx2Kernel.ExecuteQuantizedTiled over `positions` (1..256) positions and all rows, with the
 * activations already quantized by Q8KCodec.QuantizeRow, [positions][columns / 256 * 292]
 * (QuantizedKAvx2Kernel.cs:47-99): per row and block the scales once, then each position's term into that
 * position's accumulator; output [positions][rows]. */
void or_qk_matvec_quantized_tiled_avx2(const uint8_t* weights, int rows, int columns, int format,
                                       const uint8_t* activations, int positions, float* output) {
    int blocks_per_row = columns / 256;
    int block_bytes = format == OR_Q4_K ? 144 : 210;
    int q4 = format == OR_Q4_K;
    int64_t row_bytes = (int64_t)blocks_per_row * 292;
    int sub_scales[8], sub_mins[8];
    float accumulator[256];
    if (positions < 1 || positions > 256) return;
    for (int row = 0; row < rows; row++) {
        for (int p = 0; p < positions; p++) accumulator[p] = 0;
        const uint8_t* weight_row = weights + (int64_t)row * blocks_per_row * block_bytes;
        for (int block = 0; block < blocks_per_row; block++) {
            const uint8_t* bw = weight_row + block * block_bytes;
            float d, dmin = 0;
            if (q4) {
                for (int sub = 0; sub < 8; sub++) or_q4k_get_scale_min(sub, bw + 4, &sub_scales[sub], &sub_mins[sub]);
                d = or_half_to_float(rd16(bw));
                dmin = or_half_to_float(rd16(bw + 2));
            } else {
                d = or_half_to_float(rd16(bw + 208));
            }
            for (int p = 0; p < positions; p++) {
                const uint8_t* activation = activations + p * row_bytes + (int64_t)block * 292;
                float activation_scale = rdf32(activation);
                if (activation_scale == 0) continue;
                accumulator[p] += q4 ? q4k_dot_quantized_avx2(bw, activation, sub_scales, sub_mins, d * activation_scale,
                                                              dmin * activation_scale)
                                     : activation_scale * d * (float)q6k_dot_product_avx2(bw, activation);
            }
        }
        for (int p = 0; p < positions; p++) output[(int64_t)p * rows + row] = accumulator[p];
    }
}
