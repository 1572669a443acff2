/*
 * satori_hip.h: C ABI of libsatori_hip.so, the MI355X (gfx950) backend for Satori's quantized
 * MatVec hot path (Ternary2 blocks of 64/128/256, GGUF Q8_0 / Q4_0 / Q4_K / Q6_K).
 *
 * The library is the drop-in under the reference's C# surfaces. Each entry point below names the
 * reference member it stands in for (paths relative to the reference repository root). Plain
 * pointers and sizes only; no C++ or torch types cross this boundary.
 *
 * Conventions
 *  - Every function returns a satori_hip_status. A non-zero status maps 1:1 to the exception the
 *    reference throws for the same condition; satori_hip_last_error() returns the message (per
 *    calling thread, valid until that thread's next call).
 *  - Host-pointer MatVec calls are synchronous and commit the output only on success: on any
 *    failure the caller's output buffer is left untouched
 *    (src/Satori.Core/IQuantizedMatrix.cs:6).
 *  - Weight payloads are copied (uploaded) before the create call returns; the caller may release
 *    or unmap them immediately afterwards (docs/vulkan-backend-v1.md:21).
 *  - A context serialises its calls with a mutex and owns one HIP stream at default priority.
 *    Calls on different contexts may run concurrently.
 */
#ifndef SATORI_HIP_H
#define SATORI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SATORI_HIP_ABI_VERSION 4

typedef struct satori_hip_context satori_hip_context;
typedef struct satori_hip_matrix satori_hip_matrix;
typedef struct satori_hip_group satori_hip_group;
typedef struct satori_hip_step satori_hip_step;
typedef struct satori_hip_gguf satori_hip_gguf;

typedef enum satori_hip_status {
    SATORI_HIP_OK = 0,
    SATORI_HIP_E_ARGUMENT = 1,                 /* System.ArgumentException */
    SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE = 2,    /* System.ArgumentOutOfRangeException */
    SATORI_HIP_E_INVALID_DATA = 3,             /* System.IO.InvalidDataException */
    SATORI_HIP_E_NOT_SUPPORTED = 4,            /* System.NotSupportedException */
    SATORI_HIP_E_OBJECT_DISPOSED = 5,          /* System.ObjectDisposedException */
    SATORI_HIP_E_PLATFORM_NOT_SUPPORTED = 6,   /* System.PlatformNotSupportedException (no gfx950 device) */
    SATORI_HIP_E_OUT_OF_MEMORY = 7,            /* System.OutOfMemoryException */
    SATORI_HIP_E_DEVICE = 8,                   /* System.InvalidOperationException: HIP runtime failure */
    SATORI_HIP_E_OVERFLOW = 9,                 /* System.OverflowException (checked arithmetic) */
    SATORI_HIP_E_ARGUMENT_NULL = 10,           /* System.ArgumentNullException */
    SATORI_HIP_E_KEY_NOT_FOUND = 11,           /* System.Collections.Generic.KeyNotFoundException */
    SATORI_HIP_E_INVALID_OPERATION = 12        /* System.InvalidOperationException (misuse, not the device) */
} satori_hip_status;

/* Values of Satori.Core.BlockQuantization (src/Satori.Core/BlockQuantization.cs:3), plus Ternary2. */
typedef enum satori_hip_format {
    SATORI_HIP_Q8_0 = 0,
    SATORI_HIP_Q4_0 = 1,
    SATORI_HIP_Q4_K = 2,
    SATORI_HIP_Q6_K = 3,
    SATORI_HIP_TERNARY2 = 16
} satori_hip_format;

/* ---- library ---- */

/* Library plumbing with no counterpart in the reference (it is a managed library): the ABI revision of
 * this header, the calling thread's last failure message and the visible device count. */
int satori_hip_abi_version(void);

/* Message of the calling thread's last failure ("" after success). */
const char* satori_hip_last_error(void);

/* Number of gfx950 devices visible to the process. */
int satori_hip_device_count(int* count);

/* ---- context: stands in for VulkanContext.TryCreate / Dispose
 *      (src/Satori.Backends.Vulkan/VulkanContext.cs:57), the IQuantizedMatrixFactory owner ---- */

/* Besides its stream, a context keeps grow-only device buffers until it is destroyed: the host-call staging
 * of inputs and outputs, the split-attention partials per stream, and the upload staging of the formats
 * regrouped on the device (Ternary2, bitplanes, Q6_K, Q8_0, Q4_0: at most 64 MB, or one 64-row Ternary2
 * panel of a wider matrix). */
int satori_hip_context_create(int device, satori_hip_context** context);
/* Idempotent: NULL is accepted. Matrices created on the context must be destroyed first. */
int satori_hip_context_destroy(satori_hip_context* context);
/* The context's HIP stream (hipStream_t), for the *_device entry points and resident pipelines. */
int satori_hip_context_stream(satori_hip_context* context, void** stream);

/* ---- matrices ---- */

/* Ternary2Matrix.FromPacked (src/Satori.Core/Ternary2Matrix.cs:73-81) + ValidatePayload (:83-101),
 * then upload. Also the upload step of MappedTernary2Matrix (src/Satori.Core/MappedTernary2Matrix.cs:9-35):
 * pass the mapped payload window. The payload is copied to the device as is, regrouped and checked there;
 * a failing payload is named by the reference's rule (first failing block, its scale before its codes) and
 * fails with its message. */
int satori_hip_ternary2_create(satori_hip_context* context, int rows, int columns, int block_size,
                               const void* payload, size_t payload_length, satori_hip_matrix** matrix);

/* IQuantizedMatrixFactory.Create (src/Satori.Core/IQuantizedMatrixFactory.cs:6) with the
 * QuantizedMatrixShape checks (src/Satori.Core/QuantizedMatrixShape.cs:5-22) and
 * QuantizedMatVec.ValidatePayload (src/Satori.Core/QuantizedMatVec.cs:28-42): the payload is uploaded (Q6_K,
 * Q8_0 and Q4_0 regrouped on the device) and its block scales checked there; a non-finite scale frees the
 * copy and fails with the first bad block's offset, as the reference names it. */
int satori_hip_quantized_create(satori_hip_context* context, int rows, int columns, int format,
                                const void* payload, size_t payload_length, satori_hip_matrix** matrix);

/* MappedTernary2Matrix(path) (src/Satori.Core/MappedTernary2Matrix.cs:9-35): opens an STQ2 file,
 * validates header and payload, uploads; corrupt files fail with SATORI_HIP_E_INVALID_DATA. */
int satori_hip_ternary2_open(satori_hip_context* context, const char* path, satori_hip_matrix** matrix);

/* ---- ternary bitplane layout (src/Satori.Core/TernaryBitplaneMatrix.cs) ----
 * Blocks of the FP32 scale, B/8 bytes of positive-plane bits, B/8 bytes of negative-plane bits; same shape
 * and byte length as Ternary2. The device copy is the lossless Ternary2 equivalent, so execution is the
 * Ternary2 MatVec (TernaryBitplaneMatVec.Execute, src/Satori.Core/TernaryBitplaneMatVec.cs:8-12) and the
 * matrix reports format SATORI_HIP_TERNARY2. */
/* TernaryBitplaneMatrix.FromPacked (TernaryBitplaneMatrix.cs:56-62) + Validate (:64-85), then upload: the
 * bitplane payload is copied to the device as is, converted, regrouped and checked there. */
int satori_hip_bitplane_create(satori_hip_context* context, int rows, int columns, int block_size,
                               const void* payload, size_t payload_length, satori_hip_matrix** matrix);
/* TernaryBitplaneMatrix.Load (TernaryBitplaneMatrix.cs:98-117) of an STB1 file, then upload; every file
 * defect fails with SATORI_HIP_E_INVALID_DATA. */
int satori_hip_bitplane_open(satori_hip_context* context, const char* path, satori_hip_matrix** matrix);
/* TernaryBitplaneMatrix.Load on the host: shape and payload of a valid STB1 file. With payload NULL only
 * the shape and length are returned; otherwise capacity must be at least the payload length. */
int satori_hip_bitplane_load(const char* path, int* rows, int* columns, int* block_size, void* payload,
                             size_t capacity, int64_t* length);
/* Host conversions and validation: TernaryBitplaneMatrix.FromTernary2 (:19-36, the Ternary2 payload is
 * validated first), ToTernary2 (:38-54, the bitplane payload is validated first) and Validate. */
int satori_hip_bitplane_from_ternary2(int rows, int columns, int block_size, const void* ternary2,
                                      size_t ternary2_length, void* bitplane, size_t bitplane_length);
int satori_hip_bitplane_to_ternary2(int rows, int columns, int block_size, const void* bitplane,
                                    size_t bitplane_length, void* ternary2, size_t ternary2_length);
int satori_hip_bitplane_validate(int rows, int columns, int block_size, const void* payload, size_t payload_length);

/* A second resident copy of already validated weights (device-to-device; no reference counterpart):
 * distinct copies for rotating-buffer measurements or for use from several streams. */
int satori_hip_matrix_clone(satori_hip_matrix* source, satori_hip_matrix** clone);

/* IDisposable.Dispose: idempotent per handle; NULL is accepted. */
int satori_hip_matrix_destroy(satori_hip_matrix* matrix);

/* Shape query: format is a satori_hip_format; block_size is 64/128/256 for Ternary2, else the
 * format's block elements; byte_length is the payload length. Any out pointer may be NULL. */
int satori_hip_matrix_shape(const satori_hip_matrix* matrix, int* rows, int* columns, int* format,
                            int* block_size, int64_t* byte_length);

/* ---- MatVec, host buffers, synchronous ----
 * Ternary2MatVec.Execute (src/Satori.Core/Ternary2MatVec.cs:9), MappedTernary2Matrix.Execute
 * (src/Satori.Core/MappedTernary2Matrix.cs:43), QuantizedMatVec.Execute
 * (src/Satori.Core/QuantizedMatVec.cs:12), GgufQuantizedMatrix.Execute
 * (src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:38) and IQuantizedMatrix.Execute
 * (src/Satori.Core/IQuantizedMatrix.cs:7): FP32 activations for every format (K formats use the
 * float decode of Q4KCodec.DotBlock / Q6KCodec.DotBlock). input_length must equal columns and
 * output_length rows; overlapping buffers are rejected (ArgumentException). Non-finite inputs are rejected
 * for the GGUF formats, whose call is the IQuantizedMatrix.Execute plugin seam of a GPU backend
 * (src/Satori.Backends.Vulkan/VulkanQ8Matrix.cs:82-83), and accepted and propagated for Ternary2, as
 * Ternary2MatVec.Execute does (src/Satori.Core/Ternary2MatVec.cs:30-36, 52-76). */
int satori_hip_matvec(satori_hip_matrix* matrix, const float* input, size_t input_length, float* output,
                      size_t output_length);

/* QuantizedMatVec.ExecuteBatch (src/Satori.Core/QuantizedMatVec.cs:104-120) and
 * GgufQuantizedMatrix.ExecuteBatch (src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:43-48):
 * input [positions][columns] -> output [positions][rows]. K formats quantize each position to
 * Q8_K on the device and use the integer product (at most 256 positions, as
 * src/Satori.Core/QuantizedKAvx2Kernel.cs:50-51; any width); Q8_0 / Q4_0 use the FP32 product. Non-finite
 * inputs are accepted and propagate as in the reference (QuantizedMatVec.cs:104-116). Ternary2 is
 * rejected with SATORI_HIP_E_NOT_SUPPORTED (the reference has no batched Ternary2 product). */
int satori_hip_matvec_batch(satori_hip_matrix* matrix, const float* input, size_t input_length, int positions,
                            float* output, size_t output_length);

/* Q8KCodec.QuantizeRow (src/Satori.Core/Q8KCodec.cs:85-93) on the device: columns a positive
 * multiple of 256, output_length = columns / 256 * 292; bytes identical to the reference. */
int satori_hip_quantize_q8k(satori_hip_context* context, const float* input, int columns, void* output,
                            size_t output_length);

/* ---- MatVec, device buffers, asynchronous (resident pipelines and benchmarks) ----
 * Same arithmetic as the host-buffer calls. input/output are device pointers; the work is enqueued on
 * `stream` (NULL = the context stream) and the call returns without waiting. No input validation
 * beyond shapes; the caller keeps the buffers alive until the stream has passed the work.
 * A matrix's launches share its device workspace (Ternary2: the exchange slots or partial sums of its
 * launch plan; K formats: the packed Q8_K of many-position products; Q8_0 / Q4_0: the split activations of
 * many-position products), so executions of one matrix on different streams must not overlap in time:
 * the outputs of overlapping executions are undefined. Later executions are not affected (each Ternary2
 * launch tags its exchanges with its own number, so nothing an overlapping launch leaves behind is added
 * in), except the replays of a captured step or capture that overlapped: those reuse their recorded
 * launch's number, so recreate such a step. For concurrent streams, give each stream its own copy
 * (satori_hip_matrix_clone). The same holds for groups (satori_hip_group_execute; a K group of more than four
 * members that share one input of more than 16 blocks also keeps that input's Q8_K bytes in a workspace of
 * its own, quantized once per launch). */
int satori_hip_matvec_device(satori_hip_matrix* matrix, const float* input, float* output, void* stream);
int satori_hip_matvec_batch_device(satori_hip_matrix* matrix, const float* input, int positions, float* output,
                                   void* stream);

/* ---- device buffers for the *_device entry points (no counterpart in the reference, whose buffers
 *      are host spans; a resident caller needs device activations) ---- */

int satori_hip_device_alloc(satori_hip_context* context, size_t bytes, void** device_ptr);
int satori_hip_device_free(satori_hip_context* context, void* device_ptr);
/* Copies `bytes` between host and device memory in the direction `kind` (1: host to device, 2: device to
 * host, 3: device to device), ordered on the context stream, and waits for completion. */
int satori_hip_copy(satori_hip_context* context, void* destination, const void* source, size_t bytes, int kind);
/* Waits for all work enqueued on the context stream. */
int satori_hip_synchronize(satori_hip_context* context);

/* ---- projection groups: one launch for several matrices of one format and width ----
 * Members share format, block size and column count (row counts may differ); member i reads
 * inputs[i] and writes outputs[i] (device pointers fixed at creation). quantized_activations
 * selects the Q8_K integer product for K formats (as ExecuteBatch at one position) instead of
 * the FP32 one. This has no counterpart in the reference: it is the launch shape the decode step
 * of DenseForward.Step (src/Satori.Core/Model/DenseForward.cs:100-162) needs for projections that
 * share an input (q/k/v, gate/up). */
int satori_hip_group_create(satori_hip_context* context, satori_hip_matrix* const* matrices, int count,
                            const float* const* inputs, float* const* outputs, int quantized_activations,
                            satori_hip_group** group);
int satori_hip_group_execute(satori_hip_group* group, void* stream);
/* The group's members over `positions` (1..256) positions: member i reads inputs[i] as [positions][columns]
 * and writes outputs[i] as [positions][rows_i] (the creation pointers), exactly as
 * satori_hip_matvec_batch_device per member. K-format groups with quantized activations only
 * (SATORI_HIP_E_NOT_SUPPORTED otherwise); members sharing an input pointer share its Q8_K quantization. The
 * prefill counterpart of the group launch: the q/k/v projections of DenseForward.LayerBatch
 * (src/Satori.Core/Model/DenseForward.cs:187-196) read one input, and so do gate/up (:243-248). The first call at a position count allocates the group's workspace (not while
 * capturing: SATORI_HIP_E_INVALID_OPERATION). */
int satori_hip_group_execute_batch(satori_hip_group* group, int positions, void* stream);
/* Input transforms: a K-format group with quantized activations can compute its (shared) input inside its
 * own launch from the operands of the decode-step operator that would produce it, instead of reading
 * inputs[i]; the operator's launch then disappears. The values are those of the operator bit for bit.
 *  SATORI_HIP_INPUT_ADD_RMS_NORM: input = RmsNorm(a + b, weights, epsilon) (b may be NULL: RmsNorm(a)),
 *    as satori_hip_add_rms_norm / satori_hip_rms_norm compute it; when residual_out is not NULL the launch
 *    also writes a + b there (it must not overlap a, b, the weights or the members' outputs);
 *  SATORI_HIP_INPUT_SWIGLU: input = SwiGlu(a, b), as satori_hip_swiglu;
 *  SATORI_HIP_INPUT_Q8K: `a` points at the input already quantized to Q8_K (Q8KCodec.QuantizeRow bytes,
 *    columns / 256 * 292, as satori_hip_swiglu_q8k or satori_hip_quantize_q8k_device write them): the launch
 *    reads those bytes instead of quantizing (b, weights, epsilon and residual_out are ignored); the outputs
 *    are those of the plain launch over the FP32 input the bytes were quantized from, bit for bit;
 *  SATORI_HIP_INPUT_PLAIN: back to reading inputs[i].
 * Vectors have the members' column count. One-position launches only (satori_hip_group_execute_batch
 * fails with SATORI_HIP_E_NOT_SUPPORTED). Not while steps replay the group (SATORI_HIP_E_ARGUMENT) or while
 * capturing. No counterpart in the reference, whose DenseForward.Step (src/Satori.Core/Model/
 * DenseForward.cs:100-162) runs RmsNorm (:107, :151), Add (:148, :160) and SwiGlu (:156) as separate
 * TransformerOps calls between its projections. */
#define SATORI_HIP_INPUT_PLAIN 0
#define SATORI_HIP_INPUT_ADD_RMS_NORM 1
#define SATORI_HIP_INPUT_SWIGLU 2
#define SATORI_HIP_INPUT_Q8K 3
int satori_hip_group_set_input(satori_hip_group* group, int kind, const float* a, const float* b,
                               const float* weights, float epsilon, float* residual_out);
/* Output transforms: a K-format group with quantized activations of two members with the same row count, a
 * multiple of 256 (gate, then up), can carry the SwiGlu that follows it inside its own launch:
 *  SATORI_HIP_OUTPUT_SWIGLU: besides the members' outputs (unchanged, bit for bit), the launch writes
 *    SwiGlu(gate output, up output) to `activated` (rows floats), exactly what satori_hip_swiglu writes from
 *    the two outputs; each workgroup computes the same rows of both members. When `q8k` is not NULL the
 *    launch also writes the Q8KCodec.QuantizeRow bytes of that vector there (rows / 256 * 292 bytes), as
 *    satori_hip_swiglu_q8k does, for a down group reading them through SATORI_HIP_INPUT_Q8K: the last
 *    workgroup to finish a run of 256 rows, found by an arrival count in a device buffer the group owns,
 *    quantizes that run;
 *  SATORI_HIP_OUTPUT_PLAIN: back to the members' outputs only.
 * `activated` and `q8k` must not overlap each other, the inputs or the outputs. Combines with any input
 * transform but SATORI_HIP_INPUT_SWIGLU. One-position launches only (satori_hip_group_execute_batch fails
 * with SATORI_HIP_E_NOT_SUPPORTED). Not while steps replay the group (SATORI_HIP_E_ARGUMENT) or while
 * capturing. Launches of one such group must not overlap (two streams at once): with `q8k` the arrival
 * counts are shared, and overlapping launches leave `activated` and `q8k` undefined for those launches
 * (later ones are unaffected). No counterpart in the reference, whose DenseForward.Step
 * (src/Satori.Core/Model/DenseForward.cs:152-158) runs the gate and up projections, then SwiGlu, then the
 * down projection, which quantizes its input (QuantizedMatVec.ExecuteBatch, QuantizedMatVec.cs:144-149). */
#define SATORI_HIP_OUTPUT_PLAIN 0
#define SATORI_HIP_OUTPUT_SWIGLU 1
int satori_hip_group_set_output(satori_hip_group* group, int kind, float* activated, void* q8k);
/* Fails with SATORI_HIP_E_ARGUMENT while a step replays the group. A matrix cannot be destroyed while a
 * group launches it (same status). */
int satori_hip_group_destroy(satori_hip_group* group);

/* ---- steps: an ordered list of groups replayed as one HIP graph ----
 * satori_hip_step_create waits for the context stream, then captures the launches of `count` groups, in
 * order, into one graph; satori_hip_step_execute replays it on `stream` (null: the context stream), in
 * the order the groups' launches would run eagerly, reading and writing the groups' device buffers. No
 * counterpart in the reference: it is the resident form of the projection sequence of DenseForward.Step
 * (src/Satori.Core/Model/DenseForward.cs:100-162), whose cost per token the reference attributes to
 * per-call overheads; one replay replaces a launch per projection. Replays that overlap in time share
 * the groups' scratch buffers and must be serialised by the caller. */
int satori_hip_step_create(satori_hip_context* context, satori_hip_group* const* groups, int count,
                           satori_hip_step** step);
int satori_hip_step_execute(satori_hip_step* step, void* stream);
int satori_hip_step_destroy(satori_hip_step* step);

/* ---- host-only entry points (CPU; no device needed, never on the MatVec path) ---- */

/* Ternary2Shape.ByteLength (src/Satori.Core/Ternary2Shape.cs:5-15) when format is SATORI_HIP_TERNARY2
 * (block_size 64/128/256), else QuantizedMatrixShape.ByteLength (src/Satori.Core/QuantizedMatrixShape.cs:5-22;
 * block_size ignored). Invalid shapes fail as the constructors do. */
int satori_hip_payload_length(int format, int rows, int columns, int block_size, int64_t* length);

/* Ternary2Matrix.FromPacked checks (src/Satori.Core/Ternary2Matrix.cs:73-101). */
int satori_hip_ternary2_validate(int rows, int columns, int block_size, const void* payload, size_t payload_length);

/* QuantizedMatrix constructor checks (src/Satori.Core/QuantizedMatrix.cs:8-13, QuantizedMatVec.cs:28-42). */
int satori_hip_quantized_validate(int rows, int columns, int format, const void* payload, size_t payload_length);

/* Ternary2Matrix.Quantize (src/Satori.Core/Ternary2Matrix.cs:38-71): FP32 weights [rows][columns] to a
 * Ternary2 payload (absmean FP32 block scale, FP64 threshold); non-finite weights are rejected. */
int satori_hip_ternary2_quantize(const float* weights, int rows, int columns, int block_size, void* payload,
                                 size_t payload_length);

/* Round-to-nearest Q8_0 / Q4_0 / Q4_K / Q6_K quantizers used to build seeded synthetic matrices. No
 * counterpart in the reference, which only decodes these formats; the packing is the exact inverse of
 * its decoders (Q4KCodec.GetScaleMin, Q4KCodec.DecodeBlock, Q6KCodec.DecodeBlock). */
int satori_hip_quantize_weights(int format, const float* weights, int rows, int columns, void* payload,
                                size_t payload_length);

/* Stream capture (no reference counterpart; for resident decode loops): everything the calls between begin
 * and end enqueue on the context stream (stream argument NULL) -- group launches, *_device MatVecs, the
 * decode-step operators, row decodes -- is recorded into one graph, which capture_end turns into a step
 * replayed by satori_hip_step_execute and freed by satori_hip_step_destroy. The step keeps the matrices and
 * groups it launches from being destroyed. While capturing, calls that synchronise, allocate or copy
 * through the host fail with SATORI_HIP_E_INVALID_OPERATION (a many-position K product must have run once
 * before, so its workspace exists), and no other thread may use the context. The step records the device
 * addresses of the workspaces it launches with (a matrix's or group's Q8_K buffer, the split attention's
 * partials): while it lives, a call that would grow one of them fails with SATORI_HIP_E_INVALID_OPERATION. */
int satori_hip_capture_begin(satori_hip_context* context);
int satori_hip_capture_end(satori_hip_context* context, satori_hip_step** step);

/* ---- decode-step operators (src/Satori.Core/TransformerOps.cs), device pointers ----
 * Enqueued on `stream` (NULL: the context stream), like the *_device MatVec calls. Each computes in FP64 as
 * the reference does and rounds its outputs to FP32 once; outputs agree with the reference's to about one
 * unit in the last place (Add exactly). Argument checks and their exceptions follow the reference. */
/* RmsNorm (TransformerOps.cs:13-21) over `count` consecutive vectors of `length`; output == input allowed. */
int satori_hip_rms_norm(satori_hip_context* context, const float* input, const float* weights, float epsilon,
                        int length, int count, float* output, void* stream);
/* RmsNormHeads (TransformerOps.cs:117-130), in place. */
int satori_hip_rms_norm_heads(satori_hip_context* context, float* vector, const float* weights, float epsilon,
                              int head_dim, int length, void* stream);
/* Rope (TransformerOps.cs:23-38, pairs (j, j + 1), base 10000) and RopeHalf (:94-114), in place. */
int satori_hip_rope(satori_hip_context* context, float* vector, int length, int head_dim, int position, void* stream);
int satori_hip_rope_half(satori_hip_context* context, float* vector, int length, int head_dim, int position,
                         double frequency_base, int rotary_dimensions, void* stream);
/* SwiGlu (TransformerOps.cs:40-50) and Add (:52-57); output may equal an input. */
int satori_hip_swiglu(satori_hip_context* context, const float* gate, const float* up, int length, float* output,
                      void* stream);
int satori_hip_add(satori_hip_context* context, const float* left, const float* right, int length, float* output,
                   void* stream);
/* SwiGlu (TransformerOps.cs:40-50) and Q8KCodec.QuantizeRow of its output (src/Satori.Core/Q8KCodec.cs:85-93)
 * in one launch: the activation of the down projection of DenseForward.Step (DenseForward.cs:156-160), which
 * the reference quantizes inside ExecuteBatch (QuantizedMatVec.cs:136-219), quantized once by its producer for
 * a group reading it with SATORI_HIP_INPUT_Q8K. length a positive multiple of 256; q8k receives
 * length / 256 * 292 bytes, identical to the reference's; output (FP32, as satori_hip_swiglu) may be NULL. */
int satori_hip_swiglu_q8k(satori_hip_context* context, const float* gate, const float* up, int length, float* output,
                          void* q8k, void* stream);
/* satori_hip_quantize_q8k over device buffers, enqueued like the operators: `positions` rows of `columns`
 * floats (a positive multiple of 256) to [positions][columns / 256 * 292] Q8_K bytes. */
int satori_hip_quantize_q8k_device(satori_hip_context* context, const float* input, int columns, int positions,
                                   void* output, void* stream);
/* Fused steps of DenseForward.Step, bit-identical to the separate calls: Add then RmsNorm
 * (DenseForward.cs:156-158: residual += addend, normed = RmsNorm(residual)), and the attention inputs of one
 * position (DenseForward.cs:128-151: the q/k/v bias adds when biases are given (NULL: none), RopeHalf of the
 * query in place and of the key into key_out, the value into value_out -- key_out / value_out being the
 * cache slots). */
int satori_hip_add_rms_norm(satori_hip_context* context, float* residual, const float* addend, const float* weights,
                            float epsilon, int length, float* normed, void* stream);
/* satori_hip_add_rms_norm, and Q8KCodec.QuantizeRow of `normed` (src/Satori.Core/Q8KCodec.cs:85-93) into q8k
 * in the same launch: the input of the projections after the residual add of DenseForward.Step
 * (DenseForward.cs:149, :156-158), which the reference quantizes inside ExecuteBatch, quantized once by its
 * producer for a group reading it with SATORI_HIP_INPUT_Q8K. length a positive multiple of 256; q8k receives
 * length / 256 * 292 bytes, identical to the reference's; normed and residual as satori_hip_add_rms_norm. */
int satori_hip_add_rms_norm_q8k(satori_hip_context* context, float* residual, const float* addend,
                                const float* weights, float epsilon, int length, float* normed, void* q8k,
                                void* stream);
int satori_hip_attention_inputs(satori_hip_context* context, float* query, const float* query_bias, const float* key,
                                const float* key_bias, float* key_out, const float* value, const float* value_bias,
                                float* value_out, int query_heads, int kv_heads, int head_dim, int position,
                                double frequency_base, int rotary_dimensions, void* stream);
/* GroupedAttention (TransformerOps.cs:135-179; Attention :61-91 is query_heads == kv_heads): keys/values
 * token-major [tokens][kv_heads * head_dim]. The scores live on the device (no scratch argument). Prefixes
 * longer than 32 tokens are split over several workgroups per head, whose partial sums go to a workspace the
 * context keeps per stream: it is allocated by the first split attention on that stream and grows with the
 * prefix; attentions on different streams never share one. While capturing, and while captured steps use the
 * context stream's workspace, a call that would have to grow it fails with SATORI_HIP_E_INVALID_OPERATION. */
int satori_hip_grouped_attention(satori_hip_context* context, const float* query, const float* keys,
                                 const float* values, int query_heads, int kv_heads, int head_dim, int tokens,
                                 float* output, void* stream);
/* The sines and cosines of the RoPE angles (RopeHalf, TransformerOps.cs:94-114) of positions 0 .. positions - 1
 * for (rotary_dimensions, frequency_base), as the rotation kernels compute them: row p holds the
 * rotary_dimensions / 2 sines then the cosines, as doubles (positions * rotary_dimensions of them). A table for
 * satori_hip_attention_decode, computed once per session instead of once per token. */
int satori_hip_rope_table(satori_hip_context* context, int positions, int rotary_dimensions, double frequency_base,
                          double* table, void* stream);
/* The attention of one decode position with its inputs (DenseForward.cs:128-152):
 * satori_hip_attention_inputs(query, query_bias, key, key_bias, keys + position * kv_width, value, value_bias,
 * values + position * kv_width, ...) then satori_hip_grouped_attention(query, keys, values, ..., position + 1,
 * output), with the same results bit for bit (the query rotated in place, the key and value written to row
 * `position` of the caches); past 32 tokens the transform runs inside the split attention's launches, one
 * launch fewer. Biases may be NULL. keys/values are the caches [position + 1][kv_heads * head_dim]; key and
 * value must not overlap them. rope_table is a satori_hip_rope_table table of at least position + 1 rows for
 * (rotary_dimensions, frequency_base), or NULL (the angles are then computed in the launch). The workspace rules
 * are those of satori_hip_grouped_attention. */
int satori_hip_attention_decode(satori_hip_context* context, float* query, const float* query_bias, const float* key,
                                const float* key_bias, const float* value, const float* value_bias, float* keys,
                                float* values, int query_heads, int kv_heads, int head_dim, int position,
                                double frequency_base, int rotary_dimensions, const double* rope_table, float* output,
                                void* stream);
/* satori_hip_grouped_attention without any allocation. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, hosts that forbid
 * allocation after start-up). Same arguments, checks and results (the same kernels); the split partials go
 * to a static device workspace of 4 MiB per device (resolved when the context is created, held until the
 * process ends) instead of a context workspace: a call whose partials, query_heads * splits * (head_dim + 2)
 * * 8 bytes, exceed it fails with SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE (12 heads of 128 lanes: prefixes up to
 * 688,128 tokens). Every call on a device shares that workspace and leaves its partials there: calls that
 * overlap in time on one device (other streams, other contexts) race and must be serialised by the caller. */
int satori_hip_grouped_attention_static(satori_hip_context* context, const float* query, const float* keys,
                                        const float* values, int query_heads, int kv_heads, int head_dim, int tokens,
                                        float* output, void* stream);
/* GgufQuantizedMatrix.ReadRow (src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:54-61): row `row` of a resident
 * Q8_0 / Q4_K / Q6_K matrix decoded to FP32 `columns` floats (QuantizedRow.DecodeRow), bit-identical to the
 * reference's decode. Q4_0 and Ternary2 fail with SATORI_HIP_E_NOT_SUPPORTED. */
int satori_hip_matrix_decode_row(satori_hip_matrix* matrix, int row, float* output, void* stream);

/* ---- GGUF containers (src/Satori.Formats.Gguf) ----
 * A GGUF v3 file mapped read-only and its catalogue parsed strictly, with the reference's limits and
 * failure kinds: GgufFile(path) and GgufFile.Parse (src/Satori.Formats.Gguf/GgufFile.cs:17-35, 78-176),
 * GgufCursor (src/Satori.Formats.Gguf/GgufCursor.cs:7-56). Corrupt structure fails with
 * SATORI_HIP_E_INVALID_DATA, files outside the supported profile with SATORI_HIP_E_NOT_SUPPORTED. A file
 * handle needs no context; after close, calls on it fail with SATORI_HIP_E_OBJECT_DISPOSED. Names and
 * keys returned by the info calls, and windows, stay valid until the file is closed. */
int satori_hip_gguf_open(const char* path, satori_hip_gguf** file);
/* GgufFile.Dispose (src/Satori.Formats.Gguf/GgufFile.cs:206): idempotent; NULL is accepted. */
int satori_hip_gguf_close(satori_hip_gguf* file);
/* GgufFile.DataOffset (src/Satori.Formats.Gguf/GgufFile.cs:40). */
int satori_hip_gguf_data_offset(const satori_hip_gguf* file, int64_t* offset);
/* GgufFile.Tensors (src/Satori.Formats.Gguf/GgufFile.cs:38): count, lookup by name
 * (SATORI_HIP_E_KEY_NOT_FOUND when absent) and the GgufTensor record of entry `index` in declaration
 * order (src/Satori.Formats.Gguf/GgufTensor.cs:5-20): dims[0] is the contiguous dimension; offset is
 * absolute in the file. Any out pointer may be NULL. */
int satori_hip_gguf_tensor_count(const satori_hip_gguf* file, int64_t* count);
int satori_hip_gguf_tensor_find(const satori_hip_gguf* file, const char* name, int64_t* index);
int satori_hip_gguf_tensor_info(const satori_hip_gguf* file, int64_t index, const char** name, int* rank,
                                int64_t dims[4], uint32_t* type, int64_t* offset, int64_t* byte_length);
/* GgufFile.ReadTensor (src/Satori.Formats.Gguf/GgufFile.cs:42-49): the window [offset, offset + length) of
 * the tensor's payload, zero-copy. A window beyond the payload fails with
 * SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE. */
int satori_hip_gguf_tensor_window(const satori_hip_gguf* file, int64_t index, int64_t offset, int64_t length,
                                  const void** bytes);
/* GgufFile.Metadata (src/Satori.Formats.Gguf/GgufFile.cs:39): count, lookup by key, and the GgufMetadata
 * record (src/Satori.Formats.Gguf/GgufMetadata.cs:3-4); element_type and element_count are -1 for
 * scalars. */
int satori_hip_gguf_metadata_count(const satori_hip_gguf* file, int64_t* count);
int satori_hip_gguf_metadata_find(const satori_hip_gguf* file, const char* key, int64_t* index);
int satori_hip_gguf_metadata_info(const satori_hip_gguf* file, int64_t index, const char** key, uint32_t* type,
                                  int64_t* offset, int64_t* byte_length, int64_t* element_type,
                                  int64_t* element_count);
/* GgufFile.ReadMetadata (src/Satori.Formats.Gguf/GgufFile.cs:51-56): the value bytes of entry `index`
 * (for strings the u64 length comes first, as in the file), zero-copy. */
int satori_hip_gguf_metadata_window(const satori_hip_gguf* file, int64_t index, const void** bytes, int64_t* length);
/* new GgufQuantizedMatrix(file, name) + CreateExecution (src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:13-36):
 * a rank-2 Q8_0 / Q4_0 / Q4_K / Q6_K tensor within Int32 limits (else SATORI_HIP_E_NOT_SUPPORTED) as
 * rows = dims[1], columns = dims[0], uploaded from the mapping straight to a resident device matrix. The
 * block-scale check of QuantizedMatVec.ValidatePayload (src/Satori.Core/QuantizedMatVec.cs:28-42) runs on
 * the device over the uploaded copy; a non-finite scale frees it and fails with SATORI_HIP_E_INVALID_DATA. */
int satori_hip_gguf_matrix_create(satori_hip_context* context, const satori_hip_gguf* file, int64_t index,
                                  satori_hip_matrix** matrix);

#ifdef __cplusplus
}
#endif
#endif /* SATORI_HIP_H */
