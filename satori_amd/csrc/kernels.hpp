// Launch descriptors and launchers shared by the host runtime and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace satori {

// Formats: BlockQuantization values (src/Satori.Core/BlockQuantization.cs:3) plus Ternary2.
enum Format : int { kQ8_0 = 0, kQ4_0 = 1, kQ4_K = 2, kQ6_K = 3, kTernary2 = 16 };

// Bytes of one Q8_K activation block (src/Satori.Core/Q8KCodec.cs:31).
constexpr int kQ8KBlockBytes = 292;

// One matrix of a launch. Row-major payload: row r starts at w + r * row_bytes.
struct MatDesc {
    const uint8_t* w;   // weights (device; the payload, or its regrouped device layout)
    const float* x;     // FP32 activations [positions][columns]
    float* y;           // output [positions][rows]
    int rows;
    int pad_;
};

// Shape shared by every member of a launch.
struct LaunchShape {
    int format;         // Format
    int columns;        // C
    int block_size;     // Ternary2 B, else the format's block elements
    int blocks;         // blocks per row
    int64_t row_bytes;  // payload bytes per row
    int positions;      // activation vectors per call
    int rows_max;       // largest member row count (grid extent)
    int rows_per_wg;    // rows one workgroup owns (launcher-chosen)
    int chunk_blocks;   // integer K product: blocks of the activation row staged in LDS at a time (launcher-chosen)
};

// FP32-activation MatVec for the GGUF formats (Q8_0, Q4_0, Q4_K, Q6_K) on the packed row-major payload.
// `group` is a device array of `count` descriptors or nullptr, in which case `one` is used and count must be 1.
hipError_t launch_gemv_float(const MatDesc& one, const MatDesc* group, int count, LaunchShape shape,
                             hipStream_t stream);

// ---- Ternary2 device layout ("panels") ----
// The device copy of a Ternary2 matrix is regrouped so that one wave (64 lanes, one row each) reads whole
// cache lines: rows form panels of 64; a row's code stream (2 bits per column, LSB first, padded to whole
// blocks) is cut into 64-column chunks of 16 bytes; chunk k of the 64 rows of panel p is stored as 64
// consecutive 16-byte records, each record rotated left by 2 bits as one 128-bit little-endian integer (so
// a single mask exposes a nibble per byte). Block scales follow all codes, 64 consecutive floats per
// (panel, block slot).
// Chunks per row are rounded up to an even number (one 128-column tile = two chunks); padding rows, chunks
// and slots are zero. The total equals the packed payload up to that padding.
constexpr int kT2PanelRows = 64;
constexpr int kT2TileColumns = 128;

struct T2Layout {
    int panels;           // ceil(rows / 64)
    int tiles;            // 128-column tiles per row
    int chunks;           // 2 * tiles
    int slots;            // scale slots per panel row: chunks * 64 / B
    int64_t codes_bytes;  // panels * chunks * 1024
    int64_t bytes;        // codes_bytes + panels * slots * 256
};

inline T2Layout t2_layout(int rows, int columns, int block_size) {
    T2Layout l{};
    const int blocks = (columns + block_size - 1) / block_size;
    l.panels = (rows + kT2PanelRows - 1) / kT2PanelRows;
    l.tiles = (blocks * block_size + kT2TileColumns - 1) / kT2TileColumns;
    l.chunks = 2 * l.tiles;
    l.slots = l.chunks * 64 / block_size;
    l.codes_bytes = static_cast<int64_t>(l.panels) * l.chunks * 1024;
    l.bytes = l.codes_bytes + static_cast<int64_t>(l.panels) * l.slots * 256;
    return l;
}

// Upload-time regrouping on the device (upload.hip), one chunk of whole units at a time, into a destination
// the caller has zeroed. Ternary2: rows [64 first_panel, 64 first_panel + chunk_rows) of the packed payload
// (their bytes start at `packed`; Ternary2 or ternary bitplane blocks) into the panel layout; *bad is set to 1
// when a block breaks the payload rule of Ternary2Matrix.ValidatePayload (for bitplanes, equivalently,
// TernaryBitplaneMatrix.Validate; the caller names it from the host bytes).
struct T2Regroup {
    int first_panel, chunk_rows;      // the chunk: whole panels
    int columns, block_size, blocks;  // the matrix
    int block_bytes;
    int64_t row_bytes;
    int chunks, slots;                // T2Layout of the matrix
    int64_t codes_bytes;
    int bitplanes;                    // nonzero: the source blocks are ternary bitplane blocks
};
hipError_t launch_t2_regroup(const uint8_t* packed, const T2Regroup& r, uint8_t* out, uint32_t* bad,
                             hipStream_t stream);
// Q6_K: blocks [first, first + count) of a matrix of n blocks, their packed bytes at `packed`.
hipError_t launch_q6k_regroup(const uint8_t* packed, int64_t first, int64_t count, int64_t n, uint8_t* out,
                              hipStream_t stream);
// Q8_0 / Q4_0: likewise.
hipError_t launch_legacy_regroup(const uint8_t* packed, int64_t first, int64_t count, int64_t n, int format,
                                 uint8_t* out, hipStream_t stream);

// ---- Q6_K device layout ----
// The device copy of a Q6_K matrix holds the same bytes regrouped so that every load is aligned: for its
// n = rows * blocks blocks in row-major order, n records of 192 code bytes (block quarter c = 2h + t at
// 48c: ql[64h + 16t, +16), ql[64h + 32 + 16t, +16), qh[32h + 16t, +16)), then n records of 16 scale bytes
// (quarter c's sc[8h + 2k + t] at 4c + k), then n FP16 d values.

// ---- Q8_0 / Q4_0 device layout ----
// The same bytes regrouped so that code loads are aligned: for the n = rows * blocks blocks in row-major
// order, n code records (Q8_0: the 32 signed bytes; Q4_0: the 16 nibble bytes XOR 0x88, so each nibble holds
// q - 8 in two's complement), then the n FP16 scales.
constexpr int legacy_record_bytes(int format) { return format == kQ8_0 ? 32 : 16; }

// How a Ternary2 launch is cut: workgroups of `waves` waves (one 64-row panel each) take equal ranges of
// the launch's (panel group, tile) units; items cut between two ranges are finished by a second kernel.
// The launch needs a device scratch buffer of `scratch_bytes` whose start holds the plan's tables (range
// starts, cut items): copy `tables` there once before the first launch; the rest holds per-workgroup
// partial sums. A single matrix at one position small enough for the chip to hold all its workgroups at
// once is instead sliced: one kernel, workgroup (panel, column slice), slices joined through atomic
// exchange slots in the scratch (`tables` is their zeroed image); each launch tags its exchanges with a
// generation, a nonzero number that differs from the previous launches' (next_t2_generation).
// Launches that share a scratch buffer must not overlap in time: overlapping ones give undefined outputs,
// and the generation tags keep what they leave in the slots from reaching later launches. A plan is valid
// for the launch shape, member count and positions it was made for, on the device that was current.
struct T2Fixup {
    int member, position, panel0;  // the cut item
    int first, last;               // ranges holding its pieces
    int first_slot;                // slot of the piece in range `first` (0: its first segment, 1: its last)
    int pad_[2];
};

struct T2Plan {
    int rows_max, columns, block_size, count, positions;  // what the plan was made for
    int waves;                                            // waves per workgroup: 4, 8 or 16 (sliced: 1-16)
    int workgroups;                                       // ranges (one workgroup each)
    int staged_tiles;                                     // longest segment: activation tiles staged in LDS
    int fixups;                                           // items cut between ranges
    int slices;               // > 0: one matrix at one position, sliced (the column slices of a panel are
                              // joined in the kernel); 0: stream-K ranges plus the fix-up kernel
    int slice_groups;         // sliced: tiles per column slice
    size_t fixup_offset, partial_offset, scratch_bytes;  // scratch layout
    std::vector<uint8_t> tables;                         // host image of [starts][fixups] (sliced: zeroed
                                                         // exchange slots)
};

// Throws nothing; returns a plan with workgroups == 0 when the launch is too large to plan (more than
// 2^31 - 1 tiles of work).
T2Plan t2_plan(int rows_max, int columns, int block_size, int count, int positions);

// Workgroups of one Ternary2 kernel variant that fit on a CU at once (0 if unknown).
int t2_resident_workgroups(int block_size, int waves, int staged_tiles);

// Ternary2 MatVec on the panel layout (MatDesc::w points at it), with the plan made for this launch and
// its scratch buffer (tables already copied).
hipError_t launch_t2(const MatDesc& one, const MatDesc* group, int count, LaunchShape shape, const T2Plan& plan,
                     void* scratch, uint32_t generation, hipStream_t stream);

// The next launch's generation for a scratch buffer whose last launch used `last` (1, 2, ..., skipping 0).
inline uint32_t next_t2_generation(uint32_t& last) {
    if (++last == 0) last = 1;
    return last;
}

// Q8_K quantization of `positions` rows of `columns` floats (columns a multiple of 256), bit-exact with
// Q8KCodec.QuantizeRow. Output [positions][columns / 256 * 292].
hipError_t launch_q8k_quantize(const float* x, int columns, int positions, uint8_t* out, hipStream_t stream);

// Integer K-format product (Q4_K or Q6_K) against the Q8_K quantization of the FP32 activations, which each
// workgroup computes itself (bit-exact with Q8KCodec.QuantizeRow); outputs bit-exact with the reference's
// ExecuteQuantizedTiled composition. `members` is a host array of the `count` descriptors; launches of up to
// kKintInlineMembers pass them in the kernel arguments, larger ones read `device_members` (the same
// descriptors in device memory).
constexpr int kKintInlineMembers = 4;
hipError_t launch_gemv_kint(const MatDesc* members, const MatDesc* device_members, int count, LaunchShape shape,
                            hipStream_t stream);

// The shared input of a one-position K-format launch computed inside it from the decode step's operands
// instead of read from `x` (every workgroup computes it; the operator's launch disappears):
//  kInputAddRmsNorm: input = RmsNorm(a + b, w, epsilon) as add_rms_norm_kernel computes it (b may be null:
//    RmsNorm(a)); a + b is written to residual_out (if not null) by one workgroup;
//  kInputSwiGlu: input = SwiGlu(a, b) as swiglu_kernel computes it;
//  kInputQ8K: `a` points at the input already quantized (Q8KCodec.QuantizeRow bytes, 292 per block), as the
//    producer of the activation wrote it; the launch copies it instead of quantizing.
constexpr int kInputPlain = 0, kInputAddRmsNorm = 1, kInputSwiGlu = 2, kInputQ8K = 3;
struct InputTransform {
    int kind;
    float epsilon;
    const float* a;
    const float* b;
    const float* w;
    float* residual_out;
};
hipError_t launch_gemv_kint_transformed(const MatDesc* members, const MatDesc* device_members, int count,
                                        LaunchShape shape, const InputTransform& input, hipStream_t stream);

// The output of a two-member one-position K launch (members[0] = gate, members[1] = up, equal row counts, a
// multiple of 256) carried on inside it: each workgroup owns the same rows of both members, writes both
// members' outputs as the plain launch does, and SwiGlu(gate, up) of its rows to `activated`. With `q8k`, the
// last workgroup to finish a run of 256 rows also writes that run's Q8_K block (Q8KCodec.QuantizeBlock of the
// SwiGlu values) there, the down projection's input; `counters` holds one arrival count per 256 rows, zeroed
// once when the buffer is made: every launch adds exactly its arrivals per run (a power of two), so the count
// is never reset and wraps harmlessly.
struct OutputSwiGluQ8K {
    float* activated;
    uint8_t* q8k;
    uint32_t* counters;
};
hipError_t launch_gemv_kint_swiglu(const MatDesc* members, LaunchShape shape, const InputTransform& input,
                                   const OutputSwiGluQ8K& output, hipStream_t stream);

// Integer K-format product (Q4_K or Q6_K) over `positions` positions on the matrix cores: quantizes the FP32
// activations x ([positions][blocks * 256]) to Q8_K into `workspace` (kmfma_workspace_bytes), then the
// product; outputs bit-exact with launch_gemv_kint's. Used from kmfma_min_positions() positions on. `w` is
// the resident payload for Q4_K (row_bytes per row) and the matrix's weight planes for Q6_K.
hipError_t launch_gemv_kmfma(const uint8_t* w, int format, const float* x, uint8_t* workspace, float* y, int rows,
                             int blocks, int64_t row_bytes, int positions, hipStream_t stream);
size_t kmfma_workspace_bytes(int blocks, int positions);

// FP32-activation product (Q8_0 or Q4_0) over `positions` positions on the matrix cores (gemv_fbatch.hip):
// splits x ([positions][columns]) into three exact bf16 parts in `workspace` (fbatch_workspace_bytes), then
// the product on the resident device layout `w`; within 1e-5 * sum |w x| of the scalar reference like the
// single-position kernel. Used from fbatch_min_positions() positions on.
int fbatch_min_positions();
size_t fbatch_workspace_bytes(int columns, int positions);
hipError_t launch_gemv_fbatch(const uint8_t* w, int format, const float* x, uint8_t* workspace, float* y, int rows,
                              int columns, int positions, hipStream_t stream);

// The Q6_K matrix-core product reads the weights as pre-scaled int8 planes (2.02 bytes a weight, layout in
// gemv_kmfma.hip), built once from the regrouped resident layout `w` into a buffer of kmfma_planes_bytes.
size_t kmfma_planes_bytes(int rows, int blocks);
hipError_t launch_kmfma_planes(const uint8_t* w, int rows, int blocks, uint8_t* planes, hipStream_t stream);

// The same product in two steps, for several matrices of one format and width: launch_kmfma_pack quantizes
// one activation array into a workspace, and launch_kmfma_product runs up to kKmfmaMaxMembers products in one
// launch, member i reading the workspace packed from its input (members may share one).
constexpr int kKmfmaMaxMembers = 4;
struct KmfmaMember {
    const uint8_t* w;          // Q4_K: the resident payload; Q6_K: the weight planes (launch_kmfma_planes)
    const uint8_t* workspace;  // packed activations (launch_kmfma_pack, kmfma_workspace_bytes)
    float* y;                  // output [positions][rows]
    int rows;
    int pad_;
    int64_t row_bytes;         // Q4_K
};
struct KmfmaArgs {
    KmfmaMember m[kKmfmaMaxMembers];
    int units[kKmfmaMaxMembers];
    int count, blocks, positions, tiles;
};
// Workspace layout for `tiles` 32-position tiles: codes (8 KB per block and tile), then FP32 scales (32 per
// block and tile), then FP16 group sums (1 KB per block and tile).
__host__ __device__ inline size_t kmfma_scales_offset(int blocks, int tiles) {
    return static_cast<size_t>(blocks) * tiles * 8192;
}
__host__ __device__ inline size_t kmfma_sums_offset(int blocks, int tiles) {
    return static_cast<size_t>(blocks) * tiles * (8192 + 32 * sizeof(float));
}
hipError_t launch_kmfma_pack(int format, const float* x, int blocks, int positions, uint8_t* workspace,
                             hipStream_t stream);
hipError_t launch_kmfma_product(int format, const KmfmaMember* members, int count, int blocks, int positions,
                                hipStream_t stream);

// Decode-step operators (transformer_ops.hip): TransformerOps in FP64 with FP32 outputs, and the embedding row
// decode of a resident Q8_0 / Q4_K / Q6_K matrix.
hipError_t launch_rms_norm(const float* x, const float* w, float epsilon, int length, int count, float* y,
                           hipStream_t stream);
hipError_t launch_rms_norm_heads(float* v, const float* w, float epsilon, int head_dim, int heads, hipStream_t stream);
hipError_t launch_rope(float* v, int heads, int head_dim, int position, double base, int rotary, bool half_split,
                       hipStream_t stream);
hipError_t launch_swiglu(const float* gate, const float* up, int length, float* out, hipStream_t stream);
// SwiGlu and the Q8_K quantization of its output (Q8KCodec.QuantizeRow bytes) in one launch; `out` may be
// null (no FP32 output). length a multiple of 256.
hipError_t launch_swiglu_q8k(const float* gate, const float* up, int length, float* out, uint8_t* q8k,
                             hipStream_t stream);
hipError_t launch_add(const float* left, const float* right, int length, float* out, hipStream_t stream);
hipError_t launch_add_rms_norm(float* residual, const float* addend, const float* w, float epsilon, int length,
                               float* normed, hipStream_t stream);
// launch_add_rms_norm, and the Q8_K bytes of `normed` (Q8KCodec.QuantizeRow) into q8k; length a multiple of 256.
hipError_t launch_add_rms_norm_q8k(float* residual, const float* addend, const float* w, float epsilon, int length,
                                   float* normed, uint8_t* q8k, hipStream_t stream);
hipError_t launch_attention_inputs(float* q, const float* q_bias, const float* k, const float* k_bias, float* k_out,
                                   const float* v, const float* v_bias, float* v_out, int heads, int kv_heads,
                                   int head_dim, int position, double base, int rotary, hipStream_t stream);
// Grouped attention over `tokens` cached positions. Up to 32 tokens one workgroup per head; longer prefixes
// are split over several workgroups per head (attention_splits) whose FP64 partials go to `scratch`
// (attention_scratch_bytes: the bytes for `tokens`, which also cover every shorter prefix of these heads).
// attention_supported is false only where one split's exponentials and staged query would not fit the LDS
// (more than 134 million tokens).
hipError_t launch_attention(const float* q, const float* k, const float* v, int query_heads, int kv_heads,
                            int head_dim, int tokens, float* out, double* scratch, hipStream_t stream);
int attention_splits(int tokens);
size_t attention_scratch_bytes(int query_heads, int head_dim, int tokens);
bool attention_supported(int tokens, int head_dim);
// The attention-input transform of the decoded position (launch_attention_inputs with the cache slots of row
// `position`) followed by the attention over the position + 1 cached rows, with the same results bit for bit;
// on the split path the transform runs inside the split and combine launches (one launch fewer).
// `rope` is row `position` of a launch_rope_table table for (rotary, base), or null (computed in the launch).
hipError_t launch_attention_decode(float* q, const float* q_bias, const float* k_new, const float* k_bias,
                                   const float* v_new, const float* v_bias, float* k_cache, float* v_cache,
                                   int query_heads, int kv_heads, int head_dim, int position, double base, int rotary,
                                   const double* rope, float* out, double* partials, hipStream_t stream);
// RoPE sines and cosines of positions 0 .. positions - 1: row p = rotary / 2 sines, then the cosines (doubles).
hipError_t launch_rope_table(int positions, int rotary, double base, double* table, hipStream_t stream);
// Partials one call of `tokens` tokens writes (0 when one workgroup per head needs none).
size_t attention_partials_bytes(int query_heads, int head_dim, int tokens);
// The no-allocation attention's partials: a file-scope device array of kStaticAttentionBytes per device. Its
// device address on the current device (call with that device current; the address differs per device).
constexpr size_t kStaticAttentionBytes = size_t(4) << 20;
hipError_t static_attention_partials(double** partials);
hipError_t launch_decode_row(const uint8_t* w, int format, int rows, int columns, int row, float* out,
                             hipStream_t stream);

// Block-scale finiteness of an uploaded GGUF matrix (device layout; `blocks` = rows * blocks per row): a
// non-zero *flag afterwards (the caller zeroes it first) means some block has a non-finite scale.
hipError_t launch_scale_check(const uint8_t* payload, int64_t blocks, int format, uint32_t* flag, hipStream_t stream);
// Copies `bytes` (a multiple of 4, at most kKernelCopyMaxBytes; both addresses 16-byte aligned) with a kernel
// on `stream`; either side may be pinned host memory from hipHostMalloc.
constexpr size_t kKernelCopyMaxBytes = size_t(1) << 20;
hipError_t launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t stream);
int kmfma_min_positions();

// Blocks of the activation row the integer product stages in LDS at once (with the block terms of the
// workgroup's rows); wider rows are processed in chunks of this many blocks, in block order.
int kint_max_blocks();

}  // namespace satori
