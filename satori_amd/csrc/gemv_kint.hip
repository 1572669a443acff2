// Q8_K activation quantizer and the integer K-format products (Q4_K x Q8_K, Q6_K x Q8_K) for gfx950.
//
// Both reproduce the reference bit for bit:
//  - the quantizer is Q8KCodec.QuantizeBlock (src/Satori.Core/Q8KCodec.cs:44-76): first-largest |x| with
//    a strict comparison, -127/max and 1/inverse as correctly rounded divisions, the product and the
//    12582912 add rounded separately (the library is compiled with -ffp-contract=off and the operations
//    are spelled with explicit round-to-nearest intrinsics);
//  - the products are exact int32 sums (v_dot4_i32_i8), and the per-block FP32 expression and the
//    block-order accumulation of each row are those of QuantizedKAvx2Kernel.ExecuteQuantizedTiled
//    (src/Satori.Core/QuantizedKAvx2Kernel.cs:47-99), so each output equals the reference's float.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"
#include "ops_device.hpp"
#include "q8k_device.hpp"

namespace satori {
namespace {

// ------------------------------------------------------------------------------------------------
// Q8_K quantizer (one wave per block; the per-block arithmetic is in q8k_device.hpp).
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void q8k_quantize_kernel(const float* __restrict__ x, int columns,
                                                          uint8_t* __restrict__ out) {
    const int block = blockIdx.x;
    const int position = blockIdx.y;
    const int blocks = columns / 256;
    const int lane = threadIdx.x;
    const float* src = x + static_cast<int64_t>(position) * columns + block * 256;
    uint8_t* dst = out + (static_cast<int64_t>(position) * blocks + block) * kQ8KBlockBytes;
    float v[4];
    q8k_load_values(src, lane, v);
    const Q8KLane q = q8k_quantize_values(v, lane);
    if (q.zero) {
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
        for (int i = lane; i < kQ8KBlockBytes / 4; i += 64) d32[i] = 0u;
        return;
    }
    reinterpret_cast<uint32_t*>(dst + 4)[lane] = q.packed;
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(dst + 260)[lane >> 2] = static_cast<int16_t>(q.group_sum);
    if (lane == 0) reinterpret_cast<float*>(dst)[0] = q.scale;
}

// ------------------------------------------------------------------------------------------------
// Integer product. A workgroup owns s.rows_per_wg rows (4 to 64) of one member at one position. It quantizes the
// position's FP32 activation row to Q8_K itself (one wave per block, bit-exact as above; every workgroup
// computes the same bytes) straight into LDS as separate arrays (codes, group sums, scales), so no separate
// quantization launch precedes the product and code reads are 16-byte aligned.
// Work items are (row, block) pairs, 4 lanes of 64 weights each; the G lanes' int32 partials are summed
// exactly, the pair's leader forms the block's FP32 term and stores it in LDS, and finally one thread per row
// adds its terms in block order. A row wider than the LDS holds (more than kint_max_blocks() blocks) is
// staged and summed in chunks of blocks, in block order, so the sum is the same sequential one.
// ------------------------------------------------------------------------------------------------
constexpr int kThreads = 256;
constexpr int kTileRows = 64;
// The staged Q8_K codes of block b start at dword kCodeStride * b: 64 code dwords plus 4 of padding, so the
// 16 (row, block) pairs of a wave, which read 16 consecutive blocks at the same offset, hit 16 different
// groups of LDS banks instead of the same four.
constexpr int kCodeStride = 68;
constexpr int kActDwords = kCodeStride + 1 + 8;  // codes, scale, group sums per block
// Activation loads a thread issues before the weight loads: passes of 16 Q8_K blocks (48 blocks preloaded)
// and elements of the RmsNorm sum of squares (2,048 columns).
constexpr int kQ8KPasses = 3;  // 48 blocks
constexpr int kNormPreload = 8;
// An RmsNorm input row of at most this many columns keeps its summed values (residual + addend) in LDS
// between the sum of squares and the quantization, instead of reading both operands again.
constexpr int kNormStageColumns = 8192;


__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

struct ActTile {
    uint32_t* codes;   // [blocks][64] dwords
    int16_t* sums;     // [blocks][16]
    float* scales;     // [blocks]
};

// Q4_K pair, lane c of 4 = group g: qs[32g, 32g + 32), low nibbles are weights 64g + i of sub-block 2g,
// high nibbles weights 64g + 32 + i of sub-block 2g + 1 (Q4KCodec.DotProduct / MinProduct, Q4KCodec.cs:117-153).
struct Q4KRaw {
    u32x4 head;  // d, dmin, scales[12]
    u32x4 qs0, qs1;
};

__device__ __forceinline__ void q4k_load(const uint8_t* block, int c, Q4KRaw& r) {
    r.head = load16_a4(block);
    r.qs0 = load16_a4(block + 16 + 32 * c);
    r.qs1 = load16_a4(block + 32 + 32 * c);
}

__device__ __forceinline__ void q4k_dot(const Q4KRaw& r, const ActTile& act, int b, int g, int& dot, int& min_part) {
    int s0, m0, s1, m1;
    q4k_scale_min(2 * g, r.head, s0, m0);
    q4k_scale_min(2 * g + 1, r.head, s1, m1);
    const uint32_t* codes = act.codes + kCodeStride * b + 16 * g;
    const u32x4 lo0 = *reinterpret_cast<const u32x4*>(codes), lo1 = *reinterpret_cast<const u32x4*>(codes + 4);
    const u32x4 hi0 = *reinterpret_cast<const u32x4*>(codes + 8), hi1 = *reinterpret_cast<const u32x4*>(codes + 12);
    int lo = 0, hi = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        lo = sdot4(r.qs0[w] & 0x0F0F0F0Fu, lo0[w], lo);
        lo = sdot4(r.qs1[w] & 0x0F0F0F0Fu, lo1[w], lo);
        hi = sdot4((r.qs0[w] >> 4) & 0x0F0F0F0Fu, hi0[w], hi);
        hi = sdot4((r.qs1[w] >> 4) & 0x0F0F0F0Fu, hi1[w], hi);
    }
    dot = s0 * lo + s1 * hi;
    const int16_t* sums = act.sums + 16 * b;
    min_part = m0 * (sums[4 * g] + sums[4 * g + 1]) + m1 * (sums[4 * g + 2] + sums[4 * g + 3]);
}

// Q6_K pair, lane c of 4: half h = c / 2, slice t = c % 2, i.e. weights 128h + 32k + 16t + i
// (Q6KCodec.DotProduct, Q6KCodec.cs:114-146, with the -32 centring applied through the group sums:
// sum sc * (q - 32) * code = sum sc * q * code - 32 * sum sc * bsum, both exact), read from the regrouped
// device layout (Q6KLayout).
using Q6KRaw = Q6KQuarter;

__device__ __forceinline__ int q6k_dot(const Q6KRaw& r, const ActTile& act, int b, int c) {
    const int h = c >> 1, t = c & 1;
    int dotk[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t a = r.qla[w], bq = r.qlb[w], hb = r.qh[w];
        const uint32_t q[4] = {
            (a & 0x0F0F0F0Fu) | ((hb << 4) & 0x30303030u),
            (bq & 0x0F0F0F0Fu) | ((hb << 2) & 0x30303030u),
            ((a >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u),
            ((bq >> 4) & 0x0F0F0F0Fu) | ((hb >> 2) & 0x30303030u),
        };
#pragma unroll
        for (int k = 0; k < 4; ++k)
            dotk[k] = sdot4(q[k], act.codes[kCodeStride * b + 32 * h + 8 * k + 4 * t + w], dotk[k]);
    }
    const int16_t* sums = act.sums + 16 * b;
    int total = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int sc = static_cast<int8_t>(r.sc >> (8 * k));  // scale 8h + 2k + t
        total += sc * (dotk[k] - 32 * sums[8 * h + 2 * k + t]);
    }
    return total;
}

// LDS: staged activations, the row terms, then (input transforms) 256 doubles for the RmsNorm reduction at an
// 8-byte aligned dword offset. Sized for the largest tile so one bound serves every launch.
__host__ __device__ inline int kint_red_offset(int blocks, int tile_rows) {
    return ((kActDwords + tile_rows) * blocks + 1) & ~1;
}

static_assert(kThreads == kOpsThreads, "the RmsNorm reduction is the operators' 256-thread tree");

// The members of a launch of up to kKintInlineMembers matrices travel in the kernel arguments, so the first
// weight loads depend on no global-memory read; larger groups read a device array of descriptors.
struct KintMembers {
    MatDesc m[kKintInlineMembers];
};

// PAIRED: a two-member launch (gate, up) whose workgroups own the same s.rows_per_wg rows of both members
// (2 * rows_per_wg <= 64 row sums, all in the first wave), carrying SwiGlu and its Q8_K bytes on (see
// OutputSwiGluQ8K).
template <int FORMAT, int XF, bool INLINE, bool PAIRED>
__global__ __launch_bounds__(kThreads) void gemv_kint_kernel(KintMembers inline_members,
                                                              const MatDesc* __restrict__ group, LaunchShape s,
                                                              InputTransform xf, OutputSwiGluQ8K out) {
    static_assert(!PAIRED || INLINE, "paired launches pass their two members in the kernel arguments");
    constexpr int G = 4;  // lanes per (row, block) pair
    constexpr int kBlockBytes = FORMAT == kQ4_K ? 144 : 210;
    constexpr int kPairsPerStep = kThreads / G;
    using Raw = typename std::conditional<FORMAT == kQ4_K, Q4KRaw, Q6KRaw>::type;
    // Inline members come from the kernel arguments through the scalar cache; a larger group's descriptor is
    // one global load.
    const MatDesc m = INLINE ? inline_members.m[PAIRED ? 0 : blockIdx.y] : group[blockIdx.y];
    const int tile_rows = s.rows_per_wg;
    const int row_begin = blockIdx.x * tile_rows;
    if (row_begin >= m.rows) return;
    const int rows = min(tile_rows, m.rows - row_begin);
    // Rows of the workgroup's terms: its rows of m, then (paired) the same rows of the second member.
    const int vrows = PAIRED ? 2 * rows : rows;
    const int vtile = PAIRED ? 2 * tile_rows : tile_rows;
    const int position = blockIdx.z;
    const int nb = s.blocks;
    // Blocks staged at a time: the whole row when it fits the LDS, else chunks of K blocks walked in block
    // order (each chunk's terms are added to the row sums before the next chunk is staged).
    const int K = s.chunk_blocks;

    extern __shared__ uint32_t smem[];
    ActTile act;
    act.codes = smem;                                                          // kCodeStride * K dwords
    act.scales = reinterpret_cast<float*>(smem + kCodeStride * K);             // K
    act.sums = reinterpret_cast<int16_t*>(smem + (kCodeStride + 1) * K);       // 16 * K int16 = 8 * K dwords
    float* terms = reinterpret_cast<float*>(smem + kActDwords * K);            // tile_rows * K

    // Work items are (row, block) pairs of the chunk in row-major order; the G lanes of a pair share its
    // index, so the DPP group sums stay inside the pair. The next pair's payload is loaded before the
    // current one is reduced.
    const int lane = threadIdx.x & 63;
    const int c = lane % G;
    const uint8_t* w1 = PAIRED ? inline_members.m[1].w : m.w;  // the second member's payload (paired)
    // Pair p of the chunk starting at block b0 with kb blocks: row p / kb of the tile (paired: rows past
    // `rows` are the second member's), block b0 + p % kb.
    auto load_pair = [&](int b0, int kb, int p, Raw& r) {
        int row = p / kb;
        const int b = b0 + p % kb;
        const uint8_t* w = m.w;
        if (PAIRED && row >= rows) {
            row -= rows;
            w = w1;
        }
        if constexpr (FORMAT == kQ4_K) {
            q4k_load(w + static_cast<int64_t>(row_begin + row) * s.row_bytes + b * kBlockBytes, c, r);
        } else {
            // Q6_K: block b of tile row `row` is block (row_begin + row) * nb + b of the matrix.
            q6k_load_quarter(w, static_cast<int64_t>(m.rows) * nb, static_cast<int64_t>(row_begin + row) * nb + b,
                             c, r);
        }
    };
    // This slot's pairs are p0, p0 + kPairsPerStep, ...; kDepth of them are loaded before the activations
    // are staged, and each processed pair's registers are refilled with the pair kDepth further on, so kDepth
    // loads stay in flight.
    constexpr int kDepth = 3;
    const int p0 = threadIdx.x / G;
    int kb = min(K, nb);
    int mine = p0 < vrows * kb ? (vrows * kb - 1 - p0) / kPairsPerStep + 1 : 0;
    const float* xrow = m.x + static_cast<int64_t>(position) * s.columns;
    auto quad = [](const float* p, int i) {
        const u32x4 raw = load16_a4(reinterpret_cast<const uint8_t*>(p + i));
        return f32x4{__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                     __uint_as_float(raw[3])};
    };

    // The activation side is loaded first, then the weights: the waits for the activations then do not
    // cover the weight loads issued after them. Every thread issues the same loads (addresses past the end
    // are clamped and their values unused), so the load counts the waits are computed from are static.
    // Launches of up to kKintInlineMembers members (the decode step's latency-bound groups) do this; larger
    // groups stream from HBM and keep the registers for occupancy (the preloads take the plain-input Q4_K
    // kernel from 127 to 138 VGPRs, three waves per SIMD instead of four: 8960 x 1536 grouped measured
    // 5.53 against 5.86 TB/s).
    constexpr bool kPreload = INLINE;
    const int tid = threadIdx.x;
    const int j16 = tid & 15, bl0 = tid >> 4;
    f32x4 xpre[4];                 // plain input: this thread's 16 values of the first pass
    // Q8_K input: lane j16 of a 16-lane row copies block bl's code dwords [4 j16, 4 j16 + 4), and lane 0 its
    // scale, lanes 1 and 2 its group sums; the first kQ8KPasses passes are loaded here.
    u32x4 qcodes[kQ8KPasses], qaux[kQ8KPasses];
    auto q8k_load = [&](const uint8_t* row, int bl, u32x4& codes, u32x4& aux) {
        const uint8_t* block = row + static_cast<int64_t>(bl) * kQ8KBlockBytes;
        codes = load16_a4(block + 4 + 16 * j16);
        aux = load16_a4(block + (j16 == 0 ? 0 : 260 + 16 * (min(j16, 2) - 1)));
    };
    float npre_a[kNormPreload], npre_b[kNormPreload];  // RmsNorm input: the first terms of the sum of squares
    f32x4 wpre[4];                                      // RmsNorm input: the norm weights of the first pass
    if constexpr (XF == kInputPlain && kPreload) {
        const int i0 = 256 * min(bl0, kb - 1) + 16 * j16;
#pragma unroll
        for (int q = 0; q < 4; ++q) xpre[q] = quad(xrow, i0 + 4 * q);
    } else if constexpr (XF == kInputQ8K && kPreload) {
#pragma unroll
        for (int k = 0; k < kQ8KPasses; ++k)
            q8k_load(reinterpret_cast<const uint8_t*>(xf.a), min(bl0 + 16 * k, kb - 1), qcodes[k], qaux[k]);
    } else if constexpr (XF == kInputAddRmsNorm) {
#pragma unroll
        for (int k = 0; k < kNormPreload; ++k) {
            const int i = min(tid + kThreads * k, s.columns - 1);
            npre_a[k] = xf.a[i];
            npre_b[k] = xf.b ? xf.b[i] : 0.0f;
        }
        const int i0 = 256 * min(bl0, kb - 1) + 16 * j16;
#pragma unroll
        for (int q = 0; q < 4; ++q) wpre[q] = quad(xf.w, i0 + 4 * q);
    }
    Raw buf[kDepth];
#pragma unroll
    for (int i = 0; i < kDepth; ++i) load_pair(0, kb, min(p0 + i * kPairsPerStep, vrows * kb - 1), buf[i]);

    // Q8_K of the position's activations: one 16-lane row per block, sixteen blocks per pass. With an input
    // transform the activations are computed here from the operator's operands, in the operator's own
    // arithmetic (the RmsNorm sum of squares over the same 256-thread partition and tree, over the whole row).
    double scale = 0.0;
    // Summed RmsNorm input (residual + addend) kept in LDS after the reduction's 256 doubles.
    float* rstage = reinterpret_cast<float*>(smem + kint_red_offset(K, vtile) + 2 * kThreads);
    const bool rstaged = XF == kInputAddRmsNorm && s.columns <= kNormStageColumns;
    if constexpr (XF == kInputAddRmsNorm) {
        double* red = reinterpret_cast<double*>(smem + kint_red_offset(K, vtile));
        const bool writer = xf.residual_out && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
        double part = 0;
        auto term = [&](int i, float a, float b) {
            const float r = xf.b ? __fadd_rn(a, b) : a;
            if (writer) xf.residual_out[i] = r;
            if (rstaged) rstage[i] = r;  // visible to every thread after the reduction's barriers
            const double v = r;
            part = part + v * v;
        };
#pragma unroll
        for (int k = 0; k < kNormPreload; ++k)
            if (tid + kThreads * k < s.columns) term(tid + kThreads * k, npre_a[k], npre_b[k]);
        for (int i = tid + kThreads * kNormPreload; i < s.columns; i += kThreads)
            term(i, xf.a[i], xf.b ? xf.b[i] : 0.0f);
        scale = rms_scale(block_sum_256(part, red), s.columns, xf.epsilon);
    }
    // Block order from +0, as the reference accumulator (QuantizedKAvx2Kernel.cs:63, 90-94). A skipped
    // block stores +0, and adding +0 to a sum that starts at +0 never changes it.
    float acc = 0.0f;
    for (int b0 = 0;;) {
        if constexpr (XF == kInputQ8K) {
            // The producer's Q8_K row (Q8KCodec layout, 292 bytes per block: scale, 256 codes, 16 int16 group
            // sums) copied into the LDS arrays, one 16-lane row per block.
            const uint8_t* row = reinterpret_cast<const uint8_t*>(xf.a) + static_cast<int64_t>(b0) * kQ8KBlockBytes;
            auto put = [&](int bl, const u32x4& codes, const u32x4& aux) {
                *reinterpret_cast<u32x4*>(act.codes + kCodeStride * bl + 4 * j16) = codes;
                if (j16 == 0) {
                    act.scales[bl] = __uint_as_float(aux[0]);
                } else if (j16 <= 2) {
                    uint32_t* sums = reinterpret_cast<uint32_t*>(act.sums) + 8 * bl + 4 * (j16 - 1);
#pragma unroll
                    for (int e = 0; e < 4; ++e) sums[e] = aux[e];
                }
            };
            int bl = bl0;
            if (kPreload && b0 == 0) {
#pragma unroll
                for (int k = 0; k < kQ8KPasses; ++k)
                    if (bl0 + 16 * k < kb) put(bl0 + 16 * k, qcodes[k], qaux[k]);
                bl += 16 * kQ8KPasses;
            }
            for (; bl < kb; bl += kThreads / 16) {
                u32x4 codes, aux;
                q8k_load(row, bl, codes, aux);
                put(bl, codes, aux);
            }
        } else {
            auto stage = [&](int bl, const f32x4 (&x4)[4]) {
                float v[16];
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[4 * q + e] = x4[q][e];
                const Q8KRow16 qr = q8k_quantize_row16(v, lane);
                *reinterpret_cast<u32x4*>(act.codes + kCodeStride * bl + 4 * j16) =
                    u32x4{qr.packed[0], qr.packed[1], qr.packed[2], qr.packed[3]};
                act.sums[16 * bl + j16] = static_cast<int16_t>(qr.group_sum);
                if (j16 == 0) act.scales[bl] = qr.scale;
            };
            int bl = bl0;
            if constexpr (XF == kInputPlain && kPreload) {
                if (b0 == 0) {
                    if (bl < kb) stage(bl, xpre);
                    bl += kThreads / 16;
                }
            }
            for (; bl < kb; bl += kThreads / 16) {
                const int i0 = 256 * (b0 + bl) + 16 * j16;
                f32x4 x4[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if constexpr (XF == kInputPlain) {
                        x4[q] = quad(xrow, i0 + 4 * q);
                    } else if constexpr (XF == kInputAddRmsNorm) {
                        const bool first = b0 == 0 && bl == bl0;  // the pass whose weights were preloaded
                        const f32x4 w4 = first ? wpre[q] : quad(xf.w, i0 + 4 * q);
                        f32x4 r4;
                        if (rstaged) {
                            r4 = *reinterpret_cast<const f32x4*>(rstage + i0 + 4 * q);
                        } else {
                            const f32x4 a4 = quad(xf.a, i0 + 4 * q);
                            f32x4 b4 = {0.0f, 0.0f, 0.0f, 0.0f};
                            if (xf.b) b4 = quad(xf.b, i0 + 4 * q);
#pragma unroll
                            for (int e = 0; e < 4; ++e) r4[e] = xf.b ? __fadd_rn(a4[e], b4[e]) : a4[e];
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) x4[q][e] = rms_value(r4[e], scale, w4[e]);
                    } else {
                        const f32x4 g4 = quad(xf.a, i0 + 4 * q), u4 = quad(xf.b, i0 + 4 * q);
#pragma unroll
                        for (int e = 0; e < 4; ++e) x4[q][e] = swiglu_value(g4[e], u4[e]);
                    }
                }
                stage(bl, x4);
            }
        }
        __syncthreads();  // activations of the chunk staged
        // The FP32 term of pair p (valid on the pair's last lane).
        auto term_of = [&](const Raw& cur, int p) {
            const int bl = p % kb;  // block of the chunk (its staged activations)
            float term = 0.0f;
            if constexpr (FORMAT == kQ4_K) {
                int dot, min_part;
                q4k_dot(cur, act, bl, c, dot, min_part);
                dot = group_sum_last_int<G>(dot);
                min_part = group_sum_last_int<G>(min_part);
                const float a = act.scales[bl];
                if (a != 0.0f) {  // zero activation block: skipped (QuantizedKAvx2Kernel.cs:86)
                    const float dA = __fmul_rn(half_bits_to_float(cur.head[0] & 0xFFFFu), a);
                    const float dminA = __fmul_rn(half_bits_to_float(cur.head[0] >> 16), a);
                    term = __fsub_rn(__fmul_rn(dA, static_cast<float>(dot)),
                                     __fmul_rn(dminA, static_cast<float>(min_part)));
                }
            } else {
                int dot = q6k_dot(cur, act, bl, c);
                dot = group_sum_last_int<G>(dot);
                const float a = act.scales[bl];
                if (a != 0.0f) term = __fmul_rn(__fmul_rn(a, q6k_d(cur)), static_cast<float>(dot));
            }
            return term;
        };
        // The slot's pairs in order; each processed pair's registers are refilled with the pair kDepth further
        // on. (Computing a round's kDepth pairs unconditionally, to interleave their chains, measured slower on
        // the decode step's small launches: the slots there hold fewer than kDepth pairs.)
        for (int base = 0; base < mine; base += kDepth) {
#pragma unroll
            for (int i = 0; i < kDepth; ++i) {
                const int k = base + i;
                if (k < mine) {
                    const float t = term_of(buf[i], p0 + k * kPairsPerStep);
                    if (c == G - 1) terms[p0 + k * kPairsPerStep] = t;
                    if (k + kDepth < mine) load_pair(b0, kb, p0 + (k + kDepth) * kPairsPerStep, buf[i]);
                }
            }
        }
        __syncthreads();  // the chunk's terms are in LDS
        if (threadIdx.x < vrows) {
            const float* t = terms + threadIdx.x * kb;
            for (int b = 0; b < kb; ++b) acc = __fadd_rn(acc, t[b]);
        }
        b0 += K;
        if (b0 >= nb) break;
        // Next chunk: its first pairs' payload is requested before the LDS is released.
        kb = min(K, nb - b0);
        mine = p0 < vrows * kb ? (vrows * kb - 1 - p0) / kPairsPerStep + 1 : 0;
#pragma unroll
        for (int i = 0; i < kDepth; ++i) load_pair(b0, kb, min(p0 + i * kPairsPerStep, vrows * kb - 1), buf[i]);
        __syncthreads();  // every thread is done with this chunk's activations and terms
    }
    if constexpr (!PAIRED) {
        if (threadIdx.x < rows) store_f32(m.y + static_cast<int64_t>(position) * m.rows + row_begin + threadIdx.x, acc);
    } else if (threadIdx.x < 64) {
        // The first wave holds every row sum: lane t < rows the first member's row row_begin + t, lane rows + t
        // the second member's.
        const int t = threadIdx.x;
        if (t < vrows) store_f32((t < rows ? m.y : inline_members.m[1].y) + row_begin + (t < rows ? t : t - rows), acc);
        const float up = __shfl(acc, (t + rows) & 63, 64);
        const float activated = swiglu_value(acc, up);
        if (!out.q8k) {  // SwiGlu only
            if (t < rows) store_f32(out.activated + row_begin + t, activated);
            return;
        }
        // SwiGlu of the workgroup's rows, stored as agent-scope atomics so the workgroup that quantizes the run
        // reads them coherently from any XCD, then waited for (every store of this wave acknowledged) before
        // this workgroup is counted in: a count the quantizer sees implies the values it reads are there.
        if (t < rows)
            __hip_atomic_store(out.activated + row_begin + t, activated, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t seen = 0;
        if (t == 0)
            seen = __hip_atomic_fetch_add(out.counters + (row_begin >> 8), 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        seen = static_cast<uint32_t>(__shfl(static_cast<int>(seen), 0, 64));
        const uint32_t arrivals = 256u / static_cast<uint32_t>(tile_rows);  // a power of two
        if (((seen + 1u) & (arrivals - 1u)) == 0u) {
            // The last of the run's workgroups: Q8_K of its 256 SwiGlu values (Q8KCodec.QuantizeBlock).
            const int run = row_begin >> 8;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v[i] = __hip_atomic_load(out.activated + 256 * run + 4 * t + i, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            const Q8KLane q = q8k_quantize_values(v, t);
            uint8_t* dst = out.q8k + static_cast<int64_t>(run) * kQ8KBlockBytes;
            if (q.zero) {
                uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
                for (int i = t; i < kQ8KBlockBytes / 4; i += 64) d32[i] = 0u;
            } else {
                reinterpret_cast<uint32_t*>(dst + 4)[t] = q.packed;
                if ((t & 3) == 0) reinterpret_cast<int16_t*>(dst + 260)[t >> 2] = static_cast<int16_t>(q.group_sum);
                if (t == 0) reinterpret_cast<float*>(dst)[0] = q.scale;
            }
        }
    }
}

}  // namespace

hipError_t launch_q8k_quantize(const float* x, int columns, int positions, uint8_t* out, hipStream_t stream) {
    if (columns <= 0 || positions <= 0) return hipSuccess;
    dim3 grid(columns / 256, positions);
    q8k_quantize_kernel<<<grid, 64, 0, stream>>>(x, columns, out);
    return hipGetLastError();
}

size_t kint_lds_bytes(int blocks, int rms_columns) {
    const size_t staged = rms_columns <= kNormStageColumns ? static_cast<size_t>(rms_columns) * sizeof(float) : 0;
    return static_cast<size_t>(kint_red_offset(blocks, kTileRows)) * sizeof(uint32_t) + kThreads * sizeof(double) +
           staged;
}

int kint_max_blocks() {
    return static_cast<int>((64 * 1024 - kThreads * sizeof(double) - 4) / ((kActDwords + kTileRows) * sizeof(uint32_t)));
}

namespace {

template <int XF, bool PAIRED = false>
hipError_t launch_kint(const MatDesc* members, const MatDesc* device_members, int count, LaunchShape s,
                       const InputTransform& xf, hipStream_t stream, const OutputSwiGluQ8K& out = {}) {
    if (count <= 0 || s.rows_max <= 0 || s.positions <= 0) return hipSuccess;
    if (count > kKintInlineMembers && !device_members) return hipErrorInvalidValue;
    if (PAIRED && (count != 2 || s.positions != 1 || s.rows_max % 256 != 0 || members[0].rows != s.rows_max ||
                   members[1].rows != s.rows_max))
        return hipErrorInvalidValue;
    // Rows per workgroup: 64, halved (down to 4) while the grid has fewer than 1024 workgroups and either a
    // thread slot would hold more than three (row, block) pairs (the pairs it prefetches before quantizing)
    // or the grid has fewer than 192 workgroups. Measured on the decode step's groups: q/k/v and o take 8-16
    // rows, gate/up 32, down (35 blocks) 4; large grouped launches keep 64. Then halved while a workgroup
    // would stream more than 256 KB of payload, so long rows leave no long tail of workgroups at the end of
    // a launch (1536 x 8960 grouped: Q6_K 5.43 -> 5.76 TB/s, Q4_K 5.70 -> 5.86 TB/s at 32 rows; 16 rows
    // measured slower).
    const int64_t launched = static_cast<int64_t>(count) * s.positions;
    auto groups_for = [&](int t) { return launched * ((s.rows_max + t - 1) / t); };
    int tile = kTileRows;
    while (tile > 4 && groups_for(tile) < 1024 && (tile * s.blocks > 192 || groups_for(tile) < 192)) tile /= 2;
    while (tile > 4 && static_cast<int64_t>(tile) * s.row_bytes > 256 * 1024) tile /= 2;
    // Paired: each workgroup owns `tile` rows of both members, so half the rows of the unpaired tile keep the
    // work per workgroup and the workgroup count (at most 32 rows, so the 2 * tile row sums fit one wave).
    if (PAIRED) tile = max(4, min(32, tile / 2));
    s.rows_per_wg = tile;
    // Rows wider than the LDS holds are staged kint_max_blocks() blocks at a time.
    s.chunk_blocks = s.blocks < kint_max_blocks() ? s.blocks : kint_max_blocks();
    dim3 grid((s.rows_max + tile - 1) / tile, PAIRED ? 1 : count, s.positions);
    const size_t lds = kint_lds_bytes(s.chunk_blocks, XF == kInputAddRmsNorm ? s.columns : 0);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    KintMembers inline_members{};
    const MatDesc* group = nullptr;
    if (count <= kKintInlineMembers)
        for (int i = 0; i < count; ++i) inline_members.m[i] = members[i];
    else
        group = device_members;
    if constexpr (PAIRED) {
        if (s.format == kQ4_K)
            gemv_kint_kernel<kQ4_K, XF, true, true><<<grid, kThreads, lds, stream>>>(inline_members, group, s, xf, out);
        else if (s.format == kQ6_K)
            gemv_kint_kernel<kQ6_K, XF, true, true><<<grid, kThreads, lds, stream>>>(inline_members, group, s, xf, out);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (s.format == kQ4_K && group)
        gemv_kint_kernel<kQ4_K, XF, false, false><<<grid, kThreads, lds, stream>>>(inline_members, group, s, xf, out);
    else if (s.format == kQ4_K)
        gemv_kint_kernel<kQ4_K, XF, true, false><<<grid, kThreads, lds, stream>>>(inline_members, group, s, xf, out);
    else if (s.format == kQ6_K && group)
        gemv_kint_kernel<kQ6_K, XF, false, false><<<grid, kThreads, lds, stream>>>(inline_members, group, s, xf, out);
    else if (s.format == kQ6_K)
        gemv_kint_kernel<kQ6_K, XF, true, false><<<grid, kThreads, lds, stream>>>(inline_members, group, s, xf, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_kint(const MatDesc* members, const MatDesc* device_members, int count, LaunchShape s,
                            hipStream_t stream) {
    return launch_kint<kInputPlain>(members, device_members, count, s, InputTransform{}, stream);
}

hipError_t launch_gemv_kint_transformed(const MatDesc* members, const MatDesc* device_members, int count,
                                        LaunchShape s, const InputTransform& xf, hipStream_t stream) {
    if (s.positions != 1 || !xf.a) return hipErrorInvalidValue;
    switch (xf.kind) {
        case kInputPlain: return launch_kint<kInputPlain>(members, device_members, count, s, xf, stream);
        case kInputAddRmsNorm:
            if (!xf.w) return hipErrorInvalidValue;
            return launch_kint<kInputAddRmsNorm>(members, device_members, count, s, xf, stream);
        case kInputSwiGlu:
            if (!xf.b) return hipErrorInvalidValue;
            return launch_kint<kInputSwiGlu>(members, device_members, count, s, xf, stream);
        case kInputQ8K: return launch_kint<kInputQ8K>(members, device_members, count, s, xf, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_kint_swiglu(const MatDesc* members, LaunchShape s, const InputTransform& xf,
                                   const OutputSwiGluQ8K& out, hipStream_t stream) {
    if (s.positions != 1 || !out.activated || (out.q8k && !out.counters)) return hipErrorInvalidValue;
    switch (xf.kind) {
        case kInputPlain: return launch_kint<kInputPlain, true>(members, nullptr, 2, s, xf, stream, out);
        case kInputAddRmsNorm:
            if (!xf.a || !xf.w) return hipErrorInvalidValue;
            return launch_kint<kInputAddRmsNorm, true>(members, nullptr, 2, s, xf, stream, out);
        case kInputQ8K:
            if (!xf.a) return hipErrorInvalidValue;
            return launch_kint<kInputQ8K, true>(members, nullptr, 2, s, xf, stream, out);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace satori
