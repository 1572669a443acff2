// FP32-activation MatVec over packed GGUF blocks for gfx950: Q8_0, Q4_0, Q4_K and Q6_K, computed directly
// on the payload without materialising weights (Ternary2 has its own kernel on a panel layout).
//
// Work decomposition. A row is cut into fixed "chunks" (one Q8_0/Q4_0 block, an eighth of a Q4_K block, a
// quarter of a Q6_K block). A wave64 handles 64 / L rows at a time with L lanes per row; lane j of a row
// owns chunks j, j + L, ... Consecutive lanes read consecutive chunks, so a row's payload is read by
// contiguous loads. The activation vector is staged once per workgroup in LDS; when every row has at most
// L chunks each lane pulls its chunk's activations into registers once and keeps them for every row it
// visits.
// Row sums are reduced across the L lanes by cross-lane shuffles.
//
// Arithmetic per format follows the reference decoders (file:line cited on each decoder); products
// and sums are FP32, accumulated in a different order from the scalar reference, which the tests bound
// by the reference's own 1e-5 * sum|w*x| criterion.
#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

// Workgroups are 256 threads, or 512 when the staged activations take more than a third of the LDS (long
// rows): the LDS then caps the workgroups per CU, and wider workgroups keep more waves resident.
constexpr int kThreads = 256;
constexpr int kWideThreads = 512;
constexpr int kWideLdsBytes = 40 * 1024;

// ------------------------------------------------------------------------------------------------
// Q8_0: f16 d + 32 int8, w = d * q (docs/gguf-subset-v1.md:94; QuantizedMatVec.ExecuteScalar,
// src/Satori.Core/QuantizedMatVec.cs:66-74). 34-byte blocks are 2-byte aligned: codes are assembled from
// aligned dword loads with v_alignbyte; int8 -> float is one SDWA conversion per weight.
// ------------------------------------------------------------------------------------------------
struct Q8_0Chunk {
    static constexpr int kRowUnroll = 2;
    static constexpr bool kPipelineShortLanes = false;
    // Payload cap per workgroup (0: none): more, smaller workgroups leave a shorter tail at the end of a large
    // launch (4096x4096 grouped: 5.79 -> 5.96 TB/s); Q4_0 measured slower with the cap (its longer rows make
    // the per-workgroup activation staging the larger cost).
    static constexpr int kMaxWorkgroupPayload = 256 * 1024;
    static constexpr int kWeights = 32;
    static constexpr int kPadShift = 5;
    struct Regs {
        uint32_t q[8];
        uint32_t scale;  // FP16 bits, converted where the dot uses them (not at the load, which would wait)
    };
    struct Consts {};
    __device__ static Consts consts() { return Consts{}; }
    __device__ static int chunks(const LaunchShape& s) { return s.blocks; }
    __device__ static int padded_columns(const LaunchShape& s) { return s.columns; }
    // Regrouped device layout: 32-byte code records, then the FP16 scales. A row's records and scales start
    // at fixed addresses, computed once per row.
    struct Row {
        const uint8_t* codes;
        const uint8_t* scales;
    };
    __device__ static Row row_ref(const MatDesc& m, const LaunchShape& s, int row) {
        const int64_t first = static_cast<int64_t>(row) * s.blocks;
        return Row{m.w + first * 32, m.w + static_cast<int64_t>(m.rows) * s.blocks * 32 + first * 2};
    }
    __device__ static void load(const Row& w, int chunk, Regs& r) {
        const u32x4 a = load16_a4(w.codes + chunk * 32), b = load16_a4(w.codes + chunk * 32 + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.q[i] = a[i];
            r.q[4 + i] = b[i];
        }
        r.scale = load2_a2(w.scales + chunk * 2);
    }
    template <class XF>
    __device__ static void load_x(XF xf, int chunk, float (&x)[kWeights]) {
#pragma unroll
        for (int j = 0; j < kWeights; j += 4) xf.quad(32 * chunk + j, x + j);
    }
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const Consts&) {
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            acc0 = __builtin_fmaf(sbyte_to_float(r.q[d], 0), x[4 * d + 0], acc0);
            acc1 = __builtin_fmaf(sbyte_to_float(r.q[d], 1), x[4 * d + 1], acc1);
            acc0 = __builtin_fmaf(sbyte_to_float(r.q[d], 2), x[4 * d + 2], acc0);
            acc1 = __builtin_fmaf(sbyte_to_float(r.q[d], 3), x[4 * d + 3], acc1);
        }
        return half_bits_to_float(r.scale) * (acc0 + acc1);
    }
};

// ------------------------------------------------------------------------------------------------
// Q4_0: f16 d + 16 bytes, w[j] = d * ((b[j] & 15) - 8), w[j + 16] = d * ((b[j] >> 4) - 8)
// (docs/gguf-subset-v1.md:93; QuantizedMatVec.cs:71-72). The device copy holds every code byte XOR 0x88
// (applied at upload), so each nibble is q ^ 8, whose signed 4-bit value is q - 8; a mask (and a shift for
// the low nibbles) per four weights turns the nibbles into the signed bytes 16 * (q - 8), and the conversion
// is one SDWA op per weight; the factor 16 is removed exactly with the power-of-two scale 1/16.
// ------------------------------------------------------------------------------------------------
struct Q4_0Chunk {
    static constexpr int kRowUnroll = 2;
    // Long rows with fewer than 64 lanes each load the next two chunks while computing the current two
    // (4096 x 11008 grouped: 5.23 -> 5.71 TB/s at 163 VGPRs, three waves per SIMD instead of four); the
    // other formats' register sets are larger, and their loops keep one step in flight.
    static constexpr bool kPipelineShortLanes = true;
    static constexpr int kMaxWorkgroupPayload = 0;
    static constexpr int kWeights = 32;
    static constexpr int kPadShift = 5;
    struct Regs {
        uint32_t q[4];
        uint32_t scale;  // FP16 bits, converted where the dot uses them (not at the load, which would wait)
    };
    struct Consts {};
    __device__ static Consts consts() { return Consts{}; }
    __device__ static int chunks(const LaunchShape& s) { return s.blocks; }
    __device__ static int padded_columns(const LaunchShape& s) { return s.columns; }
    // Regrouped device layout: 16-byte code records (bytes XOR 0x88), then the FP16 scales.
    struct Row {
        const uint8_t* codes;
        const uint8_t* scales;
    };
    __device__ static Row row_ref(const MatDesc& m, const LaunchShape& s, int row) {
        const int64_t first = static_cast<int64_t>(row) * s.blocks;
        return Row{m.w + first * 16, m.w + static_cast<int64_t>(m.rows) * s.blocks * 16 + first * 2};
    }
    // Non-temporal code loads: the codes are read once, and keeping them out of the caches leaves the staged
    // activations' lines resident (11008 x 4096 grouped: 5.31 -> 5.72 TB/s; Q8_0 measured slower with them).
    __device__ static void load(const Row& w, int chunk, Regs& r) {
        const u32x4 a = stream16(w.codes + chunk * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = a[i];
        r.scale = load2_a2(w.scales + chunk * 2);
    }
    template <class XF>
    __device__ static void load_x(XF xf, int chunk, float (&x)[kWeights]) {
#pragma unroll
        for (int j = 0; j < kWeights; j += 4) xf.quad(32 * chunk + j, x + j);
    }
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const Consts&) {
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t v = r.q[d];                       // nibbles q ^ 8 (signed 4-bit value q - 8)
            const uint32_t lo = (v << 4) & 0xF0F0F0F0u;      // bytes 16 * (q_low - 8): weights 4d + i
            const uint32_t hi = v & 0xF0F0F0F0u;             // bytes 16 * (q_high - 8): weights 16 + 4d + i
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc0 = __builtin_fmaf(sbyte_to_float(lo, i), x[4 * d + i], acc0);
                acc1 = __builtin_fmaf(sbyte_to_float(hi, i), x[16 + 4 * d + i], acc1);
            }
        }
        return half_bits_to_float(r.scale) * ((acc0 + acc1) * 0.0625f);
    }
};

// ------------------------------------------------------------------------------------------------
// Q4_K, FP32 activations (Q4KCodec.DotBlock, src/Satori.Core/Q4KCodec.cs:39-65): 144-byte super-block,
// f16 d @0, f16 dmin @2, 6-bit scales/mins @4..15 (Q4KCodec.GetScaleMin, :24-36), nibbles @16.
// Chunk k of a block (k = 0..7) is qs[16k .. 16k + 16): low nibbles are weights 64g + 16h + i of
// sub-block 2g, high nibbles weights 64g + 32 + 16h + i of sub-block 2g + 1 (g = k / 2, h = k % 2).
// The weight d*s*q - dmin*m is one FMA.
// ------------------------------------------------------------------------------------------------

struct Q4_KChunk {
    static constexpr int kRowUnroll = 2;
    static constexpr bool kPipelineShortLanes = false;
    static constexpr int kMaxWorkgroupPayload = 0;
    static constexpr int kWeights = 32;
    static constexpr int kPadShift = 6;
    struct Regs {
        u32x4 head;
        u32x4 qs;
        int g;
    };
    struct Consts {};
    __device__ static Consts consts() { return Consts{}; }
    __device__ static int chunks(const LaunchShape& s) { return s.blocks * 8; }
    __device__ static int padded_columns(const LaunchShape& s) { return s.columns; }
    using Row = const uint8_t*;  // the row's first block
    __device__ static Row row_ref(const MatDesc& m, const LaunchShape& s, int row) {
        return m.w + static_cast<int64_t>(row) * s.row_bytes;
    }
    __device__ static void load(Row w, int chunk, Regs& r) {
        const uint8_t* block = w + (chunk >> 3) * 144;
        r.head = load16_a4(block);
        r.qs = load16_a4(block + 16 + 16 * (chunk & 7));
        r.g = (chunk & 7) >> 1;
    }
    template <class XF>
    __device__ static void load_x(XF xf, int chunk, float (&x)[kWeights]) {
        const int base = (chunk >> 3) * 256 + 64 * ((chunk & 7) >> 1) + 16 * (chunk & 1);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            xf.quad(base + i, x + i);
            xf.quad(base + 32 + i, x + 16 + i);
        }
    }
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const Consts&) {
        const float d = half_bits_to_float(r.head[0] & 0xFFFFu);
        const float dmin = half_bits_to_float(r.head[0] >> 16);
        int s0, m0, s1, m1;
        q4k_scale_min(2 * r.g, r.head, s0, m0);
        q4k_scale_min(2 * r.g + 1, r.head, s1, m1);
        const float dl = d * static_cast<float>(s0), ml = dmin * static_cast<float>(m0);
        const float dh = d * static_cast<float>(s1), mh = dmin * static_cast<float>(m1);
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t lo = r.qs[w] & 0x0F0F0F0Fu;
            const uint32_t hi = (r.qs[w] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc0 = __builtin_fmaf(__builtin_fmaf(dl, byte_to_float(lo, i), -ml), x[4 * w + i], acc0);
                acc1 = __builtin_fmaf(__builtin_fmaf(dh, byte_to_float(hi, i), -mh), x[16 + 4 * w + i], acc1);
            }
        }
        return acc0 + acc1;
    }
};

// ------------------------------------------------------------------------------------------------
// Q6_K, FP32 activations (Q6KCodec.DotBlock, src/Satori.Core/Q6KCodec.cs:22-51): 210-byte super-block,
// ql[128] @0, qh[64] @128, int8 scales[16] @192, f16 d @208, read from the regrouped device layout
// (Q6KLayout). Chunk = quarter c = 2h + t of a block: l in [16t, 16t + 16) for all four k, i.e. weights
// 128h + 32k + l with scale 8h + 2k + t. Weight d*sc*(q - 32) is fma(d*sc, q, -32*d*sc), the same single
// rounding of the same product as the reference's (d*sc)*(q-32) since 32*d*sc is exact.
// ------------------------------------------------------------------------------------------------
struct Q6_KChunk {
    static constexpr int kRowUnroll = 1;
    static constexpr bool kPipelineShortLanes = false;
    static constexpr int kMaxWorkgroupPayload = 0;
    static constexpr int kWeights = 64;
    static constexpr int kPadShift = 7;
    using Regs = Q6KQuarter;
    struct Consts {};
    __device__ static Consts consts() { return Consts{}; }
    __device__ static int chunks(const LaunchShape& s) { return s.blocks * 4; }
    __device__ static int padded_columns(const LaunchShape& s) { return s.columns; }
    struct Row {
        const uint8_t* w;
        int64_t count, first;  // blocks of the matrix; the row's first block
    };
    __device__ static Row row_ref(const MatDesc& m, const LaunchShape& s, int row) {
        return Row{m.w, static_cast<int64_t>(m.rows) * s.blocks, static_cast<int64_t>(row) * s.blocks};
    }
    __device__ static void load(const Row& w, int chunk, Regs& r) {
        q6k_load_quarter(w.w, w.count, w.first + (chunk >> 2), chunk & 3, r);
    }
    template <class XF>
    __device__ static void load_x(XF xf, int chunk, float (&x)[kWeights]) {
        const int base = (chunk >> 2) * 256 + 128 * ((chunk & 3) >> 1) + 16 * (chunk & 1);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int i = 0; i < 16; i += 4) xf.quad(base + 32 * k + i, x + 16 * k + i);
    }
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const Consts&) {
        float ds[4], bias[4];
        const float d = q6k_d(r);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int8_t s = static_cast<int8_t>(r.sc >> (8 * k));  // scale 8h + 2k + t
            ds[k] = d * static_cast<float>(s);
            bias[k] = -32.0f * ds[k];
        }
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t a = r.qla[w], b = r.qlb[w], h = r.qh[w];
            const uint32_t q[4] = {
                (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u),
                (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u),
                ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u),
                ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u),
            };
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float weight = __builtin_fmaf(ds[k], byte_to_float(q[k], i), bias[k]);
                    if (i & 1)
                        acc1 = __builtin_fmaf(weight, x[16 * k + 4 * w + i], acc1);
                    else
                        acc0 = __builtin_fmaf(weight, x[16 * k + 4 * w + i], acc0);
                }
        }
        return acc0 + acc1;
    }
};

// Reads of the activations by aligned quads (i % 4 == 0): one 16-byte LDS read of the staged copy (element i
// at i + 4 * (i >> PAD), so a quad stays contiguous and the quads of neighbouring lanes, 32, 64 or 128
// elements apart plus the padding, start on different banks), or of global memory, zero past the end.
template <int PAD, bool XLDS>
struct XReader {
    const float* xs;
    const float* x;
    int columns;
    __device__ __forceinline__ void quad(int i, float* out) const {
        if constexpr (XLDS) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(xs + i + ((i >> PAD) << 2));
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = v[e];
        } else if (i + 3 < columns) {
            const u32x4 v = load16_a4(reinterpret_cast<const uint8_t*>(x + i));
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = __uint_as_float(v[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = i + e < columns ? load_f32(x + i + e) : 0.0f;
        }
    }
};

// ------------------------------------------------------------------------------------------------
// The kernel. Grid: x = row tiles of s.rows_per_wg rows, y = group member, z = position.
// ONE: every row has at most L chunks, so a lane's activations are loaded once per workgroup.
// XLDS: the activations fit the LDS budget; otherwise they are read from global memory (L2).
// ------------------------------------------------------------------------------------------------
template <class F, int L, bool ONE, bool XLDS, int THREADS>
__global__ __launch_bounds__(THREADS) void gemv_float_kernel(MatDesc one, const MatDesc* __restrict__ group,
                                                               LaunchShape s) {
    const MatDesc m = group ? group[blockIdx.y] : one;
    const int row_begin = blockIdx.x * s.rows_per_wg;
    if (row_begin >= m.rows) return;  // whole workgroup leaves together
    const int row_end = min(row_begin + s.rows_per_wg, m.rows);
    const int position = blockIdx.z;
    const float* __restrict__ x = m.x + static_cast<int64_t>(position) * s.columns;
    float* __restrict__ y = m.y + static_cast<int64_t>(position) * m.rows;
    const int columns = s.columns;

    // Staged activations: element i lives at i + 4 * (i >> kPadShift), which spreads the 128-bit reads
    // of neighbouring lanes over all 32 LDS banks.
    extern __shared__ float xs[];
    if constexpr (XLDS) {
        const int padded = F::padded_columns(s);
        for (int i = threadIdx.x; i < padded; i += THREADS)
            xs[i + ((i >> F::kPadShift) << 2)] = i < columns ? load_f32(x + i) : 0.0f;
        __syncthreads();
    }
    const XReader<F::kPadShift, XLDS> xf{xs, x, columns};

    constexpr int kRowsPerPass = 64 / L;
    constexpr int kStride = THREADS / 64 * kRowsPerPass;  // rows between a lane's consecutive rows
    constexpr int kRowUnroll = F::kRowUnroll;
    constexpr int kStep = kStride * kRowUnroll;      // rows per iteration of the whole workgroup
    // Software-pipelined chunk loop (see the format): staged activations and fewer than 64 lanes per row.
    constexpr bool kPipelined = F::kPipelineShortLanes && L < 64 && XLDS;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane / L;
    const int lr = lane % L;
    const int nchunks = F::chunks(s);
    const typename F::Consts k = F::consts();
    const int first = row_begin + wave * kRowsPerPass;  // wave-uniform

    float xr[F::kWeights];
    if constexpr (ONE) {
        // Each lane owns one chunk of every row: its activations stay in registers, and the next
        // iteration's rows are loaded while the current ones are computed.
        const bool active = lr < nchunks;
        if (active) {
            F::load_x(xf, lr, xr);
        } else {
#pragma unroll
            for (int j = 0; j < F::kWeights; ++j) xr[j] = 0.0f;
        }
        typename F::Regs cur[kRowUnroll], nxt[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const int row = first + u * kStride + sub;
            if (active && row < row_end) F::load(F::row_ref(m, s, row), lr, cur[u]);
        }
        for (int base = first; base < row_end; base += kStep) {
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int row = base + kStep + u * kStride + sub;
                if (active && row < row_end) F::load(F::row_ref(m, s, row), lr, nxt[u]);
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int row = base + u * kStride + sub;
                const float partial = (active && row < row_end) ? F::dot(cur[u], xr, k) : 0.0f;
                const float total = group_sum_last<L>(partial);
                if (lr == L - 1 && row < row_end) store_f32(y + row, total);
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) cur[u] = nxt[u];
        }
    } else {
        for (int base = first; base < row_end; base += kStep) {
            float acc[kRowUnroll];
            typename F::Row rows[kRowUnroll];  // (rows past the end are never loaded)
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                acc[u] = 0.0f;
                rows[u] = F::row_ref(m, s, base + u * kStride + sub);
            }
            int c = lr;
            if constexpr (kPipelined) {
                // Two chunks per step, the next step's loaded while this step's are computed: register sets A
                // and B take turns. Rows past the end load and compute on the last live row (nothing is
                // stored for them), so no load sits behind a branch.
                typename F::Row live[kRowUnroll];
#pragma unroll
                for (int u = 0; u < kRowUnroll; ++u)
                    live[u] = F::row_ref(m, s, min(base + u * kStride + sub, row_end - 1));
                auto load_pair = [&](int cc, typename F::Regs (&r0)[kRowUnroll],
                                     typename F::Regs (&r1)[kRowUnroll]) {
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) {
                        F::load(live[u], cc, r0[u]);
                        F::load(live[u], cc + L, r1[u]);
                    }
                };
                auto dot_pair = [&](int cc, const typename F::Regs (&r0)[kRowUnroll],
                                    const typename F::Regs (&r1)[kRowUnroll]) {
                    F::load_x(xf, cc, xr);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) acc[u] += F::dot(r0[u], xr, k);
                    F::load_x(xf, cc + L, xr);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) acc[u] += F::dot(r1[u], xr, k);
                };
                // The steady-state loop issues its loads unconditionally, so the compiler's wait before each
                // step counts exactly the loads issued after that step's own.
                typename F::Regs a0[kRowUnroll], a1[kRowUnroll], b0[kRowUnroll], b1[kRowUnroll];
                int pairs = lr < nchunks ? (nchunks - lr + L - 1) / L / 2 : 0;
                if (pairs > 0) {
                    load_pair(c, a0, a1);
                    for (; pairs >= 3; pairs -= 2) {  // (scheduling barriers keep each step's loads in place)
                        load_pair(c + 2 * L, b0, b1);
                        __builtin_amdgcn_sched_barrier(0);
                        dot_pair(c, a0, a1);
                        __builtin_amdgcn_sched_barrier(0);
                        load_pair(c + 4 * L, a0, a1);
                        __builtin_amdgcn_sched_barrier(0);
                        dot_pair(c + 2 * L, b0, b1);
                        __builtin_amdgcn_sched_barrier(0);
                        c += 4 * L;
                    }
                    if (pairs == 2) {
                        load_pair(c + 2 * L, b0, b1);
                        dot_pair(c, a0, a1);
                        dot_pair(c + 2 * L, b0, b1);
                        c += 4 * L;
                    } else {
                        dot_pair(c, a0, a1);
                        c += 2 * L;
                    }
                }
            } else {
                for (; c + L < nchunks; c += 2 * L) {  // two chunks per step: both rows' loads of both in flight
                    typename F::Regs ra[kRowUnroll], rb[kRowUnroll];
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) {
                        const int row = base + u * kStride + sub;
                        if (row < row_end) {
                            F::load(rows[u], c, ra[u]);
                            F::load(rows[u], c + L, rb[u]);
                        }
                    }
                    F::load_x(xf, c, xr);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) {
                        const int row = base + u * kStride + sub;
                        if (row < row_end) acc[u] += F::dot(ra[u], xr, k);
                    }
                    F::load_x(xf, c + L, xr);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) {
                        const int row = base + u * kStride + sub;
                        if (row < row_end) acc[u] += F::dot(rb[u], xr, k);
                    }
                }
            }
            for (; c < nchunks; c += L) {
                F::load_x(xf, c, xr);
                typename F::Regs regs[kRowUnroll];
#pragma unroll
                for (int u = 0; u < kRowUnroll; ++u) {
                    const int row = base + u * kStride + sub;
                    if (row < row_end) F::load(rows[u], c, regs[u]);
                }
#pragma unroll
                for (int u = 0; u < kRowUnroll; ++u) {
                    const int row = base + u * kStride + sub;
                    if (row < row_end) acc[u] += F::dot(regs[u], xr, k);
                }
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int row = base + u * kStride + sub;
                const float total = group_sum_last<L>(acc[u]);
                if (lr == L - 1 && row < row_end) store_f32(y + row, total);
            }
        }
    }
}

// LDS budget for the staged activations.
constexpr int kMaxLdsBytes = 64 * 1024;

template <class F>
size_t staged_lds_bytes(int padded) {
    return static_cast<size_t>(padded + 4 * (padded >> F::kPadShift) + 4) * sizeof(float);
}

template <class F, int L, bool ONE, int THREADS>
hipError_t launch_variant(const MatDesc& one, const MatDesc* group, const LaunchShape& s, dim3 grid, int padded,
                          hipStream_t stream) {
    const size_t lds = staged_lds_bytes<F>(padded);
    if (lds <= kMaxLdsBytes)
        gemv_float_kernel<F, L, ONE, true, THREADS><<<grid, THREADS, lds, stream>>>(one, group, s);
    else
        gemv_float_kernel<F, L, ONE, false, THREADS><<<grid, THREADS, 0, stream>>>(one, group, s);
    return hipGetLastError();
}

template <class F, int L>
hipError_t launch_lanes(const MatDesc& one, const MatDesc* group, const LaunchShape& s, dim3 grid, int padded,
                        bool one_chunk, bool wide, hipStream_t stream) {
    if (one_chunk) return launch_variant<F, L, true, kThreads>(one, group, s, grid, padded, stream);
    if (wide) return launch_variant<F, L, false, kWideThreads>(one, group, s, grid, padded, stream);
    return launch_variant<F, L, false, kThreads>(one, group, s, grid, padded, stream);
}

template <class F>
hipError_t launch_format(const MatDesc& one, const MatDesc* group, int count, LaunchShape s, int chunks,
                         int padded, hipStream_t stream) {
    // Lanes per row: enough for one chunk per lane when the row is short, capped at the wave. A longer row
    // takes, among the lane counts (64, 32, 16, 8) that still give the launch at least 1024 workgroups, the
    // one that leaves the fewest lanes idle in its last pass, the larger on a tie (4096 x 11008 Q4_0
    // grouped: 344 chunks are 43 passes of 8 lanes, against 6 passes of 64 with 40 lanes idle in the last);
    // fewer rows per wave pass mean more rows per workgroup, so a single matrix keeps 64.
    int lanes = 8;
    while (lanes < 64 && lanes < chunks) lanes <<= 1;
    const bool one_chunk = chunks <= lanes;
    const size_t lds = staged_lds_bytes<F>(padded);
    const bool wide = !one_chunk && lds > kWideLdsBytes && lds <= kMaxLdsBytes;
    const int64_t launched = static_cast<int64_t>(count) * s.positions;
    if (!one_chunk) {
        int64_t best = -1;
        for (int l = 64; l >= 8; l >>= 1) {
            const int64_t rows_per_iteration = (wide ? kWideThreads : kThreads) / 64 * (64 / l) * F::kRowUnroll;
            const int64_t workgroups = launched * ((s.rows_max + rows_per_iteration - 1) / rows_per_iteration);
            if (l < 64 && workgroups < 1024) continue;
            const int64_t slots = static_cast<int64_t>((chunks + l - 1) / l) * l;
            if (best < 0 || slots < best) {
                best = slots;
                lanes = l;
            }
        }
    }
    const int waves = (wide ? kWideThreads : kThreads) / 64;
    const int rows_per_pass = 64 / lanes;
    const int rows_per_iteration = waves * rows_per_pass * F::kRowUnroll;
    // Rows per workgroup: at least one full iteration; grow while the grid keeps >= 2048 workgroups
    // (8 per CU on 256 CUs), so small matrices still spread over the whole chip.
    const int64_t groups_total = launched;
    int rows_per_wg = rows_per_iteration;
    while (rows_per_wg < 1024 &&
           groups_total * ((s.rows_max + 2 * rows_per_wg - 1) / (2 * rows_per_wg)) >= 2048)
        rows_per_wg *= 2;
    if (F::kMaxWorkgroupPayload > 0)
        while (rows_per_wg > rows_per_iteration &&
               static_cast<int64_t>(rows_per_wg) * s.row_bytes > F::kMaxWorkgroupPayload)
            rows_per_wg /= 2;
    s.rows_per_wg = rows_per_wg;
    dim3 grid((s.rows_max + rows_per_wg - 1) / rows_per_wg, count, s.positions);
    switch (lanes) {
        case 8: return launch_lanes<F, 8>(one, group, s, grid, padded, one_chunk, wide, stream);
        case 16: return launch_lanes<F, 16>(one, group, s, grid, padded, one_chunk, wide, stream);
        case 32: return launch_lanes<F, 32>(one, group, s, grid, padded, one_chunk, wide, stream);
        default: return launch_lanes<F, 64>(one, group, s, grid, padded, one_chunk, wide, stream);
    }
}

}  // namespace

hipError_t launch_gemv_float(const MatDesc& one, const MatDesc* group, int count, LaunchShape s,
                             hipStream_t stream) {
    if (count <= 0 || s.rows_max <= 0 || s.positions <= 0) return hipSuccess;
    switch (s.format) {
        case kQ8_0: return launch_format<Q8_0Chunk>(one, group, count, s, s.blocks, s.columns, stream);
        case kQ4_0: return launch_format<Q4_0Chunk>(one, group, count, s, s.blocks, s.columns, stream);
        case kQ4_K: return launch_format<Q4_KChunk>(one, group, count, s, s.blocks * 8, s.columns, stream);
        case kQ6_K: return launch_format<Q6_KChunk>(one, group, count, s, s.blocks * 4, s.columns, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace satori
