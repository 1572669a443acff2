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
    static constexpr int kSums = 0;
    struct Consts {};
    __device__ static Consts consts(int) { return Consts{}; }
    __device__ static void sums(const float (&)[kWeights], float (&)[1]) {}
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
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const float (&)[1], const Consts&) {
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
    static constexpr int kSums = 0;
    struct Consts {};
    __device__ static Consts consts(int) { return Consts{}; }
    __device__ static void sums(const float (&)[kWeights], float (&)[1]) {}
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
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const float (&)[1], const Consts&) {
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
// Chunk g of a block (g = 0..3) is qs[32g .. 32g + 32): the low nibbles are weights 64g + i of sub-block 2g,
// the high nibbles weights 64g + 32 + i of sub-block 2g + 1, so the chunk's 64 activations are contiguous.
// The chunk's dot is factored per sub-block: sum (d s q - dmin m) x = (d s) sum q x - (dmin m) sum x, so a
// weight costs one conversion and one FMA; the two sums of 32 activations are the same for every row and are
// computed once per workgroup (Sums). The high nibbles are used in place (the bytes 16 q) and the factor 16
// is removed with the power-of-two 1/16. A chunk's position g within its block is the same for all of a
// lane's chunks (g = chunk % 4, and a row's lanes step by a multiple of 4), so the scale and min fields a
// lane reads are fixed per lane (Consts).
// Non-finite activations: a product whose decoded weight is nonzero but whose code is 0 comes out NaN here
// where the reference's w * x gives +-Inf; the GGUF MatVec surface rejects non-finite inputs.
// ------------------------------------------------------------------------------------------------

struct Q4_KChunk {
    static constexpr int kRowUnroll = 1;
    static constexpr bool kPipelineShortLanes = false;
    static constexpr int kMaxWorkgroupPayload = 0;
    static constexpr int kWeights = 64;
    static constexpr int kPadShift = 6;
    static constexpr int kSums = 2;  // sum of the low-nibble sub-block's 32 activations, of the high one's
    struct Regs {
        u32x4 head;
        u32x4 qs0, qs1;
    };
    // Bit offsets of the 6-bit scale and min of sub-blocks 2g and 2g + 1 (GetScaleMin): for g < 2 they are
    // bytes 2g, 2g + 1 of scales[0..3] / scales[4..7]; for g >= 2 their low 4 bits are the nibbles of
    // scales[8 + 2(g - 2)], [9 + 2(g - 2)] and their high 2 bits the top bits of scales[2(g - 2)], ... .
    struct Consts {
        bool high;              // g >= 2: low bits from dword 3
        uint32_t scale_lo;      // offset of the scale's low 4 bits (in dword 1, or 3 when high)
        uint32_t min_lo;        // offset of the min's low 4 bits (in dword 2, or 3 when high)
        uint32_t top;           // offset of the 2 high bits (scale: dword 1, min: dword 2)
    };
    __device__ static Consts consts(int chunk) {
        const int g = chunk & 3;
        if (g < 2) return Consts{false, 16u * g, 16u * g, 16u * g + 4};
        const uint32_t o = 16u * (g - 2);
        return Consts{true, o, o + 4, o + 6};
    }
    __device__ static int chunks(const LaunchShape& s) { return s.blocks * 4; }
    __device__ static int padded_columns(const LaunchShape& s) { return s.columns; }
    using Row = const uint8_t*;  // the row's first block
    __device__ static Row row_ref(const MatDesc& m, const LaunchShape& s, int row) {
        return m.w + static_cast<int64_t>(row) * s.row_bytes;
    }
    __device__ static void load(Row w, int chunk, Regs& r) {
        const uint8_t* block = w + (chunk >> 2) * 144;
        r.head = load16_a4(block);
        r.qs0 = load16_a4(block + 16 + 32 * (chunk & 3));
        r.qs1 = load16_a4(block + 32 + 32 * (chunk & 3));
    }
    template <class XF>
    __device__ static void load_x(XF xf, int chunk, float (&x)[kWeights]) {
        const int base = (chunk >> 2) * 256 + 64 * (chunk & 3);
#pragma unroll
        for (int i = 0; i < kWeights; i += 4) xf.quad(base + i, x + i);
    }
    // The chunk's activation sums from its loaded activations (pairwise).
    __device__ static void sums(const float (&x)[kWeights], float (&out)[kSums]) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float t[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) t[i] = x[32 * half + i] + x[32 * half + 16 + i];
#pragma unroll
            for (int n = 8; n > 0; n >>= 1)
#pragma unroll
                for (int i = 0; i < n; ++i) t[i] += t[i + n];
            out[half] = t[0];
        }
    }
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const float (&xs)[kSums],
                                const Consts& k) {
        const float d = half_bits_to_float(r.head[0] & 0xFFFFu);
        const float dmin = half_bits_to_float(r.head[0] >> 16);
        const uint32_t ls = k.high ? r.head[3] : r.head[1], lm = k.high ? r.head[3] : r.head[2];
        const uint32_t s0 = __builtin_amdgcn_ubfe(ls, k.scale_lo, 4) | (__builtin_amdgcn_ubfe(r.head[1], k.top, 2) << 4);
        const uint32_t s1 = __builtin_amdgcn_ubfe(ls, k.scale_lo + 8, 4) |
                            (__builtin_amdgcn_ubfe(r.head[1], k.top + 8, 2) << 4);
        const uint32_t m0 = __builtin_amdgcn_ubfe(lm, k.min_lo, 4) | (__builtin_amdgcn_ubfe(r.head[2], k.top, 2) << 4);
        const uint32_t m1 = __builtin_amdgcn_ubfe(lm, k.min_lo + 8, 4) |
                            (__builtin_amdgcn_ubfe(r.head[2], k.top + 8, 2) << 4);
        float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t raw = w < 4 ? r.qs0[w] : r.qs1[w - 4];
            // Bytes q and bytes 16 q, each converted by one byte-select conversion: the empty asm keeps the
            // compiler from folding the mask into a bit-field extract per weight (two instructions a weight).
            uint32_t lo = raw & 0x0F0F0F0Fu, hi = raw & 0xF0F0F0F0u;
            asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                a0 = __builtin_fmaf(byte_to_float(lo, i), x[4 * w + i], a0);
                a1 = __builtin_fmaf(byte_to_float(lo, i + 1), x[4 * w + i + 1], a1);
                b0 = __builtin_fmaf(byte_to_float(hi, i), x[32 + 4 * w + i], b0);
                b1 = __builtin_fmaf(byte_to_float(hi, i + 1), x[32 + 4 * w + i + 1], b1);
            }
        }
        const float dl = d * static_cast<float>(s0), dh = (d * static_cast<float>(s1)) * 0.0625f;
        const float ml = dmin * static_cast<float>(m0), mh = dmin * static_cast<float>(m1);
        return __builtin_fmaf(dl, a0 + a1, __builtin_fmaf(dh, b0 + b1, -__builtin_fmaf(ml, xs[0], mh * xs[1])));
    }
};

// ------------------------------------------------------------------------------------------------
// Q6_K, FP32 activations (Q6KCodec.DotBlock, src/Satori.Core/Q6KCodec.cs:22-51): 210-byte super-block,
// ql[128] @0, qh[64] @128, int8 scales[16] @192, f16 d @208, read from the regrouped device layout
// (Q6KLayout). Chunk = quarter c = 2h + t of a block: l in [16t, 16t + 16) for all four k, i.e. weights
// 128h + 32k + l with scale 8h + 2k + t. Weight d * sc * (q - 32): the chunk's dot is sum over k of
// (d * sc_k / 4) * sum 4 (q - 32) x. Each code byte is assembled as the signed byte 4 (q - 32) (the 6-bit
// q ^ 32, i.e. q - 32 in 6-bit two's complement, in the byte's top six bits; the flip of q's bit 5 is one XOR
// on the high-bit dword for all four k), so a weight costs one signed-byte conversion and one FMA, exact
// products of the reference's integer (q - 32) with x up to the factor 4 removed with the scale.
// ------------------------------------------------------------------------------------------------
struct Q6_KChunk {
    static constexpr int kRowUnroll = 1;
    static constexpr bool kPipelineShortLanes = false;
    static constexpr int kMaxWorkgroupPayload = 0;
    static constexpr int kWeights = 64;
    static constexpr int kPadShift = 7;
    static constexpr int kSums = 0;
    using Regs = Q6KQuarter;
    struct Consts {};
    __device__ static Consts consts(int) { return Consts{}; }
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
    __device__ static void sums(const float (&)[kWeights], float (&)[1]) {}
    __device__ static float dot(const Regs& r, const float (&x)[kWeights], const float (&)[1], const Consts&) {
        float acc[4][2] = {};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t a = r.qla[w], b = r.qlb[w];
            const uint32_t h = r.qh[w] ^ 0xAAAAAAAAu;  // bit 1 of each 2-bit field (q's bit 5) flipped
            const uint32_t q[4] = {
                ((a << 2) & 0x3C3C3C3Cu) | ((h << 6) & 0xC0C0C0C0u),
                ((b << 2) & 0x3C3C3C3Cu) | ((h << 4) & 0xC0C0C0C0u),
                ((a >> 2) & 0x3C3C3C3Cu) | ((h << 2) & 0xC0C0C0C0u),
                ((b >> 2) & 0x3C3C3C3Cu) | (h & 0xC0C0C0C0u),
            };  // bytes 4 (q - 32)
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[k][i & 1] = __builtin_fmaf(sbyte_to_float(q[k], i), x[16 * k + 4 * w + i], acc[k][i & 1]);
        }
        const float d4 = q6k_d(r) * 0.25f;
        float total = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float s = static_cast<float>(static_cast<int8_t>(r.sc >> (8 * k)));  // scale 8h + 2k + t
            total = __builtin_fmaf(d4 * s, acc[k][0] + acc[k][1], total);
        }
        return total;
    }
};

// Floats of the staged activation copy (element i at i + 4 * (i >> PAD)), before the per-chunk sums.
template <class F>
__host__ __device__ inline int staged_floats(int padded) {
    return padded + 4 * (padded >> F::kPadShift) + 4;
}

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
    // Per-lane constants: a lane's chunks all sit at the same position within their block (L is a multiple of
    // the chunks per block, 8 or 4, or the row has a single pass).
    const typename F::Consts k = F::consts(lr);
    const int first = row_begin + wave * kRowsPerPass;  // wave-uniform

    // Formats that factor their dot need per-chunk sums of the activations (F::kSums per chunk): with staged
    // activations and several chunks per lane they are computed once per workgroup into a table after the
    // staged copy; otherwise from the loaded activations.
    constexpr int kS = F::kSums > 0 ? F::kSums : 1;
    constexpr bool kTable = !ONE && XLDS && F::kSums > 0;
    float* xsum_table = xs + staged_floats<F>(F::padded_columns(s));
    if constexpr (kTable) {
        for (int c = threadIdx.x; c < nchunks; c += THREADS) {
            float t[F::kWeights], o[kS];
            F::load_x(xf, c, t);
            F::sums(t, o);
#pragma unroll
            for (int j = 0; j < kS; ++j) xsum_table[kS * c + j] = o[j];
        }
        __syncthreads();
    }
    float xr[F::kWeights];
    float xsv[kS];
    // The activations of chunk c (and their sums).
    auto load_chunk = [&](int c) {
        F::load_x(xf, c, xr);
        if constexpr (kTable) {
#pragma unroll
            for (int j = 0; j < kS; ++j) xsv[j] = xsum_table[kS * c + j];
        } else if constexpr (F::kSums > 0) {
            F::sums(xr, xsv);
        }
    };
    if constexpr (ONE) {
        // Each lane owns one chunk of every row: its activations stay in registers, and the next
        // iteration's rows are loaded while the current ones are computed.
        const bool active = lr < nchunks;
        if (active) {
            load_chunk(lr);
        } else {
#pragma unroll
            for (int j = 0; j < F::kWeights; ++j) xr[j] = 0.0f;
#pragma unroll
            for (int j = 0; j < kS; ++j) xsv[j] = 0.0f;
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
                const float partial = (active && row < row_end) ? F::dot(cur[u], xr, xsv, k) : 0.0f;
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
                    load_chunk(cc);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) acc[u] += F::dot(r0[u], xr, xsv, k);
                    load_chunk(cc + L);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) acc[u] += F::dot(r1[u], xr, xsv, k);
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
                    load_chunk(c);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) {
                        const int row = base + u * kStride + sub;
                        if (row < row_end) acc[u] += F::dot(ra[u], xr, xsv, k);
                    }
                    load_chunk(c + L);
#pragma unroll
                    for (int u = 0; u < kRowUnroll; ++u) {
                        const int row = base + u * kStride + sub;
                        if (row < row_end) acc[u] += F::dot(rb[u], xr, xsv, k);
                    }
                }
            }
            for (; c < nchunks; c += L) {
                load_chunk(c);
                typename F::Regs regs[kRowUnroll];
#pragma unroll
                for (int u = 0; u < kRowUnroll; ++u) {
                    const int row = base + u * kStride + sub;
                    if (row < row_end) F::load(rows[u], c, regs[u]);
                }
#pragma unroll
                for (int u = 0; u < kRowUnroll; ++u) {
                    const int row = base + u * kStride + sub;
                    if (row < row_end) acc[u] += F::dot(regs[u], xr, xsv, k);
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

// LDS budget for the staged activations and their per-chunk sums.
constexpr int kMaxLdsBytes = 64 * 1024;

template <class F>
size_t staged_lds_bytes(int padded, int chunks) {
    return static_cast<size_t>(staged_floats<F>(padded) + chunks * F::kSums) * sizeof(float);
}

template <class F, int L, bool ONE, int THREADS>
hipError_t launch_variant(const MatDesc& one, const MatDesc* group, const LaunchShape& s, dim3 grid, int padded,
                          int chunks, hipStream_t stream) {
    const size_t lds = staged_lds_bytes<F>(padded, chunks);
    if (lds <= kMaxLdsBytes)
        gemv_float_kernel<F, L, ONE, true, THREADS><<<grid, THREADS, lds, stream>>>(one, group, s);
    else
        gemv_float_kernel<F, L, ONE, false, THREADS><<<grid, THREADS, 0, stream>>>(one, group, s);
    return hipGetLastError();
}

template <class F, int L>
hipError_t launch_lanes(const MatDesc& one, const MatDesc* group, const LaunchShape& s, dim3 grid, int padded,
                        int chunks, bool one_chunk, bool wide, hipStream_t stream) {
    if (one_chunk) return launch_variant<F, L, true, kThreads>(one, group, s, grid, padded, chunks, stream);
    if (wide) return launch_variant<F, L, false, kWideThreads>(one, group, s, grid, padded, chunks, stream);
    return launch_variant<F, L, false, kThreads>(one, group, s, grid, padded, chunks, stream);
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
    const bool one_chunk = chunks <= lanes && chunks * 8 >= lanes * 7;
    const size_t lds = staged_lds_bytes<F>(padded, chunks);
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
        case 8: return launch_lanes<F, 8>(one, group, s, grid, padded, chunks, one_chunk, wide, stream);
        case 16: return launch_lanes<F, 16>(one, group, s, grid, padded, chunks, one_chunk, wide, stream);
        case 32: return launch_lanes<F, 32>(one, group, s, grid, padded, chunks, one_chunk, wide, stream);
        default: return launch_lanes<F, 64>(one, group, s, grid, padded, chunks, one_chunk, wide, stream);
    }
}

}  // namespace

hipError_t launch_gemv_float(const MatDesc& one, const MatDesc* group, int count, LaunchShape s,
                             hipStream_t stream) {
    if (count <= 0 || s.rows_max <= 0 || s.positions <= 0) return hipSuccess;
    switch (s.format) {
        case kQ8_0: return launch_format<Q8_0Chunk>(one, group, count, s, s.blocks, s.columns, stream);
        case kQ4_0: return launch_format<Q4_0Chunk>(one, group, count, s, s.blocks, s.columns, stream);
        case kQ4_K: return launch_format<Q4_KChunk>(one, group, count, s, s.blocks * 4, s.columns, stream);
        case kQ6_K: return launch_format<Q6_KChunk>(one, group, count, s, s.blocks * 4, s.columns, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace satori
