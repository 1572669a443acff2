// Integer K-format product over many positions on the matrix cores (gfx950 int8 MFMA): the prefill form of
// ExecuteBatch (QuantizedMatVec.ExecuteBatchQuantized, src/Satori.Core/QuantizedMatVec.cs:136-219, whose
// per-position arithmetic is QuantizedKAvx2Kernel.ExecuteQuantizedTiled, QuantizedKAvx2Kernel.cs:47-99).
//
// Every integer the reference forms is formed exactly (int8 x int8 products summed in int32 by the MFMA,
// scaled by the 6-bit / int8 block scales in int32), and each block's FP32 term is the reference's
// expression, added to the (row, position) sum in block order from +0, so the outputs equal the
// single-position integer kernel's bit for bit.
//
// Two launches. The pack kernel quantizes every (position, block) to Q8_K (the same bytes as the reference
// quantizer) and stores the codes in the order the MFMA operands are read, with the block scales and the
// group sums (as FP16) in separate arrays; the product kernel stages each round's blocks in LDS.
//
// Product orientation: D = C x W^T with the positions' codes as the first operand (M = 32 positions) and the
// weights as the second (N = 32 rows). Lane l = 32h + r then holds the 16 outputs of row r at positions
// 8(i/4) + 4h + i%4 (i = 0..15), so the per-row block scales are lane-local. One wave owns one 32-row x
// 32-position tile and walks its blocks in order, loading block b+1 while it computes block b.
//
// Q4_K: Dot = sum_j s_j * D_j with D_j = sum over sub-block j (32 weights) of q * c: one 32x32x32 MFMA per
// sub-block and an int24 multiply-add by s_j (|D_j| <= 32 * 15 * 127 fits 24 bits, the sum 31); Min =
// sum_j m_j * (bsum_2j + bsum_2j+1) is one 32x32x16 FP16 product of the 16 group sums with m_(g/2), exact
// (operands of at most 11 significant bits, sums below 2^24). Q6_K reads its weights as two int8 planes of
// the pre-scaled, centred weight sc * (q - 32) (built once per matrix, below), so Dot is two 32x32x32 MFMA
// chains over the block's K steps and one combination, 128 hi + lo.
#include <type_traits>

#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "q8k_device.hpp"

namespace satori {
namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 32;      // rows and positions per wave tile

__device__ __forceinline__ i32x16 mfma32(const i32x4& c, const i32x4& w, const i32x16& acc) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(c, w, acc, 0, 0, 0);
}

__device__ __forceinline__ i32x16 mfma16(long c, long w, const i32x16& acc) {
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(c, w, acc, 0, 0, 0);
}

// One 32x32x16 FP16 product into FP32 (lane l holds k = 8 (l / 32) .. + 8 of row / column l % 32, the same
// output layout as the int8 products). Used for the block's group-sum terms, whose operands are integers of
// at most 11 significant bits (exact in FP16) and whose products and sums stay below 2^24, so the FP32
// result is the exact integer.
__device__ __forceinline__ f32x16 mfma_f16(const f16x8& a, const f16x8& b) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, f32x16{}, 0, 0, 0);
}

// Signed 24-bit multiply-add (v_mad_i32_i24): both factors must fit in 24 bits. The empty asm makes the
// result opaque to the optimizer, so each dot sum stays a sequential chain (the compiler would otherwise
// reassociate it into a tree of products that holds every MFMA result of the block in registers at once).
// It emits no instruction: the multiply-add itself is compiled code, so the compiler inserts the wait
// states a VALU read of an MFMA result needs.
__device__ __forceinline__ int mad24(int a, int b, int c) {
    int d = __mul24(a, b) + c;
    asm volatile("" : "+v"(d));
    return d;
}

// Packed activations. For block b and position tile t the 256 codes of the tile's 32 positions fill 8 KB
// at (b * tiles + t) * 8192, split into `chunks` chunks of 256 / chunks codes (8 for Q4_K: the 32x32x32
// operand, 16 for Q6_K: the 32x32x16 operand); chunk j's lane l = 32h + r holds the codes
// j * (256 / chunks) + h * (128 / chunks) .. + 128 / chunks of position 32t + r, at byte l * (128 / chunks).
// Scales: float at (b * tiles + t) * 32 + r. Group sums (the 16 Q8_K sums of 16 codes, |sum| <= 2032) as FP16
// in the first operand order of the 32x32x16 FP16 product: 1 KB per (block, tile), lane l = 32h + r holding
// sums 8h .. 8h + 7 of position 32t + r. Positions past the last are zero codes, sums and scale 0.
__device__ __forceinline__ int64_t pack_code_offset(int b, int t, int tiles, int chunks, int k, int r) {
    const int per = 256 / chunks, half = per / 2;
    const int j = k / per, h = (k % per) / half;
    return (static_cast<int64_t>(b) * tiles + t) * 8192 + j * (8192 / chunks) + (32 * h + r) * half + k % half;
}

// One wave per block and four consecutive positions, one 16-lane row per position (the 16-lane quantizer:
// lane j holds the block's group j, codes 16j .. 16j + 15, which land contiguous in the operand order and
// whose group sum needs no cross-lane step); four blocks per workgroup. Positions past the last are zero
// codes, sums and scale (computed on the last position's values, then cleared).
__global__ __launch_bounds__(256) void kmfma_pack_kernel(const float* __restrict__ x, int columns, int positions,
                                                         int tiles, int chunks, uint8_t* __restrict__ codes,
                                                         float* __restrict__ scales, _Float16* __restrict__ sums) {
    const int blocks = columns / 256;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= blocks) return;
    const int lane = threadIdx.x & 63;
    const int j = lane & 15;
    const int p = blockIdx.y * 4 + (lane >> 4);
    const int t = p >> 5, r = p & 31;
    const float* src = x + static_cast<int64_t>(min(p, positions - 1)) * columns + 256 * b + 16 * j;
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const u32x4 raw = load16_a4(reinterpret_cast<const uint8_t*>(src + 4 * q));
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * q + e] = __uint_as_float(raw[e]);
    }
    Q8KRow16 qr = q8k_quantize_row16(v, lane);
    if (p >= positions) {
#pragma unroll
        for (int w = 0; w < 4; ++w) qr.packed[w] = 0u;
        qr.group_sum = 0;
        qr.scale = 0.0f;
    }
    const int64_t bt = static_cast<int64_t>(b) * tiles + t;
    // Codes 16j .. 16j + 15 in pieces of 128 / chunks bytes (one 16-byte piece for Q4_K, two 8-byte for Q6_K).
    if (chunks == 8) {
        *reinterpret_cast<u32x4*>(codes + pack_code_offset(b, t, tiles, chunks, 16 * j, r)) =
            u32x4{qr.packed[0], qr.packed[1], qr.packed[2], qr.packed[3]};
    } else {
        *reinterpret_cast<uint2*>(codes + pack_code_offset(b, t, tiles, chunks, 16 * j, r)) =
            uint2{qr.packed[0], qr.packed[1]};
        *reinterpret_cast<uint2*>(codes + pack_code_offset(b, t, tiles, chunks, 16 * j + 8, r)) =
            uint2{qr.packed[2], qr.packed[3]};
    }
    sums[bt * 512 + (32 * (j >> 3) + r) * 8 + (j & 7)] = static_cast<_Float16>(static_cast<float>(qr.group_sum));
    if (j == 0) store_f32(scales + bt * 32 + r, qr.scale);
}

// A block's packed codes, group sums and scales staged in LDS: the 8 KB of codes in operand order, the 1 KB of
// FP16 group sums in operand order, then the tile's 32 position scales.
struct StagedBlock {
    uint8_t codes[8192];
    uint8_t sums[1024];
    float scales[32];
};

__device__ __forceinline__ f16x8 staged_sums(const StagedBlock& sb, int lane) {
    return *reinterpret_cast<const f16x8*>(sb.sums + 16 * lane);
}

__device__ __forceinline__ f32x4 staged_scales(const StagedBlock& sb, int q, int h) {
    return *reinterpret_cast<const f32x4*>(sb.scales + 8 * q + 4 * h);
}

__device__ __forceinline__ i32x4 staged_codes16(const StagedBlock& sb, int j, int lane) {
    return *reinterpret_cast<const i32x4*>(sb.codes + 1024 * j + 16 * lane);
}

// ---- Q4_K: the resident payload ----
// The weights one lane needs for one block: its row's data for its k half of every chunk.
struct Q4KRegs {
    u32x4 head;   // d, dmin, packed 6-bit scales and mins
    u32x4 qs[4];  // qs[32g + 16h, +16) for g = 0..3
};

__device__ __forceinline__ void load_weights(const uint8_t* wrow, int b, int h, Q4KRegs& r) {
    const uint8_t* block = wrow + static_cast<int64_t>(b) * 144;
    r.head = load16_a4(block);
#pragma unroll
    for (int g = 0; g < 4; ++g) r.qs[g] = load16_a4(block + 16 + 32 * g + 16 * h);
}

// The block's FP32 terms of the lane's 16 (row, position) outputs, from the staged codes. A zero activation
// block contributes +0 or -0 (the reference skips it, QuantizedKAvx2Kernel.cs:86): its scale is 0 and every
// resident block scale is finite (checked at upload), and adding a zero to a sum that starts at +0 never
// changes it, since such a sum is never -0. The sub-block (group) products are software-pipelined: the MFMA
// of sub-block j + 1 is issued before the results of j are scaled, and a scheduling barrier per step keeps
// the compiler from hoisting every MFMA of the block (which would hold all their result tiles in registers).
__device__ __forceinline__ i32x4 q4k_weights(const Q4KRegs& r, int j) {
    const u32x4 raw = r.qs[j >> 1];
    const int shift = 4 * (j & 1);
    return i32x4{static_cast<int>((raw[0] >> shift) & 0x0F0F0F0Fu), static_cast<int>((raw[1] >> shift) & 0x0F0F0F0Fu),
                 static_cast<int>((raw[2] >> shift) & 0x0F0F0F0Fu), static_cast<int>((raw[3] >> shift) & 0x0F0F0F0Fu)};
}

__device__ __forceinline__ void block_terms(const Q4KRegs& r, const StagedBlock& sb, int lane, float (&term)[16]) {
    const int h = lane >> 5;
    const float d = half_bits_to_float(r.head[0] & 0xFFFFu), dmin = half_bits_to_float(r.head[0] >> 16);
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q4k_scale_min(j, r.head, sc[j], mn[j]);
    int dot[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) dot[i] = 0;
    i32x16 cur = mfma32(staged_codes16(sb, 0, lane), q4k_weights(r, 0), i32x16{});
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        i32x16 next;
        if (j + 1 < 8) next = mfma32(staged_codes16(sb, j + 1, lane), q4k_weights(r, j + 1), i32x16{});
#pragma unroll
        for (int i = 0; i < 16; ++i) dot[i] = mad24(sc[j], cur[i], dot[i]);
        __builtin_amdgcn_sched_barrier(0);
        if (j + 1 < 8) cur = next;
    }
    // MinProduct = sum over the 16 group sums g of m_(g / 2) * sum_g: one FP16 product (|sum_g| <= 2032,
    // m <= 63, |total| < 2^21).
    f16x8 mw;
#pragma unroll
    for (int e = 0; e < 8; ++e) mw[e] = static_cast<_Float16>(static_cast<float>(h ? mn[4 + e / 2] : mn[e / 2]));
    const f32x16 mins = mfma_f16(staged_sums(sb, lane), mw);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f32x4 a4 = staged_scales(sb, q, h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            const float dA = __fmul_rn(d, a4[e]), dminA = __fmul_rn(dmin, a4[e]);
            // mins[i] is the exact integer MinProduct, i.e. its float conversion.
            term[i] = __fsub_rn(__fmul_rn(dA, static_cast<float>(dot[i])), __fmul_rn(dminA, mins[i]));
        }
    }
}

// ---- Q6_K: weight planes ----
// The Q6_K product reads each matrix's weights pre-scaled and centred (kmfma_planes_bytes): w = sc * (q - 32),
// sc the int8 scale of the weight's group of 16 and q its 6-bit code (-4064..4096), split exactly as
// w = 128 hi + lo with lo = w & 127 (0..127) and hi = (w - lo) / 128 (-32..32): two int8 planes. The block's
// integer product of the reference, Dot = sum_k sc_k (q_k - 32) c_k (Q6KCodec.DotProduct), is then
// 128 sum hi c + sum lo c, which the MFMA accumulates exactly over the block's eight K steps of 32
// (|128 sum hi c| <= 128 * 256 * 32 * 127, and the total, stay below 2^31): no group scale, code assembly
// or centring is left to the vector ALU (they took about 450 of its 574 instructions per 32 x 32 block tile
// on the resident layout). Q4_K keeps its payload: its planes (0..945 = 128 hi + lo) cost four times its
// bytes per weight in L2 traffic for little VALU saved, and measured slower (gate/up 30 -> 39 us).
//
// Record of row tile rt (32 rows; rows past the last are zero) and block b, at (rt * blocks + b) * 16,512:
//   [0, 16384)      plane p (0: hi, 1: lo), K step j (weights 32j .. 32j + 31): 1 KB in second-operand order,
//                   lane l = 32h + r holding the 16 bytes of row 32 rt + r, weights 32j + 16h .. + 15;
//   [16384, 16512)  per row r of the tile, d as a float (exact from FP16).
constexpr int kPlaneRecord = 16512;
constexpr int kPlaneScales = 16384;

// Q6_K weight k of block n of the regrouped device layout (count blocks in all) times its group scale, with
// the code centred: sc_(k/16) * (q_k - 32) (Q6KCodec.DecodeBlock's q1..q4 of half k / 128).
__device__ __forceinline__ int q6k_scaled_weight(const uint8_t* w, int64_t count, int64_t n, int k) {
    const int h = k >> 7, x = k & 127, kk = x >> 5, t = (x >> 4) & 1, i = x & 15;
    const uint8_t* quarter = w + n * 192 + 48 * (2 * h + t);
    const uint32_t ql = quarter[(kk & 1) * 16 + i];            // ql[64h + 16t + i] or ql[64h + 32 + 16t + i]
    const uint32_t low = kk >= 2 ? ql >> 4 : ql & 0xFu;
    const uint32_t high = (static_cast<uint32_t>(quarter[32 + i]) >> (2 * kk)) & 3u;  // qh[32h + 16t + i]
    const int q = static_cast<int>(low | (high << 4));
    const int sc = static_cast<int8_t>(w[count * 192 + n * 16 + 4 * (2 * h + t) + kk]);  // sc[8h + 2kk + t]
    return sc * (q - 32);
}

// One workgroup per (block, row tile) builds its record from the resident regrouped layout.
__global__ __launch_bounds__(256) void kmfma_planes_kernel(const uint8_t* __restrict__ w, int rows, int blocks,
                                                           uint8_t* __restrict__ planes) {
    const int b = blockIdx.x, rt = blockIdx.y;
    uint8_t* rec = planes + (static_cast<int64_t>(rt) * blocks + b) * kPlaneRecord;
    const int64_t count = static_cast<int64_t>(rows) * blocks;
    for (int item = threadIdx.x; item < 512; item += 256) {
        const int j = item >> 6, l = item & 63, r = l & 31, h = l >> 5;
        const int row = rt * kTile + r;
        uint32_t hi[4] = {0u, 0u, 0u, 0u}, lo[4] = {0u, 0u, 0u, 0u};
        if (row < rows) {
            for (int i = 0; i < 16; ++i) {
                const int v = q6k_scaled_weight(w, count, static_cast<int64_t>(row) * blocks + b, 32 * j + 16 * h + i);
                const int vlo = v & 127, vhi = (v - vlo) / 128;  // v = 128 vhi + vlo exactly
                lo[i >> 2] |= static_cast<uint32_t>(vlo) << (8 * (i & 3));
                hi[i >> 2] |= (static_cast<uint32_t>(vhi) & 0xFFu) << (8 * (i & 3));
            }
        }
        *reinterpret_cast<u32x4*>(rec + j * 1024 + 16 * l) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<u32x4*>(rec + (8 + j) * 1024 + 16 * l) = u32x4{lo[0], lo[1], lo[2], lo[3]};
    }
    if (threadIdx.x < kTile) {
        const int r = threadIdx.x, row = rt * kTile + r;
        float d = 0.0f;
        if (row < rows) {
            const uint8_t* dp = w + count * 208 + (static_cast<int64_t>(row) * blocks + b) * 2;
            d = half_bits_to_float(static_cast<uint32_t>(dp[0]) | (static_cast<uint32_t>(dp[1]) << 8));
        }
        *reinterpret_cast<float*>(rec + kPlaneScales + 4 * r) = d;
    }
}

// The planes one lane holds for one block, and its row's d.
struct PlaneRegs {
    i32x4 w[2][8];  // [plane][K step]
    float d;
};

__device__ __forceinline__ i32x4 load_plane(const uint8_t* rec, int p, int j, int lane) {
    return *(const SATORI_GLOBAL i32x4*)(rec + (8 * p + j) * 1024 + 16 * lane);
}

__device__ __forceinline__ float load_plane_d(const uint8_t* rec, int lane) {
    return __uint_as_float(load4_a4(rec + kPlaneScales + 4 * (lane & 31)));
}

__device__ __forceinline__ void load_planes(const uint8_t* rec, int lane, PlaneRegs& r) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        r.w[0][j] = load_plane(rec, 0, j, lane);
        r.w[1][j] = load_plane(rec, 1, j, lane);
    }
    r.d = load_plane_d(rec, lane);
}

// The block's FP32 terms (a d) Dot of the lane's 16 (row, position) outputs (QuantizedKAvx2Kernel.cs:94) from
// the staged codes, refilling each K step's plane registers with the next block's (record `next`) as soon as
// the step's two products have read them. A zero activation block contributes +0 or -0 (the reference skips
// it, QuantizedKAvx2Kernel.cs:86): its scale is 0, every resident block scale is finite (checked at upload),
// and adding a zero to a sum that starts at +0 never changes it.
__device__ __forceinline__ void block_terms(PlaneRegs& r, const uint8_t* next, const StagedBlock& sb, int lane,
                                            float (&term)[16]) {
    const int h = lane >> 5;
    i32x16 hi = {}, lo = {};
    // The next block's d is requested before its planes, so the wait for it at the end leaves them in flight.
    const float d = r.d;
    const float d_next = load_plane_d(next, lane);
    i32x4 c_next = staged_codes16(sb, 0, lane);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const i32x4 c = c_next;
        if (j + 1 < 8) c_next = staged_codes16(sb, j + 1, lane);  // read a step ahead
        hi = mfma32(c, r.w[0][j], hi);
        lo = mfma32(c, r.w[1][j], lo);
        r.w[0][j] = load_plane(next, 0, j, lane);
        r.w[1][j] = load_plane(next, 1, j, lane);
        __builtin_amdgcn_sched_barrier(0);  // the refill is issued here, ahead of its use
    }
    r.d = d_next;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f32x4 a4 = staged_scales(sb, q, h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            const float dot = static_cast<float>(hi[i] * 128 + lo[i]);  // the exact Dot, as the reference converts it
            term[i] = __fmul_rn(__fmul_rn(a4[e], d), dot);
        }
    }
}

// Blocks of one row tile are split over S waves ("ways"): way w computes blocks w, w + S, ... and, per round
// of S blocks, hands its 16 terms per lane to the others through LDS; the wave that owns an output adds the
// round's S terms in block order, so every (row, position) sum is formed exactly as the sequential one.
// A workgroup holds R = 4 / S row tiles x S ways of one position tile; the S blocks of a round are staged
// once in LDS for all of them: each thread loads its 32 S bytes of the next round's codes (and a few threads
// the scales) into registers while the current round is computed, and writes them to LDS after it.
template <int S>
struct Split {
    static constexpr int R = 4 / S;
    static constexpr int kOwned = 16 / S;  // outputs per lane each way adds up (whole quads)
};

// Workgroup u of the padded grid: consecutive units (row groups x position tiles, position tiles fastest)
// go to one XCD (workgroup ids are dealt to the 8 XCDs round-robin), so the position tiles that share a row
// group's weights share that XCD's L2.
template <int FORMAT, int S>
__global__ __launch_bounds__(256, S == 1 ? 3 : 2) void kmfma_kernel(KmfmaArgs a) {
    using SP = Split<S>;
    __shared__ StagedBlock stage[S];
    // Terms of one round: [row tile][way][quad q][lane] as float4 (conflict-free 16-byte accesses).
    __shared__ f32x4 exchange[S > 1 ? SP::R * S * 4 * 64 : 1];

    // Unit u of the launch (members one after the other, each (row group, position tile) with position tiles
    // fastest) -> member and unit within it.
    const int per_xcd = gridDim.x >> 3;
    int u = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    int mi = 0;
    while (mi + 1 < a.count && u >= a.units[mi]) u -= a.units[mi++];
    if (u >= a.units[mi]) return;  // whole workgroup
    const KmfmaMember& m = a.m[mi];
    const int rows = m.rows, blocks = a.blocks, tiles = a.tiles;
    const uint8_t* __restrict__ codes = m.workspace;
    const uint8_t* __restrict__ sums = m.workspace + kmfma_sums_offset(blocks, tiles);
    const float* __restrict__ scales = reinterpret_cast<const float*>(m.workspace + kmfma_scales_offset(blocks, tiles));
    float* __restrict__ y = m.y;
    const int positions = a.positions;
    const int group = u / tiles, t = u - group * tiles;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int way = wave % S, rt = wave / S;
    const int h = lane >> 5;
    const int row = (group * SP::R + rt) * kTile + (lane & 31);
    const int rounds = (blocks + S - 1) / S;

    // Staging of round k (blocks kS .. kS + S - 1): thread i holds bytes [16i, 16i + 16) and [4096 + 16i, +16)
    // of each block's codes (16-byte slices at a 16-byte stride: the LDS writes of a wave touch every bank once
    // per pass), bytes [4i, 4i + 4) of its group sums and, for i < 8 S, four scales.
    // With the weight planes (EXACT) every thread issues and stores the same bytes whatever k: blocks past the
    // last read (and store into their unused slots) the last block's bytes, and threads past the first 8 S
    // repeat thread i mod 8 S's scales. With no branch around them the compiler counts the loads in flight
    // exactly, and its waits leave the planes two blocks ahead in flight (below).
    constexpr bool EXACT = FORMAT == kQ6_K;
    u32x4 sc0[S], sc1[S];
    uint32_t ssum[S];
    u32x4 sscale = {0u, 0u, 0u, 0u};
    auto stage_load = [&](int k) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int b = EXACT ? min(k * S + s, blocks - 1) : k * S + s;
            if (EXACT || b < blocks) {
                const uint8_t* src = codes + (static_cast<int64_t>(b) * tiles + t) * 8192 + 16 * threadIdx.x;
                sc0[s] = load16_a4(src);
                sc1[s] = load16_a4(src + 4096);
                ssum[s] = load4_a4(sums + (static_cast<int64_t>(b) * tiles + t) * 1024 + 4 * threadIdx.x);
            }
        }
        const int q = EXACT ? static_cast<int>(threadIdx.x & (8 * S - 1)) : static_cast<int>(threadIdx.x);
        if (EXACT || q < 8 * S) {
            const int b = EXACT ? min(k * S + (q >> 3), blocks - 1) : k * S + (q >> 3);
            if (EXACT || b < blocks)
                sscale = load16_a4(
                    reinterpret_cast<const uint8_t*>(scales + (static_cast<int64_t>(b) * tiles + t) * 32 + 4 * (q & 7)));
        }
    };
    auto stage_store = [&](int k) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (EXACT || k * S + s < blocks) {
                *reinterpret_cast<u32x4*>(stage[s].codes + 16 * threadIdx.x) = sc0[s];
                *reinterpret_cast<u32x4*>(stage[s].codes + 4096 + 16 * threadIdx.x) = sc1[s];
                *reinterpret_cast<uint32_t*>(stage[s].sums + 4 * threadIdx.x) = ssum[s];
            }
        }
        const int q = EXACT ? static_cast<int>(threadIdx.x & (8 * S - 1)) : static_cast<int>(threadIdx.x);
        if (EXACT || q < 8 * S) *reinterpret_cast<u32x4*>(stage[q >> 3].scales + 4 * (q & 7)) = sscale;
    };

    // This way's accumulators: outputs way * kOwned + o of the lane (all 16 for S = 1), quads
    // q = way * (4 / S) + qq.
    float acc[SP::kOwned];
#pragma unroll
    for (int o = 0; o < SP::kOwned; ++o) acc[o] = 0.0f;

    // Adds one round's terms: directly for S = 1, else through the exchange buffer.
    auto add_round = [&](const float (&term)[16]) {
        if constexpr (S == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = __fadd_rn(acc[i], term[i]);
        } else {
            f32x4* buf = exchange + rt * (S * 4 * 64);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                buf[(way * 4 + q) * 64 + lane] = f32x4{term[4 * q], term[4 * q + 1], term[4 * q + 2], term[4 * q + 3]};
            __syncthreads();
            // The round's S terms of each owned output, added in block order. The next round's first barrier
            // orders these reads before the buffer is written again.
#pragma unroll
            for (int qq = 0; qq < 4 / S; ++qq) {
                const int q = way * (4 / S) + qq;
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) {
                    const f32x4 v = buf[(s2 * 4 + q) * 64 + lane];
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[4 * qq + e] = __fadd_rn(acc[4 * qq + e], v[e]);
                }
            }
        }
    };

    auto zero = [](float (&term)[16]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) term[i] = 0.0f;
    };
    if constexpr (FORMAT == kQ4_K) {
        // Round k: this way's block k S + way, from registers loaded one round ahead.
        const uint8_t* wrow = m.w + static_cast<int64_t>(row < rows ? row : rows - 1) * m.row_bytes;  // rows past
        auto load_w = [&](int b, Q4KRegs& r) {                                  // the last compute on a live row
            if (b < blocks) load_weights(wrow, b, h, r);
        };
        auto round = [&](int k, Q4KRegs& cur, Q4KRegs& nxt) {
            __syncthreads();  // the previous round's staged blocks (and exchanged terms) are no longer read
            stage_store(k);
            if (k + 1 < rounds) {
                stage_load(k + 1);
                load_w((k + 1) * S + way, nxt);
            }
            __syncthreads();  // round k staged
            const int b = k * S + way;
            float term[16];
            if (b < blocks)
                block_terms(cur, stage[way], lane, term);
            else
                zero(term);
            add_round(term);
        };
        Q4KRegs ra, rb;
        stage_load(0);
        load_w(way, ra);
        int k = 0;
        for (; k + 1 < rounds; k += 2) {
            round(k, ra, rb);
            round(k + 1, rb, ra);
        }
        if (k < rounds) round(k, ra, rb);
    } else {
        // The row tile's plane records (a tile past the last computes on the last one and stores nothing).
        // With two ways (two waves per SIMD, 256 VGPRs; launch_format caps the planes at two) two plane register
        // sets alternate: round k (this way's block k S + way) reads set k mod 2 and refills it with block
        // (k + 2) S + way while it runs, so each block's planes are requested two rounds ahead, after the next
        // round's codes (a wait for those leaves the planes in flight). One way (three workgroups per CU) keeps
        // one set, refilled a round ahead. Every round computes its block and stages the next round, past the
        // last ones too (their bytes are the last block's, and their terms are dropped), so every path issues the
        // same loads.
        constexpr bool kTwoAhead = S >= 2;
        const int row_tiles = (rows + kTile - 1) / kTile;
        const uint8_t* tile_rec =
            m.w + static_cast<int64_t>(min(group * SP::R + rt, row_tiles - 1)) * blocks * kPlaneRecord;
        auto rec = [&](int b) { return tile_rec + static_cast<int64_t>(min(b, blocks - 1)) * kPlaneRecord; };
        auto round = [&](int k, PlaneRegs& r) {
            __syncthreads();
            stage_store(k);
            stage_load(min(k + 1, rounds - 1));
            __syncthreads();
            const int b = k * S + way;
            float term[16];
            block_terms(r, rec(b + (kTwoAhead ? 2 : 1) * S), stage[way], lane, term);
            if (b >= blocks) zero(term);
            add_round(term);
        };
        PlaneRegs ra, rb;
        stage_load(0);
        load_planes(rec(way), lane, ra);
        if constexpr (kTwoAhead) {
            load_planes(rec(way + S), lane, rb);
            int k = 0;
            for (; k + 1 < rounds; k += 2) {
                round(k, ra);
                round(k + 1, rb);
            }
            if (k < rounds) round(k, ra);
        } else {
            for (int k = 0; k < rounds; ++k) round(k, ra);
        }
    }

    if (row >= rows) return;
#pragma unroll
    for (int o = 0; o < SP::kOwned; ++o) {
        const int i = way * SP::kOwned + o;
        const int p = t * kTile + 8 * (i >> 2) + 4 * h + (i & 3);
        if (p < positions) store_f32(y + static_cast<int64_t>(p) * rows + row, acc[o]);
    }
}

template <int FORMAT, int S>
void launch_split(KmfmaArgs& a, hipStream_t stream) {
    int total = 0;
    for (int i = 0; i < a.count; ++i) {
        const int groups = (a.m[i].rows + Split<S>::R * kTile - 1) / (Split<S>::R * kTile);
        a.units[i] = groups * a.tiles;
        total += a.units[i];
    }
    const int grid = (total + 7) / 8 * 8;
    kmfma_kernel<FORMAT, S><<<grid, 256, 0, stream>>>(a);
}

// Ways per row tile (1, 2 or 4): enough waves for about two per SIMD (2048), at most the block count, and no
// more ways than shorten the chain of rounds.
int choose_split(long wave_tiles, int blocks) {
    int s = 1;
    while (s < 4 && 2 * s <= blocks && wave_tiles * s < 2048) s *= 2;
    while (s > 1 && (blocks + s - 1) / s == (blocks + s / 2 - 1) / (s / 2)) s /= 2;
    return s;
}

template <int FORMAT>
void launch_format(KmfmaArgs& a, hipStream_t stream) {
    long wave_tiles = 0;
    for (int i = 0; i < a.count; ++i) wave_tiles += static_cast<long>((a.m[i].rows + kTile - 1) / kTile) * a.tiles;
    // Weight planes: at most two ways, whose 256-VGPR budget holds two plane sets (four ways would spill).
    const int split = choose_split(wave_tiles, a.blocks);
    switch (FORMAT == kQ6_K ? std::min(split, 2) : split) {
        case 1: launch_split<FORMAT, 1>(a, stream); break;
        case 2: launch_split<FORMAT, 2>(a, stream); break;
        default: launch_split<FORMAT, 4>(a, stream); break;
    }
}

}  // namespace

int kmfma_min_positions() { return 16; }

size_t kmfma_workspace_bytes(int blocks, int positions) {
    const int tiles = (positions + kTile - 1) / kTile;
    return kmfma_sums_offset(blocks, tiles) + static_cast<size_t>(blocks) * tiles * 1024;
}

hipError_t launch_kmfma_pack(int format, const float* x, int blocks, int positions, uint8_t* workspace,
                             hipStream_t stream) {
    if (positions <= 0 || blocks <= 0) return hipSuccess;
    if (format != kQ4_K && format != kQ6_K) return hipErrorInvalidValue;
    const int tiles = (positions + kTile - 1) / kTile;
    const int chunks = 8;  // K steps of 32 for both formats (the weight planes are pre-scaled)
    kmfma_pack_kernel<<<dim3((blocks + 3) / 4, tiles * kTile / 4), 256, 0, stream>>>(
        x, blocks * 256, positions, tiles, chunks, workspace,
        reinterpret_cast<float*>(workspace + kmfma_scales_offset(blocks, tiles)),
        reinterpret_cast<_Float16*>(workspace + kmfma_sums_offset(blocks, tiles)));
    return hipGetLastError();
}

hipError_t launch_kmfma_product(int format, const KmfmaMember* members, int count, int blocks, int positions,
                                hipStream_t stream) {
    if (count <= 0 || positions <= 0 || blocks <= 0) return hipSuccess;
    if (count > kKmfmaMaxMembers || (format != kQ4_K && format != kQ6_K)) return hipErrorInvalidValue;
    KmfmaArgs a{};
    for (int i = 0; i < count; ++i) {
        if (members[i].rows <= 0) return hipErrorInvalidValue;
        a.m[i] = members[i];
    }
    a.count = count;
    a.blocks = blocks;
    a.positions = positions;
    a.tiles = (positions + kTile - 1) / kTile;
    if (format == kQ4_K)
        launch_format<kQ4_K>(a, stream);
    else
        launch_format<kQ6_K>(a, stream);
    return hipGetLastError();
}

hipError_t launch_gemv_kmfma(const uint8_t* w, int format, const float* x, uint8_t* workspace, float* y, int rows,
                             int blocks, int64_t row_bytes, int positions, hipStream_t stream) {
    if (rows <= 0 || positions <= 0 || blocks <= 0) return hipSuccess;
    hipError_t e = launch_kmfma_pack(format, x, blocks, positions, workspace, stream);
    if (e != hipSuccess) return e;
    const KmfmaMember one{w, workspace, y, rows, 0, row_bytes};
    return launch_kmfma_product(format, &one, 1, blocks, positions, stream);
}

size_t kmfma_planes_bytes(int rows, int blocks) {
    return static_cast<size_t>((rows + kTile - 1) / kTile) * static_cast<size_t>(blocks) * kPlaneRecord;
}

hipError_t launch_kmfma_planes(const uint8_t* w, int rows, int blocks, uint8_t* planes, hipStream_t stream) {
    if (rows <= 0 || blocks <= 0) return hipSuccess;
    const int row_tiles = (rows + kTile - 1) / kTile;
    if (row_tiles > 65535) return hipErrorInvalidValue;  // grid y
    kmfma_planes_kernel<<<dim3(blocks, row_tiles), 256, 0, stream>>>(w, rows, blocks, planes);
    return hipGetLastError();
}

}  // namespace satori
