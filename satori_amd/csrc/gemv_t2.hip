// Ternary2 MatVec by pair tables (gfx950) on the panel layout.
//
// Each lane owns one row of a 64-row panel, so a wave's loads of one 64-column chunk are 1 KB contiguous
// (the panel layout is described with T2Layout). The activation slice of a workgroup is staged in LDS and
// the row is walked in tiles of 128 columns. For every tile the workgroup builds, in LDS, one 16-entry
// table per column pair (c0, c1):
//     T[p][c0 + 4 c1] = v(c0) * x[2p] + v(c1) * x[2p + 1],   v(0) = v(3) = 0, v(1) = +1, v(2) = -1,
// where c0, c1 are the 2-bit codes of the pair (docs/ternary2-v1.md; Ternary2MatVec.ExecuteScalarCore,
// src/Satori.Core/Ternary2MatVec.cs:52-76). A code nibble is then exactly the table index, so two weights
// cost one byte extraction, one LDS read and one FP32 add. All lanes of a wave read the same pair table at
// a time and a table spans 16 consecutive dwords, so the reads never conflict on LDS banks. Tables are
// double-buffered: the tables of tile t + 1 are built while tile t is consumed, one barrier per tile.
//
// Block sums are multiplied by the block scale and added to the row sum in block order, as the reference
// does; only the order of the FP32 additions inside a block differs (pair sums first). When rows alone
// cannot fill the chip the columns are split over workgroups: each split stores its row sums in a scratch
// buffer and a second kernel adds them in split order, so results do not depend on scheduling. (Letting
// the last-arriving workgroup add them needs device-scope release/acquire fences per workgroup, which on
// gfx950 write back and invalidate the L2 and cost more than the second launch.)
#include <algorithm>
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = kT2TileColumns;
constexpr int kPairs = kTile / 2;        // pair tables per tile
constexpr int kTableFloats = kPairs * 16;
constexpr int kLdsLimit = 64 * 1024;
// Tiles one workgroup stages: 64 KB less the tables, rounded down to an even count (B = 256 splits hold
// whole blocks): 112 tiles = 14,336 columns.
constexpr int kMaxTilesPerSplit = ((kLdsLimit - 2 * kTableFloats * 4) / (kTile * 4)) & ~1;
constexpr int kTargetWorkgroups = 1024;  // four per CU

struct T2Args {
    int columns;
    int tiles;
    int chunks;
    int slots;
    int splits;
    int tiles_per_split;
    int count;
    int rows_pad;     // partial stride: panels of the tallest member * 64
    float* partials;  // [positions][count][splits][rows_pad] when splits > 1
};

// Builds the 64 pair tables of local tile u into buffer BUF: thread k writes entry k & 15 of pairs
// k / 16 + 16 i. v(c0) x0 + v(c1) x1 is formed as fma(v1, x1, v0 * x0): both products are exact, so the
// entry is the correctly rounded pair sum (a zero entry may be -0, which adds like +0 to sums that start
// at +0).
template <int BUF>
__device__ __forceinline__ void build_tables(float (*tables)[kTableFloats], const float* xs, int u) {
    const int e = threadIdx.x & 15;
    const int c0 = e & 3, c1 = e >> 2;
    const float v0 = c0 == 1 ? 1.0f : (c0 == 2 ? -1.0f : 0.0f);
    const float v1 = c1 == 1 ? 1.0f : (c1 == 2 ? -1.0f : 0.0f);
#pragma unroll
    for (int k = 0; k < kTableFloats / kThreads; ++k) {
        const int pair = (threadIdx.x >> 4) + k * (kThreads / 16);
        const float2 xp = *reinterpret_cast<const float2*>(xs + kTile * u + 2 * pair);
        tables[BUF][pair * 16 + e] = __builtin_fmaf(v1, xp.y, v0 * xp.x);
    }
}

// Sum over the 32 pairs of one 16-byte code chunk (pairs [P0, P0 + 32) of the tile) with buffer BUF's
// tables. Byte k of `lo` is 4 * (low nibble of code byte k) and of `hi` 4 * (high nibble): the byte
// address inside the pair's table; the table's own position is an immediate offset of the LDS read.
template <int BUF, int P0>
__device__ __forceinline__ float chunk_sum(const u32x4& codes, const float (*tables)[kTableFloats]) {
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t lo = (codes[d] << 2) & 0x3C3C3C3Cu;
        const uint32_t hi = (codes[d] >> 2) & 0x3C3C3C3Cu;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int pair = P0 + 8 * d + 2 * k;
            const uint32_t a = __builtin_amdgcn_perm(0u, lo, 0x0C0C0C00u | k);
            const uint32_t b = __builtin_amdgcn_perm(0u, hi, 0x0C0C0C00u | k);
            const char* table = reinterpret_cast<const char*>(&tables[BUF][pair * 16]);
            s0 += *reinterpret_cast<const float*>(table + a);
            s1 += *reinterpret_cast<const float*>(table + 64 + b);
        }
    }
    return s0 + s1;
}

// The two code chunks and the scales one lane needs for one tile.
struct TileData {
    u32x4 c0, c1;  // columns [0, 64) and [64, 128) of the tile
    float s0, s1;  // block scale(s): B = 64 uses both, B = 128 and 256 only s0
};

template <int B>
__device__ __forceinline__ void load_tile(const uint8_t* codes, const uint8_t* scales, int u, int t, TileData& d) {
    d.c0 = stream16(codes + (2 * u) * 1024);
    d.c1 = stream16(codes + (2 * u + 1) * 1024);
    if constexpr (B == 64) {
        d.s0 = __uint_as_float(stream4(scales + (2 * t) * 256));
        d.s1 = __uint_as_float(stream4(scales + (2 * t + 1) * 256));
    } else if constexpr (B == 128) {
        d.s0 = __uint_as_float(stream4(scales + t * 256));
        d.s1 = 0.0f;
    } else {
        d.s0 = __uint_as_float(stream4(scales + (t >> 1) * 256));
        d.s1 = 0.0f;
    }
}

template <int B, int R>
__global__ __launch_bounds__(kThreads) void t2_kernel(MatDesc one, const MatDesc* __restrict__ group, T2Args a) {
    const MatDesc m = group ? group[blockIdx.y] : one;
    const int split = blockIdx.x % a.splits;
    const int panel0 = (blockIdx.x / a.splits) * (kWaves * R);
    const int panels = (m.rows + kT2PanelRows - 1) / kT2PanelRows;
    if (panel0 >= panels) return;  // the whole workgroup leaves together
    const int t0 = split * a.tiles_per_split;
    const int nt = min(a.tiles_per_split, a.tiles - t0);
    const int position = blockIdx.z;
    const float* x = m.x + static_cast<int64_t>(position) * a.columns + t0 * kTile;
    const int available = a.columns - t0 * kTile;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t codes_bytes = static_cast<int64_t>(panels) * a.chunks * 1024;
    const uint8_t* codes[R];
    const uint8_t* scales[R];
    int row[R];
    bool live[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int p = panel0 + wave * R + j;
        live[j] = p < panels;
        const int64_t q = live[j] ? p : panel0;  // dead panels read a live one and store nothing
        row[j] = p * kT2PanelRows + lane;
        codes[j] = m.w + (q * a.chunks + 2 * t0) * 1024 + lane * 16;
        scales[j] = m.w + codes_bytes + q * a.slots * 256 + lane * 4;
    }
    TileData cur[R], nxt[R];
#pragma unroll
    for (int j = 0; j < R; ++j) load_tile<B>(codes[j], scales[j], 0, t0, cur[j]);  // in flight while x is staged

    __shared__ float tables[2][kTableFloats];  // static, so every table read has a constant base
    extern __shared__ float xs[];              // nt * 128 activations of this split, zero past the last column
    for (int i = threadIdx.x; i < nt * kTile; i += kThreads) xs[i] = i < available ? load_f32(x + i) : 0.0f;
    __syncthreads();
    build_tables<0>(tables, xs, 0);
    float acc[R], part[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = part[j] = 0.0f;
    __syncthreads();  // tables of the first tile complete

    // Local tile u uses buffer u & 1; the loop body handles an even and an odd tile so that both buffers'
    // positions are compile-time constants.
    auto tile = [&](auto buffer_tag, int u) {
        constexpr int BUF = decltype(buffer_tag)::value;
        if (u + 1 < nt) {
            build_tables<1 - BUF>(tables, xs, u + 1);
#pragma unroll
            for (int j = 0; j < R; ++j) load_tile<B>(codes[j], scales[j], u + 1, t0 + u + 1, nxt[j]);
        }
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const float lo = chunk_sum<BUF, 0>(cur[j].c0, tables);
            const float hi = chunk_sum<BUF, 32>(cur[j].c1, tables);
            if constexpr (B == 64) {
                acc[j] += lo * cur[j].s0;  // block 2t
                acc[j] += hi * cur[j].s1;  // block 2t + 1 (zero codes and scale in the padding slot)
            } else if constexpr (B == 128) {
                acc[j] += (lo + hi) * cur[j].s0;
            } else {
                part[j] += lo + hi;
                if (u & 1) {  // second half of the block (splits start on even tiles)
                    acc[j] += part[j] * cur[j].s0;
                    part[j] = 0.0f;
                }
            }
            cur[j] = nxt[j];
        }
        __syncthreads();  // next tables built; this tile's tables no longer read
    };
    for (int u = 0; u < nt; u += 2) {
        tile(std::integral_constant<int, 0>{}, u);
        if (u + 1 < nt) tile(std::integral_constant<int, 1>{}, u + 1);
    }

    float* y = m.y + static_cast<int64_t>(position) * m.rows;
    if (a.splits == 1) {
#pragma unroll
        for (int j = 0; j < R; ++j)
            if (live[j] && row[j] < m.rows) store_f32(y + row[j], acc[j]);
        return;
    }

    const int64_t slab = (static_cast<int64_t>(position) * a.count + blockIdx.y) * a.splits + split;
#pragma unroll
    for (int j = 0; j < R; ++j)
        if (live[j] && row[j] < m.rows) store_f32(a.partials + slab * a.rows_pad + row[j], acc[j]);
}

// y[row] = sum of the splits' row sums in split order from +0; loads are issued eight at a time.
__global__ __launch_bounds__(kThreads) void t2_reduce_kernel(MatDesc one, const MatDesc* __restrict__ group,
                                                              T2Args a) {
    const MatDesc m = group ? group[blockIdx.y] : one;
    const int row = blockIdx.x * kThreads + threadIdx.x;
    if (row >= m.rows) return;
    const float* p =
        a.partials + (static_cast<int64_t>(blockIdx.z) * a.count + blockIdx.y) * a.splits * a.rows_pad + row;
    float sum = 0.0f;
    int s = 0;
    for (; s + 8 <= a.splits; s += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = load_f32(p + static_cast<int64_t>(s + k) * a.rows_pad);
#pragma unroll
        for (int k = 0; k < 8; ++k) sum += v[k];
    }
    for (; s < a.splits; ++s) sum += load_f32(p + static_cast<int64_t>(s) * a.rows_pad);
    store_f32(m.y + static_cast<int64_t>(blockIdx.z) * m.rows + row, sum);
}

template <int B, int R>
hipError_t launch(const MatDesc& one, const MatDesc* group, dim3 grid, size_t lds, const T2Args& a,
                  hipStream_t stream) {
    t2_kernel<B, R><<<grid, kThreads, lds, stream>>>(one, group, a);
    return hipGetLastError();
}

}  // namespace

T2Plan t2_plan(int rows_max, int columns, int block_size, int count, int positions) {
    const T2Layout l = t2_layout(rows_max, columns, block_size);
    const int64_t members = static_cast<int64_t>(count) * positions;
    T2Plan p{1, 1, l.tiles};
    if (members * ((l.panels + 2 * kWaves - 1) / (2 * kWaves)) >= kTargetWorkgroups) p.panels_per_wave = 2;
    const int64_t groups = members * ((l.panels + kWaves * p.panels_per_wave - 1) / (kWaves * p.panels_per_wave));
    int tps = std::min(l.tiles, kMaxTilesPerSplit);
    // Split the columns while the grid is small, keeping at least two tiles per split.
    while (groups * ((l.tiles + tps - 1) / tps) < kTargetWorkgroups && tps >= 4) tps = (tps + 1) / 2;
    if (block_size == 256) tps += tps & 1;  // B = 256 blocks span two tiles: splits end on block boundaries
    p.tiles_per_split = tps;
    p.splits = (l.tiles + tps - 1) / tps;
    return p;
}

size_t t2_scratch_bytes(const T2Plan& plan, int rows_max, int count, int positions) {
    if (plan.splits <= 1) return 0;
    const size_t rows_pad = static_cast<size_t>((rows_max + kT2PanelRows - 1) / kT2PanelRows) * kT2PanelRows;
    return static_cast<size_t>(positions) * count * plan.splits * rows_pad * sizeof(float);
}

hipError_t launch_t2(const MatDesc& one, const MatDesc* group, int count, LaunchShape s, const T2Plan& plan,
                     void* scratch, hipStream_t stream) {
    if (count <= 0 || s.rows_max <= 0 || s.positions <= 0) return hipSuccess;
    const T2Layout l = t2_layout(s.rows_max, s.columns, s.block_size);
    const int R = plan.panels_per_wave;
    if ((R != 1 && R != 2) || plan.splits < 1 || plan.tiles_per_split < 1 ||
        plan.tiles_per_split > kMaxTilesPerSplit || static_cast<int64_t>(plan.splits) * plan.tiles_per_split < l.tiles ||
        (plan.splits - 1) * plan.tiles_per_split >= l.tiles || (s.block_size == 256 && (plan.tiles_per_split & 1)) ||
        (plan.splits > 1 && scratch == nullptr))
        return hipErrorInvalidValue;
    const int groups = (l.panels + kWaves * R - 1) / (kWaves * R);
    const T2Args a{s.columns, l.tiles, l.chunks, l.slots, plan.splits, plan.tiles_per_split, count,
                   l.panels * kT2PanelRows, static_cast<float*>(scratch)};
    const dim3 grid(static_cast<unsigned>(groups * plan.splits), static_cast<unsigned>(count),
                    static_cast<unsigned>(s.positions));
    const size_t lds = static_cast<size_t>(plan.tiles_per_split) * kTile * sizeof(float);
    hipError_t e;
    switch (s.block_size * 4 + R) {
        case 64 * 4 + 1: e = launch<64, 1>(one, group, grid, lds, a, stream); break;
        case 64 * 4 + 2: e = launch<64, 2>(one, group, grid, lds, a, stream); break;
        case 128 * 4 + 1: e = launch<128, 1>(one, group, grid, lds, a, stream); break;
        case 128 * 4 + 2: e = launch<128, 2>(one, group, grid, lds, a, stream); break;
        case 256 * 4 + 1: e = launch<256, 1>(one, group, grid, lds, a, stream); break;
        case 256 * 4 + 2: e = launch<256, 2>(one, group, grid, lds, a, stream); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || plan.splits == 1) return e;
    const dim3 reduce_grid(static_cast<unsigned>((s.rows_max + kThreads - 1) / kThreads),
                           static_cast<unsigned>(count), static_cast<unsigned>(s.positions));
    t2_reduce_kernel<<<reduce_grid, kThreads, 0, stream>>>(one, group, a);
    return hipGetLastError();
}

}  // namespace satori
