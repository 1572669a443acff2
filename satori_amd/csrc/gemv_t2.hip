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
// does; only the order of the FP32 additions inside a block differs (pair sums first).
//
// Work is balanced stream-K style: an item is the `W` panels of one member that one workgroup covers, a
// launch is items x tiles units of work, and a fixed number of workgroups (what the CUs hold at once) each
// take an equal contiguous range of units. A range covers whole items, written straight to y, plus at
// most a partial item at each end, whose row sums go to a per-workgroup scratch slot; a second, small
// kernel adds the pieces of every split item in range order, so results do not depend on scheduling.
// The range starts and the list of split items depend only on the plan: the host computes them once and
// they sit at the start of the plan's scratch buffer.
// (Letting the last workgroup of an item add them itself needs device-scope release/acquire fences per
// workgroup, which on gfx950 write back and invalidate the L2 and cost more than the second launch.)
// A single matrix at one position whose workgroups all fit on the chip at once runs instead one kernel,
// t2_slice_kernel below, whose column slices meet through atomic exchanges (no fences, no second launch).
#include <algorithm>
#include <cstring>
#include <type_traits>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

constexpr int kTile = kT2TileColumns;
constexpr int kPairs = kTile / 2;        // pair tables per tile
constexpr int kTableFloats = kPairs * 16;
constexpr int kLdsLimit = 64 * 1024;
// Tiles of activations one workgroup stages at a time: 64 KB less the tables, rounded down to an even
// count (B = 256 ranges hold whole blocks): 112 tiles = 14,336 columns.
constexpr int kMaxStagedTiles = ((kLdsLimit - 2 * kTableFloats * 4) / (kTile * 4)) & ~1;

struct T2Args {
    int columns;
    int tiles;
    int chunks;
    int slots;
    int count;                 // members per position
    int groups;                // items per member: panel groups of the tallest member
    const int* starts;         // [P + 1] first tile of each range (item-major tile order)
    const T2Fixup* fixups;     // items cut between ranges
    float* partials;           // [P][2][64 * W]: a workgroup's first and last piece of a cut item
};

// Builds the 64 pair tables of local tile u into buffer BUF: thread k writes entry k & 15 of pairs
// k / 16 + 16 i. v(c0) x0 + v(c1) x1 is formed as sel(c0, x0) + sel(c1, x1) with sel(1, x) = x,
// sel(2, x) = -x and sel(0, x) = sel(3, x) = +0, so the entry is the correctly rounded pair sum, and a
// code-0 weight contributes nothing even when its activation is infinite or NaN, as the reference skips it
// (Ternary2MatVec.cs:64-70). A zero entry may be -0, which adds like +0 to sums that start at +0.
template <int BUF, int THREADS>
__device__ __forceinline__ void build_tables(float (*tables)[kTableFloats], const float* xs, int u) {
    const int e = threadIdx.x & 15;
    const int c0 = e & 3, c1 = e >> 2;
#pragma unroll
    for (int k = 0; k < kTableFloats / THREADS; ++k) {
        const int pair = (threadIdx.x >> 4) + k * (THREADS / 16);
        const float2 xp = *reinterpret_cast<const float2*>(xs + kTile * u + 2 * pair);
        const float a = c0 == 1 ? xp.x : (c0 == 2 ? -xp.x : 0.0f);
        const float b = c1 == 1 ? xp.y : (c1 == 2 ? -xp.y : 0.0f);
        tables[BUF][pair * 16 + e] = a + b;
    }
}

// Sum over the 32 pairs of one 16-byte code record (pairs [P0, P0 + 32) of the tile) with buffer BUF's
// tables. The record is stored rotated left by 2 bits (T2Layout), so bits 2-5 of every byte hold the low
// nibble of the original byte: `lo` = record & 0x3C3C3C3C gives 4 * (low nibble) per byte, and shifting
// the record right by 4 bits (dword pairs joined by v_alignbit, the last with the first) brings the high
// nibble to the same place. Each byte is then the byte address inside its pair's table; the table's own
// position is an immediate offset of the LDS read. The sums start from the first lookup (no add to +0:
// an entry of -0 then starts a sum at -0, which the +0-started row sum absorbs).
template <int BUF, int P0>
__device__ __forceinline__ float chunk_sum(const u32x4& record, const float (*tables)[kTableFloats]) {
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t lo = record[d] & 0x3C3C3C3Cu;
        const uint32_t hi = __builtin_amdgcn_alignbit(record[(d + 1) & 3], record[d], 4) & 0x3C3C3C3Cu;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int pair = P0 + 8 * d + 2 * k;
            const uint32_t a = __builtin_amdgcn_perm(0u, lo, 0x0C0C0C00u | k);
            const uint32_t b = __builtin_amdgcn_perm(0u, hi, 0x0C0C0C00u | k);
            const char* table = reinterpret_cast<const char*>(&tables[BUF][pair * 16]);
            const float ta = *reinterpret_cast<const float*>(table + a);
            const float tb = *reinterpret_cast<const float*>(table + 64 + b);
            if (d == 0 && k == 0) {
                s0 = ta;
                s1 = tb;
            } else {
                s0 += ta;
                s1 += tb;
            }
        }
    }
    return s0 + s1;
}

// The two code chunks and the scales one lane needs for one tile.
struct TileData {
    u32x4 c0, c1;  // columns [0, 64) and [64, 128) of the tile
    float s0, s1;  // block scale(s): B = 64 uses both, B = 128 and 256 only s0
};

// B = 256 blocks span two tiles; their scale is loaded with the second (odd) tile only, where it is used.
template <int B, bool ODD>
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
        d.s0 = ODD ? __uint_as_float(stream4(scales + (t >> 1) * 256)) : 0.0f;
        d.s1 = 0.0f;
    }
}

template <int B, int W>
__global__ __launch_bounds__(64 * W) void t2_kernel(MatDesc one, const MatDesc* __restrict__ group, T2Args a) {
    constexpr int kThreadsW = 64 * W;
    __shared__ float tables[2][kTableFloats];  // static, so every table read has a constant base
    extern __shared__ float xs[];              // activations of the current segment, zero past the last column
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int begin = a.starts[blockIdx.x], end = a.starts[blockIdx.x + 1];
    // Item of the first tile, as (panel group, member, position); later segments step through items.
    const int first_item = begin / a.tiles;
    int t0 = begin - first_item * a.tiles;
    int item_group = first_item % a.groups;
    int member = (first_item / a.groups) % a.count;
    int position = first_item / a.groups / a.count;

    for (int u = begin; u < end;) {
        // Segment: tiles [t0, t0 + nt) of one item. Every decision below is uniform over the workgroup.
        const int nt = min(a.tiles - t0, end - u);
        const int slot = u == begin ? 0 : 1;
        const MatDesc m = group ? group[member] : one;
        const int panels = (m.rows + kT2PanelRows - 1) / kT2PanelRows;
        const int panel0 = item_group * W;
        if (panel0 < panels) {  // else a shorter member of the group: nothing to do
            // Wave w owns panel panel0 + w, one row per lane; a wave past the last panel reads panel0 and
            // stores nothing.
            const int panel = panel0 + wave;
            const bool live = panel < panels;
            const int row = panel * kT2PanelRows + lane;
            const int64_t q = live ? panel : panel0;
            const uint8_t* codes = m.w + (q * a.chunks + 2 * t0) * 1024 + lane * 16;
            const uint8_t* scales =
                m.w + static_cast<int64_t>(panels) * a.chunks * 1024 + q * a.slots * 256 + lane * 4;

            // Two register sets alternate: the loads of tile v + 1 are issued while tile v is summed.
            TileData even, odd;
            load_tile<B, false>(codes, scales, 0, t0, even);  // in flight while x is staged

            const float* x = m.x + static_cast<int64_t>(position) * a.columns + t0 * kTile;
            const int available = a.columns - t0 * kTile;
            for (int i = threadIdx.x; i < nt * kTile; i += kThreadsW) xs[i] = i < available ? load_f32(x + i) : 0.0f;
            __syncthreads();
            build_tables<0, kThreadsW>(tables, xs, 0);
            float acc = 0.0f, part = 0.0f;
            __syncthreads();  // tables of the first tile complete

            // Local tile v uses table buffer v & 1 and register set v & 1; the loop body covers an even and an
            // odd tile so that both are fixed at compile time (constant table offsets, no register copies).
            auto tile = [&](auto buffer_tag, int v, const TileData& cur, TileData& next) {
                constexpr int BUF = decltype(buffer_tag)::value;
                if (v + 1 < nt) {
                    load_tile<B, BUF == 0>(codes, scales, v + 1, t0 + v + 1, next);  // tile v + 1 is odd if v is even
                    build_tables<1 - BUF, kThreadsW>(tables, xs, v + 1);
                }
                const float lo = chunk_sum<BUF, 0>(cur.c0, tables);
                const float hi = chunk_sum<BUF, 32>(cur.c1, tables);
                if constexpr (B == 64) {
                    acc += lo * cur.s0;  // block 2t
                    acc += hi * cur.s1;  // block 2t + 1 (zero codes and scale in the padding slot)
                } else if constexpr (B == 128) {
                    acc += (lo + hi) * cur.s0;
                } else {
                    part += lo + hi;
                    if constexpr (BUF == 1) {  // second half of the block: segments start on even tiles
                        acc += part * cur.s0;
                        part = 0.0f;
                    }
                }
                __syncthreads();  // next tables built; this tile's tables and (last tile) the activations read
            };
            for (int v = 0; v < nt; v += 2) {
                tile(std::integral_constant<int, 0>{}, v, even, odd);
                if (v + 1 < nt) tile(std::integral_constant<int, 1>{}, v + 1, odd, even);
            }

            if (live && row < m.rows) {
                if (t0 == 0 && nt == a.tiles)
                    store_f32(m.y + static_cast<int64_t>(position) * m.rows + row, acc);
                else
                    store_f32(a.partials + (static_cast<int64_t>(blockIdx.x) * 2 + slot) * kThreadsW + threadIdx.x,
                              acc);
            }
        }
        u += nt;
        t0 = 0;
        if (++item_group == a.groups) {
            item_group = 0;
            if (++member == a.count) {
                member = 0;
                ++position;
            }
        }
    }
}

// Adds the pieces of one item cut between workgroups (one workgroup per cut item), in range order from +0
// with eight loads in flight at a time.
template <int W>
__global__ __launch_bounds__(64 * W) void t2_fixup_kernel(MatDesc one, const MatDesc* __restrict__ group,
                                                          T2Args a) {
    constexpr int kThreadsW = 64 * W;
    const T2Fixup f = a.fixups[blockIdx.x];
    const MatDesc m = group ? group[f.member] : one;
    const int row = f.panel0 * kT2PanelRows + threadIdx.x;
    if (row >= m.rows) return;
    const float* p = a.partials + threadIdx.x;
    float sum = 0.0f + load_f32(p + (static_cast<int64_t>(f.first) * 2 + f.first_slot) * kThreadsW);
    int h = f.first + 1;
    for (; h + 8 <= f.last + 1; h += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = load_f32(p + static_cast<int64_t>(h + k) * 2 * kThreadsW);
#pragma unroll
        for (int k = 0; k < 8; ++k) sum += v[k];
    }
    for (; h <= f.last; ++h) sum += load_f32(p + static_cast<int64_t>(h) * 2 * kThreadsW);
    store_f32(m.y + static_cast<int64_t>(f.position) * m.rows + row, sum);
}

// ---- One matrix at one position: column slices joined in the kernel ----
//
// A single MatVec is latency-bound, and the stream-K plan's second launch is a large part of its time. Here
// workgroup (panel, slice) owns one 64-row panel and a contiguous slice of its tiles; each wave takes one
// tile at a time with its own pair tables, so no wave waits for tables another wave builds. The waves' row sums are added in LDS in wave order, and
// the S slices of a panel are joined by a binary tree of 64-bit atomic exchanges per row: the two siblings
// of a node each swap (generation << 32 | bits of their sum) into the node's slot; the one that finds no
// value of its own launch's generation there is done, the other adds the two sums (left + right, whichever
// came first) and carries the result up, and puts the slot back to empty. Each value travels inside the
// atomic that the reader sees, so no fence is needed, and the order of every addition is fixed by the tree,
// so results do not depend on scheduling. The slots start empty (zeroed with the plan's scratch) and a
// launch that overlaps no other launch of the same scratch leaves them empty. Launches that do overlap can
// leave a value behind; it carries another launch's generation (the host numbers every launch, and never
// uses 0), so a later launch takes it for an empty slot instead of adding it.
struct T2SliceArgs {
    int columns;
    int tiles;
    int chunks;
    int slots;
    int panels;
    int slices;                     // S
    int groups;                     // tiles per slice
    uint32_t generation;            // this launch's tag in the exchange slots (never 0)
    unsigned long long* exchange;   // [tree node][panels * 64]
};

constexpr int kSliceMaxWaves = 16;  // 16 waves x 4 KB of tables fill the 64 KB of LDS the kernel uses
constexpr int kSliceMaxSlices = 8;  // at most three levels of exchanges

// Orders this wave's LDS accesses across the call: the LDS executes one wave's instructions in issue
// order, so once the wave has waited for its own outstanding LDS operations, keeping the compiler from moving
// loads and stores across the point is all that the other lanes' table entries need.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int B>
__global__ __launch_bounds__(64 * kSliceMaxWaves) void t2_slice_kernel(MatDesc one, const MatDesc* __restrict__ group,
                                                                      T2SliceArgs a) {
    const MatDesc m = group ? group[0] : one;
    extern __shared__ float lds[];  // [waves][kTableFloats] tables, then [waves][64] wave sums
    const int waves = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* table = lds + wave * kTableFloats;
    const int panel = blockIdx.x / a.slices, slice = blockIdx.x - panel * a.slices;
    const int g_begin = slice * a.groups, g_end = min(a.tiles, g_begin + a.groups);
    const uint8_t* codes = m.w + static_cast<int64_t>(panel) * a.chunks * 1024 + lane * 16;
    const uint8_t* scales =
        m.w + static_cast<int64_t>(a.panels) * a.chunks * 1024 + static_cast<int64_t>(panel) * a.slots * 256 + lane * 4;
    // Table entry (c0 + 4 c1) of the lane's pair: entries 4 c1 .. 4 c1 + 3 are written as one 16-byte store.
    const auto build = [&](float x0, float x1) {
        const float4 lo = make_float4(0.0f, x0, -x0, 0.0f);
#pragma unroll
        for (int c1 = 0; c1 < 4; ++c1) {
            const float h = c1 == 1 ? x1 : (c1 == 2 ? -x1 : 0.0f);
            *reinterpret_cast<float4*>(table + lane * 16 + 4 * c1) =
                make_float4(lo.x + h, lo.y + h, lo.z + h, lo.w + h);
        }
    };
    // Wave w takes tiles g_begin + w, + waves, ... A B = 256 block spans two tiles, which may go to different
    // waves or slices: each half's sum is multiplied by the block scale on its own.
    float acc = 0.0f;
    for (int u = g_begin + wave; u < g_end; u += waves) {
        // The activations first: the table build then waits only for them, while the codes stream in.
        const int col = u * kTile + 2 * lane;
        const float x0 = col < a.columns ? load_f32(m.x + col) : 0.0f;
        const float x1 = col + 1 < a.columns ? load_f32(m.x + col + 1) : 0.0f;
        const u32x4 c0 = stream16(codes + (2 * u) * 1024);
        const u32x4 c1 = stream16(codes + (2 * u + 1) * 1024);
        float s0, s1 = 0.0f;
        if constexpr (B == 64) {
            s0 = __uint_as_float(stream4(scales + (2 * u) * 256));
            s1 = __uint_as_float(stream4(scales + (2 * u + 1) * 256));
        } else if constexpr (B == 128) {
            s0 = __uint_as_float(stream4(scales + u * 256));
        } else {
            s0 = __uint_as_float(stream4(scales + (u >> 1) * 256));
        }
        __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the build waits for x
        build(x0, x1);
        wave_lds_order();  // every lane's pair table written
        float lo = 0.0f, hi = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const u32x4& rec = half == 0 ? c0 : c1;
            float s0p = 0.0f, s1p = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t l4 = rec[d] & 0x3C3C3C3Cu;
                const uint32_t h4 = __builtin_amdgcn_alignbit(rec[(d + 1) & 3], rec[d], 4) & 0x3C3C3C3Cu;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int pair = 32 * half + 8 * d + 2 * k;
                    const uint32_t ia = __builtin_amdgcn_perm(0u, l4, 0x0C0C0C00u | k);
                    const uint32_t ib = __builtin_amdgcn_perm(0u, h4, 0x0C0C0C00u | k);
                    const char* base = reinterpret_cast<const char*>(table + pair * 16);
                    const float ta = *reinterpret_cast<const float*>(base + ia);
                    const float tb = *reinterpret_cast<const float*>(base + 64 + ib);
                    if (d == 0 && k == 0) {
                        s0p = ta;
                        s1p = tb;
                    } else {
                        s0p += ta;
                        s1p += tb;
                    }
                }
            }
            (half == 0 ? lo : hi) = s0p + s1p;
        }
        wave_lds_order();  // the tables read before the next tile's build overwrites them
        if constexpr (B == 64) {
            acc += lo * s0;
            acc += hi * s1;
        } else {
            acc += (lo + hi) * s0;
        }
    }
    __syncthreads();  // every wave is done with its tables
    float* sums = lds;
    sums[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float piece = 0.0f;
    for (int w = 0; w < waves; ++w) piece += sums[w * 64 + lane];

    const int row = panel * kT2PanelRows + lane;
    const int64_t stride = static_cast<int64_t>(a.panels) * kT2PanelRows;
    unsigned long long* level = a.exchange;
    int i = slice;
    for (int count = a.slices; count > 1; count = (count + 1) >> 1) {
        if ((i ^ 1) < count) {  // the node has both children at this level
            unsigned long long* slot = level + static_cast<int64_t>(i >> 1) * stride + row;
            const unsigned long long mine = (static_cast<unsigned long long>(a.generation) << 32) | __float_as_uint(piece);
            const unsigned long long old =
                __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // First to arrive (empty, or a value an overlapping launch left): the sibling carries the pair.
            if (static_cast<uint32_t>(old >> 32) != a.generation) return;
            const float other = __uint_as_float(static_cast<uint32_t>(old));
            piece = (i & 1) ? other + piece : piece + other;
            __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        level += static_cast<int64_t>(count >> 1) * stride;
        i >>= 1;
    }
    if (row < m.rows) store_f32(m.y + row, piece);
}

template <int B, int W>
hipError_t launch(const MatDesc& one, const MatDesc* group, const T2Plan& plan, const T2Args& a,
                  hipStream_t stream) {
    const size_t lds = static_cast<size_t>(plan.staged_tiles) * kTile * sizeof(float);
    t2_kernel<B, W><<<plan.workgroups, 64 * W, lds, stream>>>(one, group, a);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && plan.fixups > 0) {
        t2_fixup_kernel<W><<<plan.fixups, 64 * W, 0, stream>>>(one, group, a);
        e = hipGetLastError();
    }
    return e;
}

template <int B, int W>
const void* kernel_address() {
    return reinterpret_cast<const void*>(&t2_kernel<B, W>);
}

}  // namespace

int t2_resident_workgroups(int block_size, int waves, int staged_tiles) {
    const void* f = nullptr;
    switch (block_size * 10 + waves) {
        case 644: f = kernel_address<64, 4>(); break;
        case 648: f = kernel_address<64, 8>(); break;
        case 1284: f = kernel_address<128, 4>(); break;
        case 1288: f = kernel_address<128, 8>(); break;
        case 2564: f = kernel_address<256, 4>(); break;
        case 2568: f = kernel_address<256, 8>(); break;
        case 1296: f = kernel_address<128, 16>(); break;
        default: return 0;
    }
    int n = 0;
    const size_t lds = static_cast<size_t>(staged_tiles) * kTile * sizeof(float);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 64 * waves, lds) != hipSuccess) return 0;
    return n;
}

// Workgroups of the sliced kernel with `waves` waves that fit on a CU at once (1 if unknown).
static int t2_slice_resident_workgroups(int block_size, int waves) {
    const void* f = nullptr;
    switch (block_size) {
        case 64: f = reinterpret_cast<const void*>(&t2_slice_kernel<64>); break;
        case 128: f = reinterpret_cast<const void*>(&t2_slice_kernel<128>); break;
        case 256: f = reinterpret_cast<const void*>(&t2_slice_kernel<256>); break;
        default: return 1;
    }
    int n = 0;
    const size_t lds = static_cast<size_t>(waves) * kTableFloats * sizeof(float);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 64 * waves, lds) != hipSuccess || n < 1) return 1;
    return n;
}

namespace {

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace

T2Plan t2_plan(int rows_max, int columns, int block_size, int count, int positions) {
    T2Plan p{};
    p.rows_max = rows_max;
    p.columns = columns;
    p.block_size = block_size;
    p.count = count;
    p.positions = positions;
    const T2Layout l = t2_layout(rows_max, columns, block_size);
    const int step = block_size == 256 ? 2 : 1;  // B = 256 ranges hold whole blocks (tile pairs)
    int cus = 0, device = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
        cus = 256;

    // One matrix at one position: the sliced kernel, one tile per wave, when all its workgroups fit on the
    // chip at once and a panel needs at most kSliceMaxSlices slices: eight waves per workgroup if that fits
    // (more, smaller workgroups), else sixteen; otherwise sixteen waves that take several tiles each.
    if (count == 1 && positions == 1) {
        const auto fits = [&](int waves, int slices) {
            return static_cast<int64_t>(l.panels) * slices <=
                   static_cast<int64_t>(t2_slice_resident_workgroups(block_size, waves)) * cus;
        };
        int waves = 0, per = 0;
        for (const int w : {8, kSliceMaxWaves}) {
            if (ceil_div(l.tiles, w) <= kSliceMaxSlices && fits(w, static_cast<int>(ceil_div(l.tiles, w)))) {
                waves = per = w;
                break;
            }
        }
        if (waves == 0) {
            per = static_cast<int>(ceil_div(l.tiles, kSliceMaxSlices));
            if (fits(kSliceMaxWaves, static_cast<int>(ceil_div(l.tiles, per)))) waves = kSliceMaxWaves;
        }
        if (waves > 0) {
            const int slices = static_cast<int>(ceil_div(l.tiles, per));
            int64_t nodes = 0;  // exchange slots per row: the internal nodes of the slices' tree
            for (int c = slices; c > 1; c = (c + 1) >> 1) nodes += c >> 1;
            p.slices = slices;
            p.slice_groups = per;
            p.waves = std::min({waves, per, l.tiles});  // no wave without a tile
            p.workgroups = l.panels * slices;
            p.scratch_bytes = std::max<size_t>(256, static_cast<size_t>(nodes) * l.panels * kT2PanelRows * 8);
            p.tables.assign(p.scratch_bytes, 0);
            return p;
        }
    }

    // Eight waves (eight panels) per workgroup share each tile's tables when that still leaves at least
    // eight tiles per workgroup on a full chip; otherwise four. For B = 128, sixteen waves when they too
    // leave eight tiles per workgroup: half the table building per row, measured 1.1-2.2% faster from HBM at
    // 4096 x 4096, 11008 x 4096, 4096 x 11008 and 8192 x 8192 (B = 64 was 3% slower, B = 256 the same).
    const int64_t members = static_cast<int64_t>(count) * positions;
    const auto units = [&](int w) { return members * ceil_div(l.panels, w) * l.tiles; };
    const auto resident = [&](int w, int staged) {
        const int n = t2_resident_workgroups(block_size, w, staged);
        return static_cast<int64_t>(std::max(n, 1)) * cus;
    };
    const int staged_max = std::min(l.tiles, kMaxStagedTiles);
    if (units(8) < 8 * resident(8, staged_max))
        p.waves = 4;
    else if (block_size == 128 && units(16) >= 8 * resident(16, staged_max))
        p.waves = 16;
    else
        p.waves = 8;
    const int W = p.waves;
    const int groups = static_cast<int>(ceil_div(l.panels, W));
    const int64_t total = units(W);
    if (total > INT32_MAX) return p;  // workgroups == 0: not plannable
    const int64_t steps = total / step;
    // As many workgroups as the CUs hold at once, each with at least two tiles and at most what it stages.
    int64_t wgs = std::min(resident(W, std::min(l.tiles, kMaxStagedTiles)), ceil_div(total, 2));
    wgs = std::max(wgs, ceil_div(total, kMaxStagedTiles));
    wgs = std::max<int64_t>(1, std::min(wgs, steps));
    const int P = static_cast<int>(wgs);
    p.workgroups = P;

    std::vector<int> starts(P + 1);
    for (int g = 0; g <= P; ++g) starts[g] = static_cast<int>((static_cast<int64_t>(g) * steps / P) * step);
    int longest = 0;
    for (int g = 0; g < P; ++g) longest = std::max(longest, starts[g + 1] - starts[g]);
    p.staged_tiles = std::min(l.tiles, longest);
    // The range holding tile u.
    const auto owner = [&](int u) {
        return static_cast<int>(std::upper_bound(starts.begin(), starts.end(), u) - starts.begin()) - 1;
    };
    std::vector<T2Fixup> fixups;
    for (int g = 1; g < P; ++g) {
        const int item = starts[g] / l.tiles;
        const int start = item * l.tiles;
        if (starts[g] == start || owner(start) + 1 != g) continue;  // no cut here, or handled at an earlier cut
        T2Fixup f{};
        f.member = (item / groups) % count;
        f.position = item / groups / count;
        f.panel0 = (item % groups) * W;
        f.first = g - 1;
        f.last = owner(start + l.tiles - 1);
        f.first_slot = starts[g - 1] == start ? 0 : 1;
        fixups.push_back(f);
    }
    p.fixups = static_cast<int>(fixups.size());
    p.fixup_offset = align256(sizeof(int) * starts.size());
    p.partial_offset = align256(p.fixup_offset + sizeof(T2Fixup) * fixups.size());
    p.scratch_bytes = p.partial_offset + static_cast<size_t>(P) * 2 * 64 * W * sizeof(float);
    p.tables.assign(p.partial_offset, 0);
    std::memcpy(p.tables.data(), starts.data(), sizeof(int) * starts.size());
    if (!fixups.empty()) std::memcpy(p.tables.data() + p.fixup_offset, fixups.data(), sizeof(T2Fixup) * fixups.size());
    return p;
}

hipError_t launch_t2(const MatDesc& one, const MatDesc* group, int count, LaunchShape s, const T2Plan& plan,
                     void* scratch, uint32_t generation, hipStream_t stream) {
    if (count <= 0 || s.rows_max <= 0 || s.positions <= 0) return hipSuccess;
    if (generation == 0) return hipErrorInvalidValue;
    if (plan.workgroups < 1 || scratch == nullptr || plan.rows_max != s.rows_max || plan.columns != s.columns ||
        plan.block_size != s.block_size || plan.count != count || plan.positions != s.positions ||
        plan.staged_tiles > kMaxStagedTiles)
        return hipErrorInvalidValue;
    const T2Layout l = t2_layout(s.rows_max, s.columns, s.block_size);
    if (plan.slices > 0) {
        if (count != 1 || s.positions != 1 || plan.waves < 1 || plan.waves > kSliceMaxWaves ||
            plan.workgroups != l.panels * plan.slices)
            return hipErrorInvalidValue;
        const T2SliceArgs a{s.columns, l.tiles,       l.chunks,          l.slots, l.panels, plan.slices,
                            plan.slice_groups, generation, static_cast<unsigned long long*>(scratch)};
        const size_t lds = static_cast<size_t>(plan.waves) * kTableFloats * sizeof(float);
        switch (s.block_size) {
            case 64: t2_slice_kernel<64><<<plan.workgroups, 64 * plan.waves, lds, stream>>>(one, group, a); break;
            case 128: t2_slice_kernel<128><<<plan.workgroups, 64 * plan.waves, lds, stream>>>(one, group, a); break;
            case 256: t2_slice_kernel<256><<<plan.workgroups, 64 * plan.waves, lds, stream>>>(one, group, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    const int W = plan.waves;
    char* base = static_cast<char*>(scratch);
    const T2Args a{s.columns,
                   l.tiles,
                   l.chunks,
                   l.slots,
                   count,
                   static_cast<int>(ceil_div(l.panels, W)),
                   reinterpret_cast<const int*>(base),
                   reinterpret_cast<const T2Fixup*>(base + plan.fixup_offset),
                   reinterpret_cast<float*>(base + plan.partial_offset)};
    switch (s.block_size * 10 + W) {
        case 644: return launch<64, 4>(one, group, plan, a, stream);
        case 648: return launch<64, 8>(one, group, plan, a, stream);
        case 1284: return launch<128, 4>(one, group, plan, a, stream);
        case 1288: return launch<128, 8>(one, group, plan, a, stream);
        case 2564: return launch<256, 4>(one, group, plan, a, stream);
        case 2568: return launch<256, 8>(one, group, plan, a, stream);
        case 1296: return launch<128, 16>(one, group, plan, a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace satori
