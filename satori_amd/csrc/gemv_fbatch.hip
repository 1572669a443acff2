// Many-position FP32-activation product for Q8_0 and Q4_0 on the matrix cores (gfx950 bf16 MFMA): the
// batched form of QuantizedMatVec.ExecuteBatch for the legacy formats (ExecuteBatchFloat / ExecuteBatchRows,
// src/Satori.Core/QuantizedMatVec.cs:221-347), with the arithmetic of the scalar reference per block
// (QuantizedMatVec.ExecuteScalar, QuantizedMatVec.cs:45-78: sum = q . x over the block's 32 weights, then
// total += Scale * sum), so the weights are read once per 32-position tile instead of once per position.
//
// Exact operands. A block's codes q are small integers (Q8_0: -128..127; Q4_0: -8..7), exact in bf16. Each
// activation x is split into three bf16 parts x = hi + lo + lolo, each the next 8 significant bits cut by
// truncation (x - hi and (x - hi) - lo are exact in FP32, and the last part has at most 8 significant bits).
// bf16 has FP32's exponent range, but a part below 2^-126 would be a bf16 subnormal: its bits below 2^-133 do
// not fit and the matrix cores may flush it. So each position is first lifted by an exact power of two 2^k
// (k >= 0) that brings its largest |x| into [2^64, 2^65). Every nonzero bit of a lifted x then weighs at least
// 2^(-149 + k); in a position whose largest |x| is below 2^42 (k >= 23) every nonzero part is a normal bf16,
// so the split is exact for every finite element, subnormals included. In a position with a larger |x| a
// part can be subnormal only for an element below 2^-174 of the largest. From 2^64 on k = 0, so a product
// that overflows in the reference overflows here too. An infinite or NaN x keeps k = 0 for its position and
// keeps itself as hi (a NaN as the canonical quiet NaN) with zero lo and lolo, so q * x gives the IEEE
// result of the single product. Every q * part product is exact in FP32 (at most 16 significant bits), the
// sums of a lifted position stay below 2^120, and the block sum sum_k q_k x_k is three bf16 MFMA chains
// accumulating in FP32. Only the FP32 additions round, in an order of their own, and the final scaling by
// 2^-k rounds once where the result is subnormal: within 1e-5 * sum |w x| + n * 2^-149 of the reference,
// like every FP32 path here.
//
// Three launches: fbatch_lift_kernel finds each position's lifting exponent, fbatch_pack_kernel splits the
// lifted activations into a workspace in MFMA first-operand order, and fbatch_kernel runs the product: waves
// of 32-row x 32-position tiles, four row tiles per workgroup sharing the split activations staged in LDS a
// round of W blocks at a time, one block of the round per way.
#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 32;      // rows and positions per wave tile
constexpr int kPartBytes = 1024;                       // one part of one K step of one (block, tile)
constexpr int kBlockTileBytes = 3 * 2 * kPartBytes;    // 3 parts x 2 K steps of 16 columns

// Workspace: for 32-column block b and 32-position tile t, 6 KB at (b * tiles + t) * 6144: part s (0: hi,
// 1: lo, 2: lolo), K step st (columns 32b + 16st .. + 15) at (2s + st) * 1024, lane l = 32h + p holding the
// 8 bf16 of position 32t + p, columns 32b + 16st + 8h .. + 7. Positions past the last are zero. After the
// blocks x tiles records: one int32 lifting exponent k per position (tiles x 32 of them, zero past the last).

// The exponent k lifting the largest |x| of a position into [2^64, 2^65), from the largest magnitude's FP32
// bits: 0 for a zero or non-finite position, and for magnitudes of 2^64 and more.
__device__ __forceinline__ int lift_exponent(uint32_t max_bits) {
    if (max_bits == 0u || max_bits >= 0x7F800000u) return 0;
    const int e = max_bits >= 0x00800000u ? static_cast<int>(max_bits >> 23) - 127  // normal: floor(log2)
                                          : (31 - __clz(static_cast<int>(max_bits))) - 149;  // subnormal
    return e >= 64 ? 0 : 64 - e;
}

// One workgroup per position tile slot (32 per tile): the lifting exponent of position p (0 past the last).
// Rows of 16-byte-aligned activations are read in 16-byte pieces, four per thread in flight.
__global__ __launch_bounds__(256) void fbatch_lift_kernel(const float* __restrict__ x, int columns, int positions,
                                                          int* __restrict__ lift) {
    __shared__ uint32_t wave_max[4];
    const int p = blockIdx.x;
    uint32_t m = 0u;
    if (p < positions) {
        const float* row = x + static_cast<int64_t>(p) * columns;
        uint32_t m1 = 0u, m2 = 0u, m3 = 0u;
        const auto mag = [](uint32_t bits) { return bits & 0x7FFFFFFFu; };
        if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) {  // rows are 128-byte multiples: all aligned
            const int pieces = columns >> 2;
            int i = threadIdx.x;
            for (; i + 768 < pieces; i += 1024) {
                const u32x4 a = *(const SATORI_GLOBAL u32x4*)(row + 4 * i);
                const u32x4 b = *(const SATORI_GLOBAL u32x4*)(row + 4 * (i + 256));
                const u32x4 c = *(const SATORI_GLOBAL u32x4*)(row + 4 * (i + 512));
                const u32x4 d = *(const SATORI_GLOBAL u32x4*)(row + 4 * (i + 768));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    m = max(m, mag(a[e]));
                    m1 = max(m1, mag(b[e]));
                    m2 = max(m2, mag(c[e]));
                    m3 = max(m3, mag(d[e]));
                }
            }
            for (; i < pieces; i += 256) {
                const u32x4 a = *(const SATORI_GLOBAL u32x4*)(row + 4 * i);
#pragma unroll
                for (int e = 0; e < 4; ++e) m = max(m, mag(a[e]));
            }
        } else {
            for (int c = threadIdx.x; c < columns; c += 256) m = max(m, mag(__float_as_uint(load_f32(row + c))));
        }
        m = max(max(m, m1), max(m2, m3));  // magnitudes order like their bits; NaN bits exceed every finite
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), off)));
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0)
        lift[p] = lift_exponent(max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3])));
}

// The three bf16 parts of x (bit patterns in the low 16 bits).
__device__ __forceinline__ void split3(float x, uint32_t& hi, uint32_t& lo, uint32_t& lolo) {
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7F800000u) == 0x7F800000u) {  // infinite or NaN
        hi = (b & 0x007FFFFFu) ? (0x7FC0u | ((b >> 16) & 0x8000u)) : (b >> 16);
        lo = lolo = 0u;
        return;
    }
    const float h = __uint_as_float(b & 0xFFFF0000u);
    const float r = __fsub_rn(x, h);  // exact: the bits of x below its top eight
    const uint32_t rb = __float_as_uint(r);
    const float l = __uint_as_float(rb & 0xFFFF0000u);
    const float ll = __fsub_rn(r, l);  // exact, at most eight significant bits
    hi = b >> 16;
    lo = rb >> 16;
    lolo = __float_as_uint(ll) >> 16;
}

// One thread per (block, position tile, K step, lane): the 8 activations of its operand slot, split.
__global__ __launch_bounds__(256) void fbatch_pack_kernel(const float* __restrict__ x, int columns, int positions,
                                                          int tiles, uint8_t* __restrict__ workspace,
                                                          const int* __restrict__ lift) {
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int blocks = columns / 32;
    if (item >= static_cast<int64_t>(blocks) * tiles * 128) return;
    const int lane = static_cast<int>(item & 63), st = static_cast<int>((item >> 6) & 1);
    const int64_t bt = item >> 7;  // b * tiles + t
    const int b = static_cast<int>(bt / tiles), t = static_cast<int>(bt - static_cast<int64_t>(b) * tiles);
    const int p = t * kTile + (lane & 31);
    const int c0 = 32 * b + 16 * st + 8 * (lane >> 5);
    uint32_t part[3][4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    if (p < positions) {
        const float* src = x + static_cast<int64_t>(p) * columns + c0;
        const int k = lift[p];
        float v[8];
        if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
            const u32x4 a = *(const SATORI_GLOBAL u32x4*)(src), c = *(const SATORI_GLOBAL u32x4*)(src + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = __uint_as_float(a[e]);
                v[4 + e] = __uint_as_float(c[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = load_f32(src + e);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t h, l, ll;
            split3(__builtin_amdgcn_ldexpf(v[e], k), h, l, ll);  // exact: the lifted value is at most 2^65
            const int shift = 16 * (e & 1);
            part[0][e >> 1] |= h << shift;
            part[1][e >> 1] |= l << shift;
            part[2][e >> 1] |= ll << shift;
        }
    }
    uint8_t* dst = workspace + bt * kBlockTileBytes + st * kPartBytes + 16 * lane;
#pragma unroll
    for (int s = 0; s < 3; ++s)
        *reinterpret_cast<u32x4*>(dst + 2 * s * kPartBytes) = u32x4{part[s][0], part[s][1], part[s][2], part[s][3]};
}

// Two small integers as a pair of bf16 (exact: at most 8 significant bits): the high halves of their FP32
// patterns, q0 low, joined by one byte permute.
__device__ __forceinline__ uint32_t pack_bf16(int q0, int q1) {
    return __builtin_amdgcn_perm(__float_as_uint(static_cast<float>(q1)), __float_as_uint(static_cast<float>(q0)),
                                 0x07060302u);
}

// The lane's second operand (8 codes of its row) for K step st of a block, from the device layout: Q8_0
// records are the 32 signed bytes; Q4_0 records hold q - 8 per nibble (byte j: low nibble weight j, high
// nibble weight j + 16), so step 0 takes low nibbles and step 1 high nibbles of bytes 8h .. 8h + 7.
template <int FORMAT>
__device__ __forceinline__ bf16x8 codes_operand(const uint32_t (&raw)[4], int st) {
    uint32_t d[4];
    if constexpr (FORMAT == kQ8_0) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t w = raw[2 * st + k];
            d[2 * k] = pack_bf16(static_cast<int8_t>(w), static_cast<int8_t>(w >> 8));
            d[2 * k + 1] = pack_bf16(static_cast<int8_t>(w >> 16), static_cast<int8_t>(w >> 24));
        }
    } else {
        const int shift = 4 * st;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t w = raw[k];
            auto nib = [&](int byte) {
                return __builtin_amdgcn_sbfe(static_cast<int>(w), 8 * byte + shift, 4);  // q - 8, sign-extended
            };
            d[2 * k] = pack_bf16(nib(0), nib(1));
            d[2 * k + 1] = pack_bf16(nib(2), nib(3));
        }
    }
    return __builtin_bit_cast(bf16x8, u32x4{d[0], d[1], d[2], d[3]});
}

__device__ __forceinline__ f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

struct FbatchArgs {
    const uint8_t* w;          // device layout (code records, then FP16 scales)
    const uint8_t* workspace;  // split activations (fbatch_pack_kernel)
    const int* lift;           // per position: the exponent its activations were lifted by
    float* y;                  // [positions][rows]
    int rows, blocks, positions, tiles;
};

// Workgroup u of the padded grid: units (row group of four row tiles, position tile), position tiles fastest,
// consecutive units on one XCD (workgroup ids are dealt to the eight XCDs in turn), so the position tiles
// that share a row group's weights read them through one L2. W ways per row tile: a round stages W
// consecutive blocks' split activations once for the workgroup, and way w of each row tile computes the
// round's block w, so the four row tiles share every staged byte and the workgroup keeps 4 W waves busy.
// Each way sums its own blocks; the ways' sums are added once at the end, in way order.
template <int FORMAT, int W>
__global__ __launch_bounds__(256 * W) void fbatch_kernel(FbatchArgs a) {
    constexpr int kRecord = FORMAT == kQ8_0 ? 32 : 16;
    constexpr int kThreads = 256 * W;
    constexpr int kRoundBytes = W * kBlockTileBytes;
    constexpr int kChunks = kRoundBytes / 16;                                // 16-byte pieces staged per round
    constexpr int kLoads = (kChunks + kThreads - 1) / kThreads;
    constexpr int kSumBytes = (W - 1) * 4 * 16 * 64 * 4;                    // the ways' sums at the end
    __shared__ uint8_t lds[2 * kRoundBytes > kSumBytes ? 2 * kRoundBytes : kSumBytes];  // two rounds' buffers

    const int per_xcd = gridDim.x >> 3;
    const int u = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    const int groups = (a.rows + 4 * kTile - 1) / (4 * kTile);
    if (u >= groups * a.tiles) return;  // whole workgroup
    const int group = u / a.tiles, t = u - group * a.tiles;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
    const int rt = wave & 3, way = wave >> 2;
    const int row = (group * 4 + rt) * kTile + (lane & 31);
    const int row_c = row < a.rows ? row : a.rows - 1;  // rows past the last compute on a live row, store nothing
    const int blocks = a.blocks;
    const int64_t count = static_cast<int64_t>(a.rows) * blocks;
    const uint8_t* records = a.w + static_cast<int64_t>(row_c) * blocks * kRecord + 8 * h;
    const uint8_t* scales = a.w + count * kRecord + static_cast<int64_t>(row_c) * blocks * 2;
    const uint8_t* parts = a.workspace + static_cast<int64_t>(t) * kBlockTileBytes;
    const int64_t part_stride = static_cast<int64_t>(a.tiles) * kBlockTileBytes;  // block b to b + 1

    // Staging of round k (blocks W k .. W k + W - 1): thread i copies the 16-byte pieces i, i + threads, ...
    // Piece c of a round lies in block W k + c_blk of the round; its address steps by W blocks a round (an
    // addition, not a 64-bit multiply), and a block past the last reads the last one instead (unused).
    u32x4 st_regs[kLoads];
    const uint8_t* st_ptr[kLoads];
    const uint8_t* st_last[kLoads];
    int st_blk[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int off = 16 * (threadIdx.x + kThreads * j);
        st_blk[j] = off / kBlockTileBytes;
        st_ptr[j] = parts + st_blk[j] * part_stride + off % kBlockTileBytes;
        st_last[j] = parts + (blocks - 1) * part_stride + off % kBlockTileBytes;
    }
    auto stage_load = [&](int k) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            if (threadIdx.x + kThreads * j < kChunks) {
                const uint8_t* src = W * k + st_blk[j] < blocks ? st_ptr[j] : st_last[j];
                st_regs[j] = *(const SATORI_GLOBAL u32x4*)(src);
            }
            st_ptr[j] += W * part_stride;
        }
    };
    auto stage_store = [&](uint8_t* buf) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int c = threadIdx.x + kThreads * j;
            if (c < kChunks) *reinterpret_cast<u32x4*>(buf + 16 * c) = st_regs[j];
        }
    };
    // The lane's codes and scale of block b (clamped to the last block, read and unused past it).
    struct Weights {
        uint32_t raw[4];
        uint32_t scale;
    };
    auto load_weights = [&](int b, Weights& wgt) {
        const int bc = min(b, blocks - 1);
        const uint8_t* rec = records + bc * kRecord;  // within one row: 32-bit offsets
        const uint64_t lo8 = load8_a8(rec);
        wgt.raw[0] = static_cast<uint32_t>(lo8);
        wgt.raw[1] = static_cast<uint32_t>(lo8 >> 32);
        if constexpr (FORMAT == kQ8_0) {
            const uint64_t hi8 = load8_a8(rec + 16);
            wgt.raw[2] = static_cast<uint32_t>(hi8);
            wgt.raw[3] = static_cast<uint32_t>(hi8 >> 32);
        }
        wgt.scale = load2_a2(scales + 2 * bc);
    };

    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    // One block: total += Scale * sum (QuantizedMatVec.cs:74), the product and the sum rounded apart.
    auto block = [&](const Weights& wgt, const uint8_t* sb) {
        f32x16 d = {};
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const bf16x8 w = codes_operand<FORMAT>(wgt.raw, st);
#pragma unroll
            for (int s = 0; s < 3; ++s) {
                const bf16x8 x = *reinterpret_cast<const bf16x8*>(sb + (2 * s + st) * kPartBytes + 16 * lane);
                d = mfma_bf16(x, w, d);
            }
        }
        const float scale = half_bits_to_float(wgt.scale);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(scale, d[i]));
    };

    // Two LDS buffers: round k is computed from buffer k & 1 while round k + 1's parts, loaded during round
    // k - 1, are stored into the other and round k + 2's are loaded; the weights run two rounds ahead too.
    const int rounds = (blocks + W - 1) / W;
    Weights w0, w1, w2;
    stage_load(0);
    stage_store(lds);
    stage_load(1);
    load_weights(way, w0);
    load_weights(W + way, w1);
    __syncthreads();  // round 0 staged
    for (int k = 0; k < rounds; ++k) {
        uint8_t* cur = lds + (k & 1) * kRoundBytes;
        load_weights(W * (k + 2) + way, w2);  // clamped to the last block past the end
        if (W * k + way < blocks) block(w0, cur + way * kBlockTileBytes);
        if (k + 1 < rounds) {
            stage_store(lds + ((k + 1) & 1) * kRoundBytes);  // its buffer was last read in round k - 1
            if (k + 2 < rounds) stage_load(k + 2);
        }
        __syncthreads();  // round k + 1 staged, round k's buffer read
        w0 = w1;
        w1 = w2;
    }

    // The ways' sums, added in way order by way 0 (the loop's last barrier ends every read of the buffers).
    if constexpr (W > 1) {
        float* sums = reinterpret_cast<float*>(lds);  // [way - 1][row tile][output][lane]
        if (way > 0)
#pragma unroll
            for (int i = 0; i < 16; ++i) sums[(((way - 1) * 4 + rt) * 16 + i) * 64 + lane] = acc[i];
        __syncthreads();
        if (way > 0) return;
#pragma unroll
        for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = __fadd_rn(acc[i], sums[(((w2 - 1) * 4 + rt) * 16 + i) * 64 + lane]);
    }
    if (row >= a.rows) return;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int p = t * kTile + 8 * (i >> 2) + 4 * h + (i & 3);
        // Undo the position's lifting: exact unless the result is subnormal, where it rounds once.
        if (p < a.positions)
            store_f32(a.y + static_cast<int64_t>(p) * a.rows + row, __builtin_amdgcn_ldexpf(acc[i], -a.lift[p]));
    }
}

}  // namespace

// From one whole position tile on. Below it the product runs few workgroups (row groups x one tile) and is
// latency-bound: measured at 8-32 positions, 4096x4096 Q8_0 takes 56 us against 21-52 us for the
// single-position kernel per position, 11008x4096 Q4_0 44 us against 40-150 us.
int fbatch_min_positions() { return 32; }

size_t fbatch_workspace_bytes(int columns, int positions) {
    const int tiles = (positions + kTile - 1) / kTile;
    return static_cast<size_t>(columns / 32) * tiles * kBlockTileBytes + static_cast<size_t>(tiles) * kTile * 4;
}

hipError_t launch_gemv_fbatch(const uint8_t* w, int format, const float* x, uint8_t* workspace, float* y, int rows,
                              int columns, int positions, hipStream_t stream) {
    if (rows <= 0 || positions <= 0 || columns <= 0) return hipSuccess;
    if ((format != kQ8_0 && format != kQ4_0) || columns % 32 != 0) return hipErrorInvalidValue;
    const int blocks = columns / 32;
    const int tiles = (positions + kTile - 1) / kTile;
    const int64_t items = static_cast<int64_t>(blocks) * tiles * 128;
    if ((items + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
    int* lift = reinterpret_cast<int*>(workspace + static_cast<size_t>(blocks) * tiles * kBlockTileBytes);
    fbatch_lift_kernel<<<static_cast<unsigned>(tiles * kTile), 256, 0, stream>>>(x, columns, positions, lift);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    fbatch_pack_kernel<<<static_cast<unsigned>((items + 255) / 256), 256, 0, stream>>>(x, columns, positions, tiles,
                                                                                      workspace, lift);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t units = static_cast<int64_t>((rows + 4 * kTile - 1) / (4 * kTile)) * tiles;
    const int64_t grid = (units + 7) / 8 * 8;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    const FbatchArgs a{w, workspace, lift, y, rows, blocks, positions, tiles};
    // Ways per row tile: as many (4, 2, 1) as keep every workgroup resident at once (two workgroups of 16
    // waves, four of 8 or eight of 4 per CU), so no second wave of workgroups trails the first.
    const int W = units <= 512 ? 4 : (units <= 1024 ? 2 : 1);
    auto go = [&](auto kernel, int w_) { kernel<<<static_cast<unsigned>(grid), 256 * w_, 0, stream>>>(a); };
    if (format == kQ8_0) {
        if (W == 4) go(fbatch_kernel<kQ8_0, 4>, 4); else if (W == 2) go(fbatch_kernel<kQ8_0, 2>, 2); else go(fbatch_kernel<kQ8_0, 1>, 1);
    } else {
        if (W == 4) go(fbatch_kernel<kQ4_0, 4>, 4); else if (W == 2) go(fbatch_kernel<kQ4_0, 2>, 2); else go(fbatch_kernel<kQ4_0, 1>, 1);
    }
    return hipGetLastError();
}

}  // namespace satori
