// Integer K-format product over many positions on the matrix cores (gfx950 int8 MFMA): the prefill form of
// ExecuteBatch (QuantizedMatVec.ExecuteBatchQuantized, src/Satori.Core/QuantizedMatVec.cs:136-219, whose
// per-position arithmetic is QuantizedKAvx2Kernel.ExecuteQuantizedTiled, QuantizedKAvx2Kernel.cs:47-99).
//
// Every integer the reference forms is formed exactly (int8 x int8 products summed in int32 by the MFMA,
// scaled by the 6-bit / int8 block scales in int32), and each block's FP32 term is the reference's
// expression, added to the (row, position) sum in block order from +0, so the outputs equal the
// single-position integer kernel's bit for bit.
//
// Orientation: the MFMA computes D = C x W^T with the positions' Q8_K codes as the first operand (M =
// positions) and the weights' codes as the second (N = rows). Every output a lane holds then belongs to
// the lane's own weight row, so the per-row block scales are lane-local. A workgroup (4 waves) owns 128
// rows (32 per wave) and 64 positions (two 32-position MFMA tiles); blocks are walked in order with the
// positions' codes for the current block staged in LDS.
//
// Q4_K: Dot = sum_j s_j * D_j with D_j = sum over sub-block j (32 weights) of q * c: one 32x32x32 MFMA per
// sub-block and an int32 multiply-add by s_j; Min = sum_j m_j * sum_j c is one more MFMA chain whose weight
// operand is m_j repeated over the sub-block. Q6_K: Dot = sum_k sc_k * (D_k - 32 * sum_k c) over the 16
// groups of 16 weights: one 32x32x16 MFMA per group and a multiply-add by sc_k; the centring term is an
// MFMA chain whose weight operand is sc_k repeated over the group.
#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerGroup = 4 * kRowsPerWave;  // rows per workgroup
constexpr int kPositions = 64;                   // positions per workgroup (two MFMA tiles)
constexpr int kCodeStride = 272;                 // bytes per staged position: 256 codes + 16 of padding

__device__ __forceinline__ i32x16 mfma32(const i32x4& c, const i32x4& w, const i32x16& acc) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(c, w, acc, 0, 0, 0);
}

__device__ __forceinline__ i32x16 mfma16(long c, long w, const i32x16& acc) {
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(c, w, acc, 0, 0, 0);
}

// The (row, block) data one lane needs: Q4_K head (d, dmin, scales) and its half of every 32-byte group of
// nibbles.
struct Q4KLane {
    u32x4 head;
    u32x4 qs[4];  // qs[32g + 16h, +16) for g = 0..3, h = the lane's half
};

__device__ __forceinline__ void q4k_lane_load(const uint8_t* block, int h, Q4KLane& r) {
    r.head = load16_a4(block);
#pragma unroll
    for (int g = 0; g < 4; ++g) r.qs[g] = load16_a4(block + 16 + 32 * g + 16 * h);
}

// Q6_K from the regrouped device layout: the lane's half (8 bytes) of each quarter's ql / ql / qh arrays,
// the quarter scales and d.
struct Q6KLane {
    uint32_t qla[4][2], qlb[4][2], qh[4][2];
    u32x4 sc;  // quarter c's scale for form kk at byte 4c + kk
    float d;
};

__device__ __forceinline__ void q6k_lane_load(const uint8_t* w, int64_t blocks, int64_t index, int h, Q6KLane& r) {
    const uint8_t* record = w + index * 192;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint8_t* q = record + 48 * c + 8 * h;
        r.qla[c][0] = load4_a4(q);
        r.qla[c][1] = load4_a4(q + 4);
        r.qlb[c][0] = load4_a4(q + 16);
        r.qlb[c][1] = load4_a4(q + 20);
        r.qh[c][0] = load4_a4(q + 32);
        r.qh[c][1] = load4_a4(q + 36);
    }
    r.sc = load16_a4(w + blocks * 192 + index * 16);
    const uint32_t pair = load4_a4(w + blocks * 208 + (index & ~int64_t(1)) * 2);
    r.d = half_bits_to_float(pair >> (16 * static_cast<int>(index & 1)));
}

__device__ __forceinline__ uint32_t q6k_form(uint32_t a, uint32_t b, uint32_t hb, int kk) {
    switch (kk) {
        case 0: return (a & 0x0F0F0F0Fu) | ((hb << 4) & 0x30303030u);
        case 1: return (b & 0x0F0F0F0Fu) | ((hb << 2) & 0x30303030u);
        case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u);
        default: return ((b >> 4) & 0x0F0F0F0Fu) | ((hb >> 2) & 0x30303030u);
    }
}

template <int FORMAT>
__global__ __launch_bounds__(kThreads) void gemv_kmfma_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ act,
                                                             float* __restrict__ y, int rows, int blocks,
                                                             int64_t row_bytes, int positions) {
    __shared__ __attribute__((aligned(16))) uint8_t codes[kPositions * kCodeStride];
    __shared__ float pscale[kPositions];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = lane >> 5;                                            // k half of the lane
    const int row = blockIdx.x * kRowsPerGroup + wave * kRowsPerWave + (lane & 31);
    const bool row_live = row < rows;
    const int row_c = row_live ? row : rows - 1;                        // dead rows read a live one
    const int p0 = blockIdx.y * kPositions;

    float acc[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

    for (int b = 0; b < blocks; ++b) {
        // Stage the 64 positions' codes and scales of block b (zero past the last position).
        __syncthreads();  // the previous block's codes are no longer read
        for (int i = threadIdx.x; i < kPositions * 16; i += kThreads) {
            const int p = i >> 4, part = i & 15;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (p0 + p < positions)
                v = load16_a4(act + (static_cast<int64_t>(p0 + p) * blocks + b) * kQ8KBlockBytes + 4 + 16 * part);
            *reinterpret_cast<u32x4*>(codes + p * kCodeStride + 16 * part) = v;
        }
        if (threadIdx.x < kPositions) {
            const int p = threadIdx.x;
            pscale[p] = p0 + p < positions
                            ? load_f32(reinterpret_cast<const float*>(act + (static_cast<int64_t>(p0 + p) * blocks + b) *
                                                                                kQ8KBlockBytes))
                            : 0.0f;
        }
        // This lane's weights for block b, then each 32-position tile in turn: integer dot and min (Q4_K) or
        // centring (Q6_K) sums for the block, and the block's FP32 term added in block order.
        if constexpr (FORMAT == kQ4_K) {
            Q4KLane r;
            q4k_lane_load(w + row_c * row_bytes + static_cast<int64_t>(b) * 144, h, r);
            const float d = half_bits_to_float(r.head[0] & 0xFFFFu), dmin = half_bits_to_float(r.head[0] >> 16);
            __syncthreads();  // codes staged
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                int dot[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) dot[i] = 0;
                i32x16 mins = {};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int sj, mj;
                    q4k_scale_min(j, r.head, sj, mj);
                    const u32x4 raw = r.qs[j >> 1];
                    const i32x4 wq = {static_cast<int>((raw[0] >> (4 * (j & 1))) & 0x0F0F0F0Fu),
                                      static_cast<int>((raw[1] >> (4 * (j & 1))) & 0x0F0F0F0Fu),
                                      static_cast<int>((raw[2] >> (4 * (j & 1))) & 0x0F0F0F0Fu),
                                      static_cast<int>((raw[3] >> (4 * (j & 1))) & 0x0F0F0F0Fu)};
                    const int mb = mj * 0x01010101;
                    const i32x4 wm = {mb, mb, mb, mb};
                    const i32x4 c = *reinterpret_cast<const i32x4*>(codes + (32 * t + (lane & 31)) * kCodeStride +
                                                                   32 * j + 16 * h);
                    const i32x16 dj = mfma32(c, wq, i32x16{});
                    mins = mfma32(c, wm, mins);
#pragma unroll
                    for (int i = 0; i < 16; ++i) dot[i] += sj * dj[i];
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float a = pscale[32 * t + 8 * (i >> 2) + 4 * h + (i & 3)];
                    if (a == 0.0f) continue;  // zero activation block: skipped (QuantizedKAvx2Kernel.cs:86)
                    const float dA = __fmul_rn(d, a), dminA = __fmul_rn(dmin, a);
                    const float term = __fsub_rn(__fmul_rn(dA, static_cast<float>(dot[i])),
                                                 __fmul_rn(dminA, static_cast<float>(mins[i])));
                    acc[t][i] = __fadd_rn(acc[t][i], term);
                }
            }
        } else {
            Q6KLane r;
            q6k_lane_load(w, static_cast<int64_t>(rows) * blocks, static_cast<int64_t>(row_c) * blocks + b, h, r);
            __syncthreads();  // codes staged
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                int dot[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) dot[i] = 0;
#pragma unroll
                for (int k = 0; k < 16; ++k) {  // scale group k: weights 16k .. 16k + 15 of the block
                    const int c = 2 * (k >> 3) + (k & 1), kk = (k & 7) >> 1;
                    const int sc = static_cast<int8_t>(r.sc[c] >> (8 * kk));
                    const long wq = static_cast<long>(q6k_form(r.qla[c][0], r.qlb[c][0], r.qh[c][0], kk)) |
                                    (static_cast<long>(q6k_form(r.qla[c][1], r.qlb[c][1], r.qh[c][1], kk)) << 32);
                    const long cd = *reinterpret_cast<const long*>(codes + (32 * t + (lane & 31)) * kCodeStride +
                                                                   16 * k + 8 * h);
                    const i32x16 dk = mfma16(cd, wq, i32x16{});
#pragma unroll
                    for (int i = 0; i < 16; ++i) dot[i] += sc * dk[i];
                }
                // Centring: sum_k sc_k * (sum of group k's codes), one chain over the block's 32-weight chunks;
                // the lane's 16 weights of chunk u are group 2u + h.
                i32x16 cent = {};
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int k = 2 * u + h;
                    const int c = 2 * (k >> 3) + (k & 1), kk = (k & 7) >> 1;
                    const int sb = static_cast<int>(static_cast<uint8_t>(r.sc[c] >> (8 * kk))) * 0x01010101;
                    const i32x4 ws = {sb, sb, sb, sb};
                    const i32x4 cq = *reinterpret_cast<const i32x4*>(codes + (32 * t + (lane & 31)) * kCodeStride +
                                                                    32 * u + 16 * h);
                    cent = mfma32(cq, ws, cent);
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float a = pscale[32 * t + 8 * (i >> 2) + 4 * h + (i & 3)];
                    if (a == 0.0f) continue;  // zero activation block: skipped
                    // sum sc * (q - 32) * code = dot - 32 * centring, exact in int32.
                    const float term = __fmul_rn(__fmul_rn(a, r.d), static_cast<float>(dot[i] - 32 * cent[i]));
                    acc[t][i] = __fadd_rn(acc[t][i], term);
                }
            }
        }
    }
    if (!row_live) return;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int p = p0 + 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
            if (p < positions) store_f32(y + static_cast<int64_t>(p) * rows + row, acc[t][i]);
        }
}

}  // namespace

int kmfma_min_positions() { return 16; }

hipError_t launch_gemv_kmfma(const uint8_t* w, int format, const uint8_t* act, float* y, int rows, int blocks,
                             int64_t row_bytes, int positions, hipStream_t stream) {
    if (rows <= 0 || positions <= 0) return hipSuccess;
    const dim3 grid((rows + kRowsPerGroup - 1) / kRowsPerGroup, (positions + kPositions - 1) / kPositions);
    if (format == kQ4_K)
        gemv_kmfma_kernel<kQ4_K><<<grid, kThreads, 0, stream>>>(w, act, y, rows, blocks, row_bytes, positions);
    else if (format == kQ6_K)
        gemv_kmfma_kernel<kQ6_K><<<grid, kThreads, 0, stream>>>(w, act, y, rows, blocks, row_bytes, positions);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace satori
