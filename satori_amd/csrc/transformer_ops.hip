// Decode-step operators around the projections, on the device: TransformerOps (src/Satori.Core/TransformerOps.cs)
// and the embedding-row decode of GgufQuantizedMatrix.ReadRow (src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:54-61,
// QuantizedRow.DecodeRow, src/Satori.Core/QuantizedRow.cs:59-70).
//
// The reference computes these in FP64 and rounds each output to FP32 once; the kernels do the same, with
// every FP64 operation written as the reference writes it (no contraction: the library is compiled with
// -ffp-contract=off). Where the reference sums sequentially and a kernel reduces in a tree (the RMS sums of
// squares, the softmax denominator), or where exp / sin / cos / pow come from the device math library, the
// FP64 intermediate can differ in its last bits; the FP32 outputs then agree to about one unit in the last
// place. The row decode and Add are FP32 expressions of the reference and agree bit for bit.
#include <algorithm>
#include <cmath>

#include "device_common.hpp"
#include "kernels.hpp"
#include "ops_device.hpp"
#include "q8k_device.hpp"

// Split-attention partials of the no-allocation entry point: one copy per device, alive until the process
// ends, shared by every such call on that device (calls that overlap in time race on it). Host code never
// names it in a launch: the device address comes from hipGetSymbolAddress (static_attention_partials).
static __device__ __align__(256) unsigned char scratch[satori::kStaticAttentionBytes];

namespace satori {
namespace {

constexpr int kThreads = kOpsThreads;

__device__ __forceinline__ double block_sum(double v, double* red) { return block_sum_256(v, red); }

__device__ __forceinline__ double block_max(double v, double* red) { return block_tree_256(v, red, true); }

// RmsNorm (TransformerOps.cs:13-21), one workgroup per vector of `length`; output may equal input.
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const float* x, const float* __restrict__ w, float epsilon,
                                                            int length, float* y) {
    __shared__ double red[kThreads];
    const float* xv = x + static_cast<int64_t>(blockIdx.x) * length;
    float* yv = y + static_cast<int64_t>(blockIdx.x) * length;
    double part = 0;
    for (int i = threadIdx.x; i < length; i += kThreads) {
        const double v = xv[i];
        part = part + v * v;
    }
    const double scale = rms_scale(block_sum(part, red), length, epsilon);
    for (int i = threadIdx.x; i < length; i += kThreads) yv[i] = rms_value(xv[i], scale, w[i]);
}

// Add then RmsNorm (DenseForward.cs:156-158 and :149 of the next layer): residual += addend in FP32, then the
// RmsNorm of the new residual into `normed`. The per-thread partition and the reduction tree are those of
// rms_norm_kernel, so the outputs equal the two separate calls bit for bit.
__global__ __launch_bounds__(kThreads) void add_rms_norm_kernel(float* residual, const float* addend,
                                                                const float* __restrict__ w, float epsilon, int length,
                                                                float* normed) {
    __shared__ double red[kThreads];
    double part = 0;
    for (int i = threadIdx.x; i < length; i += kThreads) {
        const float r = __fadd_rn(residual[i], addend[i]);
        residual[i] = r;
        const double v = r;
        part = part + v * v;
    }
    const double scale = rms_scale(block_sum(part, red), length, epsilon);
    for (int i = threadIdx.x; i < length; i += kThreads) normed[i] = rms_value(residual[i], scale, w[i]);
}

// Add then RmsNorm as add_rms_norm_kernel, the normalised row also written as Q8_K bytes
// (Q8KCodec.QuantizeRow) for the projection that reads it: the same partition, tree and per-element
// expressions, then one wave per 256-element block quantizes the normalised values from the summed row
// kept in LDS, so `normed` equals add_rms_norm_kernel's and `q8k` the quantizer's bytes of it, bit for bit.
constexpr int kNormQ8KStaged = 12288;  // longest row kept in LDS (48 KB); longer rows take two launches
__global__ __launch_bounds__(kThreads) void add_rms_norm_q8k_kernel(float* residual, const float* addend,
                                                                    const float* __restrict__ w, float epsilon,
                                                                    int length, float* normed,
                                                                    uint8_t* __restrict__ q8k) {
    __shared__ double red[kThreads];
    extern __shared__ float summed[];  // length floats
    double part = 0;
    for (int i = threadIdx.x; i < length; i += kThreads) {
        const float r = __fadd_rn(residual[i], addend[i]);
        residual[i] = r;
        summed[i] = r;
        const double v = r;
        part = part + v * v;
    }
    const double scale = rms_scale(block_sum(part, red), length, epsilon);  // its barriers publish `summed`
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int b = wave; b < length / 256; b += kThreads / 64) {
        const int i0 = 256 * b + 4 * lane;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = rms_value(summed[i0 + e], scale, w[i0 + e]);
            normed[i0 + e] = v[e];
        }
        const Q8KLane q = q8k_quantize_values(v, lane);
        uint8_t* dst = q8k + static_cast<int64_t>(b) * kQ8KBlockBytes;
        if (q.zero) {
            uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
            for (int i = lane; i < kQ8KBlockBytes / 4; i += 64) d32[i] = 0u;
            continue;
        }
        reinterpret_cast<uint32_t*>(dst + 4)[lane] = q.packed;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(dst + 260)[lane >> 2] = static_cast<int16_t>(q.group_sum);
        if (lane == 0) reinterpret_cast<float*>(dst)[0] = q.scale;
    }
}

// The attention inputs of one decode position (DenseForward.cs:128-151): q += q_bias and k + k_bias,
// v + v_bias (when the biases are given), then RopeHalf of q and of the key, the key and value written to
// their cache slots. Same per-element operations as Add and RopeHalf, so the outputs equal the separate
// calls bit for bit. Threads: q pairs, key pairs, then the unrotated q and key lanes, then the values.
__device__ __forceinline__ float biased(const float* x, const float* bias, int i) {
    return bias ? __fadd_rn(x[i], bias[i]) : x[i];
}

// RopeHalf of lane pair (kk, kk + rotary / 2) of one head (TransformerOps.cs:94-114): the angle
// position / base^(2 kk / rotary) in FP64, then both rotated lanes in FP64, each rounded once.
__device__ __forceinline__ void rope_angle(int kk, int position, double base, int rotary, double& sn, double& cs) {
    const double angle = position / pow(base, 2.0 * kk / rotary);
    sn = sin(angle);
    cs = cos(angle);
}

__device__ __forceinline__ void rope_apply(double x, double y, double sn, double cs, float& a, float& b) {
    a = static_cast<float>(x * cs - y * sn);
    b = static_cast<float>(x * sn + y * cs);
}

__device__ __forceinline__ void rope_pair(double x, double y, int kk, int position, double base, int rotary, float& a,
                                          float& b) {
    double sn, cs;
    rope_angle(kk, position, base, rotary, sn, cs);
    rope_apply(x, y, sn, cs, a, b);
}

__global__ __launch_bounds__(kThreads) void attention_inputs_kernel(float* q, const float* q_bias, const float* k,
                                                                    const float* k_bias, float* k_out, const float* v,
                                                                    const float* v_bias, float* v_out, int heads,
                                                                    int kv_heads, int head_dim, int position,
                                                                    double base, int rotary) {
    const int pairs = rotary / 2, pass = head_dim - rotary;
    const int64_t qp = static_cast<int64_t>(heads) * pairs, kp = static_cast<int64_t>(kv_heads) * pairs;
    const int64_t qr = static_cast<int64_t>(heads) * pass, kr = static_cast<int64_t>(kv_heads) * pass;
    const int64_t vw = static_cast<int64_t>(kv_heads) * head_dim;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < qp + kp) {
        const bool is_q = i < qp;
        const int64_t index = is_q ? i : i - qp;
        const int head = static_cast<int>(index / pairs), kk = static_cast<int>(index % pairs);
        const int a = head * head_dim + kk, b = a + pairs;
        const float x = is_q ? biased(q, q_bias, a) : biased(k, k_bias, a);
        const float y = is_q ? biased(q, q_bias, b) : biased(k, k_bias, b);
        float* dst = is_q ? q : k_out;
        rope_pair(x, y, kk, position, base, rotary, dst[a], dst[b]);
        return;
    }
    i -= qp + kp;
    if (i < qr + kr) {  // lanes past the rotary dimensions pass through (biased)
        const bool is_q = i < qr;
        const int64_t index = is_q ? i : i - qr;
        const int head = static_cast<int>(index / pass), lane = rotary + static_cast<int>(index % pass);
        const int e = head * head_dim + lane;
        if (is_q)
            q[e] = biased(q, q_bias, e);
        else
            k_out[e] = biased(k, k_bias, e);
        return;
    }
    i -= qr + kr;
    if (i < vw) v_out[i] = biased(v, v_bias, static_cast<int>(i));
}

// RmsNormHeads (TransformerOps.cs:117-130): one workgroup per head, in place.
__global__ __launch_bounds__(kThreads) void rms_norm_heads_kernel(float* v, const float* __restrict__ w, float epsilon,
                                                                  int head_dim) {
    __shared__ double red[kThreads];
    float* hv = v + static_cast<int64_t>(blockIdx.x) * head_dim;
    double part = 0;
    for (int i = threadIdx.x; i < head_dim; i += kThreads) {
        const double e = hv[i];
        part = part + e * e;
    }
    const double sum = block_sum(part, red);
    const double scale = 1.0 / __dsqrt_rn(sum / head_dim + static_cast<double>(epsilon));
    for (int i = threadIdx.x; i < head_dim; i += kThreads)
        hv[i] = static_cast<float>(static_cast<double>(hv[i]) * scale * static_cast<double>(w[i]));
}

// Rope (TransformerOps.cs:23-38, pairs (j, j + 1)) and RopeHalf (:94-114, pairs (k, k + half) of the first
// `rotary` lanes): one thread per (head, pair).
__global__ __launch_bounds__(kThreads) void rope_kernel(float* v, int heads, int head_dim, int position, double base,
                                                        int rotary, int half_split) {
    const int pairs = rotary / 2;
    const int64_t index = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (index >= static_cast<int64_t>(heads) * pairs) return;
    const int head = static_cast<int>(index / pairs), k = static_cast<int>(index % pairs);
    double angle;
    int a, b;
    if (half_split) {
        angle = position / pow(base, 2.0 * k / rotary);
        a = k;
        b = k + pairs;
    } else {
        const int j = 2 * k;
        angle = position / pow(10000.0, static_cast<double>(j) / head_dim);
        a = j;
        b = j + 1;
    }
    const double sn = sin(angle), cs = cos(angle);
    float* hv = v + static_cast<int64_t>(head) * head_dim;
    const double x = hv[a], y = hv[b];
    hv[a] = static_cast<float>(x * cs - y * sn);
    hv[b] = static_cast<float>(x * sn + y * cs);
}

// SwiGlu (TransformerOps.cs:40-50) and Add (:52-57), elementwise; output may equal an input.
__global__ __launch_bounds__(kThreads) void swiglu_kernel(const float* gate, const float* up, int length, float* out) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= length) return;
    out[i] = swiglu_value(gate[i], up[i]);
}

// The RoPE angles' sines and cosines of `positions` positions (rope_angle, the same FP64 values the rotation
// kernels compute): row p holds the rotary / 2 sines, then the cosines.
__global__ __launch_bounds__(kThreads) void rope_table_kernel(int positions, int rotary, double base, double* table) {
    const int pairs = rotary / 2;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= static_cast<int64_t>(positions) * pairs) return;
    const int p = static_cast<int>(i / pairs), kk = static_cast<int>(i % pairs);
    double* row = table + static_cast<int64_t>(p) * rotary;
    rope_angle(kk, p, base, rotary, row[kk], row[pairs + kk]);
}

// SwiGlu of one 256-element block per wave (four consecutive elements per lane), then the block's Q8_K bytes
// (Q8KCodec.QuantizeBlock, the quantizer the integer products use): the down projection's activation
// quantized once by its producer. The FP32 outputs equal swiglu_kernel's.
__global__ __launch_bounds__(64) void swiglu_q8k_kernel(const float* gate, const float* up, float* out,
                                                        uint8_t* __restrict__ q8k) {
    const int block = blockIdx.x, lane = threadIdx.x;
    const int i0 = 256 * block + 4 * lane;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = swiglu_value(gate[i0 + i], up[i0 + i]);
    if (out)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i0 + i] = v[i];
    const Q8KLane q = q8k_quantize_values(v, lane);
    uint8_t* dst = q8k + static_cast<int64_t>(block) * kQ8KBlockBytes;
    if (q.zero) {
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
        for (int i = lane; i < kQ8KBlockBytes / 4; i += 64) d32[i] = 0u;
        return;
    }
    reinterpret_cast<uint32_t*>(dst + 4)[lane] = q.packed;
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(dst + 260)[lane >> 2] = static_cast<int16_t>(q.group_sum);
    if (lane == 0) reinterpret_cast<float*>(dst)[0] = q.scale;
}

__global__ __launch_bounds__(kThreads) void add_kernel(const float* left, const float* right, int length, float* out) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= length) return;
    out[i] = __fadd_rn(left[i], right[i]);
}

// GroupedAttention (TransformerOps.cs:135-179): one workgroup of 1024 threads per query head. Scores: one
// thread per token, the dot product over the head lanes in the reference's order (the query staged in LDS,
// the key row read in 16-byte loads). The maximum is exact; the exponentials and their total are FP64, and the reference's
// weight of token t, scores[t] / total, is formed once per token. Output: lane j of the head is summed over
// eight token groups (threads j + 128 g), whose FP64 partial sums are added in group order. The FP64
// reassociations stay far below the FP32 output's last place.
constexpr int kAttnThreads = 1024;
constexpr int kAttnGroups = kAttnThreads / 128;  // token groups of the output sums (head_dim <= 128 per pass)

__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                                 const float* __restrict__ v, int query_heads,
                                                                 int kv_heads, int head_dim, int tokens,
                                                                 float* __restrict__ out) {
    extern __shared__ double scores[];  // tokens
    __shared__ double red[kAttnThreads];
    const int head = blockIdx.x;
    const int kv_head = head / (query_heads / kv_heads);
    const int kv_width = kv_heads * head_dim;
    const float* qh = q + static_cast<int64_t>(head) * head_dim;
    const double scale = 1.0 / __dsqrt_rn(static_cast<double>(head_dim));
    __shared__ float qs[512];  // the head's query lanes (head_dim <= 512 staged; wider heads read global)
    for (int j = threadIdx.x; j < head_dim && j < 512; j += kAttnThreads) qs[j] = qh[j];
    __syncthreads();
    const bool staged = head_dim <= 512 && (head_dim & 3) == 0;  // 16-byte loads need 4-byte alignment only
    for (int t = threadIdx.x; t < tokens; t += kAttnThreads) {
        const float* kt = k + static_cast<int64_t>(t) * kv_width + kv_head * head_dim;
        double dot = 0;
        if (staged) {
            // The token's key row in 16-byte loads, eight in flight; the dot product in lane order.
            for (int j0 = 0; j0 < head_dim; j0 += 32) {
                f32x4 kv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (j0 + 4 * i < head_dim) {
                        const u32x4 raw = load16_a4(reinterpret_cast<const uint8_t*>(kt + j0 + 4 * i));
                        kv[i] = f32x4{__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                                      __uint_as_float(raw[3])};
                    }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (j0 + 4 * i >= head_dim) break;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        dot = dot + static_cast<double>(qs[j0 + 4 * i + e]) * static_cast<double>(kv[i][e]);
                }
            }
        } else {
            for (int j = 0; j < head_dim; ++j) dot = dot + static_cast<double>(qh[j]) * static_cast<double>(kt[j]);
        }
        scores[t] = dot * scale;
    }
    __syncthreads();
    double local_max = -INFINITY;
    for (int t = threadIdx.x; t < tokens; t += kAttnThreads) local_max = fmax(local_max, scores[t]);
    red[threadIdx.x] = local_max;
    __syncthreads();
    for (int s = kAttnThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const double max = red[0];
    __syncthreads();
    double part = 0;
    for (int t = threadIdx.x; t < tokens; t += kAttnThreads) {
        const double e = exp(scores[t] - max);
        scores[t] = e;
        part = part + e;
    }
    red[threadIdx.x] = part;
    __syncthreads();
    for (int s = kAttnThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + s];
        __syncthreads();
    }
    const double total = red[0];
    __syncthreads();
    for (int t = threadIdx.x; t < tokens; t += kAttnThreads) scores[t] = scores[t] / total;
    __syncthreads();
    const int per_group = (tokens + kAttnGroups - 1) / kAttnGroups;
    for (int j0 = 0; j0 < head_dim; j0 += 128) {
        const int j = j0 + (threadIdx.x & 127), group = threadIdx.x >> 7;
        double sum = 0;
        if (j < head_dim) {
            const int t_end = min(tokens, (group + 1) * per_group);
            const float* vj = v + kv_head * head_dim + j;
            int t = group * per_group;
            for (; t + 8 <= t_end; t += 8) {  // eight loads in flight, then the sums in token order
                float vt[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) vt[i] = vj[static_cast<int64_t>(t + i) * kv_width];
#pragma unroll
                for (int i = 0; i < 8; ++i) sum = sum + scores[t + i] * static_cast<double>(vt[i]);
            }
            for (; t < t_end; ++t) sum = sum + scores[t] * static_cast<double>(vj[static_cast<int64_t>(t) * kv_width]);
        }
        red[threadIdx.x] = sum;
        __syncthreads();
        if (threadIdx.x < 128 && j < head_dim) {
            double total_j = 0;
#pragma unroll
            for (int g = 0; g < kAttnGroups; ++g) total_j = total_j + red[threadIdx.x + 128 * g];
            out[static_cast<int64_t>(head) * head_dim + j] = static_cast<float>(total_j);
        }
        __syncthreads();
    }
}

// The same attention split over the key/value tokens (flash-decoding), for the long prefixes a single
// workgroup per head would stream through one CU: workgroup (head, split) computes its tokens' scores, their
// maximum m, the exponentials e_t = exp(score_t - m), their total l and the unnormalised sums
// o_j = sum_t e_t * v_tj, all FP64; the combine kernel rescales each split by exp(m_split - M) with M the
// head's maximum and divides by the rescaled total. Against the reference's softmax-then-sum this
// reassociates FP64 operations only (far below the FP32 output's last place). Any prefix length and head
// width: up to 32 splits of at least 32 tokens, up to 64 of at least 128 beyond 4,096 tokens, and more
// splits once a split would exceed 2,048 tokens (its exponentials stay in LDS).
constexpr int kSplitThreads = 256;
constexpr int kMinSplits = 32;         // splits of a prefix of up to 4,096 tokens
constexpr int kLongSplits = 64;        // splits of a longer prefix before the per-split token bound applies
constexpr int kMaxSplitTokens = 2048;  // tokens of one split (its FP64 exponentials in LDS: 16 KB)
constexpr int kMaxSplitsPerLaunch = 65535;
constexpr int kStagedQuery = 8192;     // query lanes staged in LDS; wider heads read the query from global memory
constexpr int kCombineChunk = 16;      // splits whose values one combine thread loads at a time
constexpr int kCombineWeights = 1024;  // split weights the combine kernel holds in LDS at a time

// Workgroup reduction of THREADS doubles (256: block_tree_256; 512: each of the first 64 threads first folds
// its eight values in thread order, then the same shuffle tree), every thread getting the result.
template <int THREADS>
__device__ __forceinline__ double split_reduce(double v, double* red, bool take_max) {
    if constexpr (THREADS == 256) {
        return block_tree_256(v, red, take_max);
    } else {
        static_assert(THREADS == 512, "split workgroups of 256 or 512 threads");
        const int t = threadIdx.x;
        auto op = [take_max](double a, double b) { return take_max ? fmax(a, b) : a + b; };
        red[t] = v;
        __syncthreads();
        if (t < 64) {
            double x = red[t];
#pragma unroll
            for (int k = 1; k < THREADS / 64; ++k) x = op(x, red[t + 64 * k]);
#pragma unroll
            for (int s2 = 32; s2 > 0; s2 >>= 1) x = op(x, __shfl_down(x, s2, 64));
            if (t == 0) red[0] = x;
        }
        __syncthreads();
        const double r = red[0];
        __syncthreads();
        return r;
    }
}

// Workgroup reduction of 256 doubles through wave shuffles and four partials in LDS (every thread gets it).
__device__ __forceinline__ double wave_reduce_256(double v, double* red4, bool take_max) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const double other = __shfl_xor(v, o, 64);
        v = take_max ? fmax(v, other) : v + other;
    }
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = red4[0];
#pragma unroll
    for (int i = 1; i < kSplitThreads / 64; ++i) r = take_max ? fmax(r, red4[i]) : r + red4[i];
    __syncthreads();
    return r;
}

// The attention inputs of the decoded position, applied inside the split attention (DecodeInputs): the query
// biased and rotated while it is staged, the new key and value (row `position`, the prefix's last) formed by
// the workgroups whose split holds that row and written to their cache slots by one of them.
struct DecodeInputs {
    const float* q_bias;
    const float* k_new;
    const float* k_bias;
    const float* v_new;
    const float* v_bias;
    const double* rope;  // the position's sines then cosines (launch_rope_table), or null: computed here
    int position;
    int rotary;
    double base;
};

// Units (key/value head, split), dealt to the 8 XCDs round-robin; each XCD runs its units' query heads on
// consecutive workgroups of its own: workgroup w is slot w / 8 of XCD w % 8, slot k serving query head k % group
// of the XCD's unit k / group. The grid has 8 * ceil(units / 8) * group workgroups; those past the last unit
// return false.
__device__ __forceinline__ bool split_unit(int w, int group, int kv_heads, int splits, int& head, int& split) {
    const int xcd = w & 7, k = w >> 3;
    const int unit = (k / group) * 8 + xcd;
    if (unit >= kv_heads * splits) return false;
    const int kv_head = unit / splits;
    split = unit - kv_head * splits;
    head = kv_head * group + k % group;
    return true;
}

int split_grid(int query_heads, int kv_heads, int splits) {
    const int group = query_heads / kv_heads;
    return 8 * ((kv_heads * splits + 7) / 8) * group;
}

template <bool INPUTS, int THREADS>
__global__ __launch_bounds__(THREADS) void attention_split_kernel(const float* __restrict__ q,
                                                                        const float* __restrict__ k,
                                                                        const float* __restrict__ v, int query_heads,
                                                                        int kv_heads, int head_dim, int tokens, int per,
                                                                        int splits, double* __restrict__ partial,
                                                                        DecodeInputs in, float* k_cache, float* v_cache) {
    extern __shared__ double es[];  // this split's exponentials (per), then the staged query lanes
    __shared__ double red[THREADS];
    // Workgroup -> (query head, split): the query heads that share a key/value head and a split run on one
    // XCD (workgroup ids are dealt to the 8 XCDs round-robin), so that XCD's L2 fetches their key and value
    // rows once for all of them (split_unit).
    const int group = query_heads / kv_heads;
    int head, split;
    if (!split_unit(blockIdx.x, group, kv_heads, splits, head, split)) return;  // whole workgroup
    const int t0 = static_cast<int>(min(static_cast<int64_t>(split) * per, static_cast<int64_t>(tokens)));
    const int t1 = min(tokens, t0 + per);
    const int kv_head = head / group;
    const int kv_width = kv_heads * head_dim;
    const double scale = 1.0 / __dsqrt_rn(static_cast<double>(head_dim));
    const float* qh = q + static_cast<int64_t>(head) * head_dim;
    float* qs = reinterpret_cast<float*>(es + per);
    const bool staged = head_dim <= kStagedQuery;
    const float* qsrc = staged ? qs : qh;
    // With the inputs fused, the new row (the last token) is held in LDS, not read from the cache.
    const bool has_new = INPUTS && t0 <= in.position && in.position < t1;
    float* ks_new = qs + head_dim;
    float* vs_new = ks_new + head_dim;
    // With the inputs fused (heads of at most 256 lanes), thread j owns lane j of the head: it loads what the
    // transformed query lane needs (and, where the new row lives, the key and value lanes) before anything
    // else, then rotates them after the cache loads below are issued.
    // Every thread issues the same loads (lane indices clamped, absent operands replaced by present ones whose
    // values are then unused), so the waits below are counted statically and do not cover the cache loads.
    const int pairs = in.rotary / 2, jl = min(static_cast<int>(threadIdx.x), head_dim - 1);
    const bool rot = jl < in.rotary;
    const int kk = jl < pairs ? jl : (rot ? jl - pairs : 0);
    const int ia = rot ? kk : jl, ib = rot ? kk + pairs : jl;  // the lane pair read (one lane past the rotation)
    float qx = 0.0f, qy = 0.0f, qxb = 0.0f, qyb = 0.0f, kx = 0.0f, ky = 0.0f, kxb = 0.0f, kyb = 0.0f;
    float vl = 0.0f, vlb = 0.0f;
    double sn = 0.0, cs = 0.0;
    if (INPUTS) {
        const int qb = head * head_dim;
        const float* qbias = in.q_bias ? in.q_bias : q;
        const double* rope = in.rope ? in.rope : partial;
        qx = q[qb + ia];
        qy = q[qb + ib];
        qxb = qbias[qb + ia];
        qyb = qbias[qb + ib];
        sn = rope[kk];
        cs = rope[pairs + kk];
    }
    // The first 16 values of this thread's output lane and token part are loaded before anything else, so
    // they arrive while the scores are computed. Lane j of the head is summed in THREADS / 128 consecutive
    // token parts (threads j, j + 128, ...).
    constexpr int kParts = THREADS / 128;
    const int count = t1 - t0, half = (count + kParts - 1) / kParts;
    const int vj0 = threadIdx.x & 127, vgroup = threadIdx.x >> 7;
    const int va = t0 + vgroup * half, vb = min(t1, va + half);
    const bool v_new_here = has_new && vb == t1 && va < vb;  // this token part ends with the new row
    const int vbc = v_new_here ? vb - 1 : vb;                // the part's rows read from the cache
    float vpre[16];
    if (vj0 < head_dim) {
        const float* vj = v + kv_head * head_dim + vj0;
#pragma unroll
        for (int i = 0; i < 16; ++i) vpre[i] = va + i < vbc ? vj[static_cast<int64_t>(va + i) * kv_width] : 0.0f;
    }
    // Key quads of this thread's first score (heads of up to 128 lanes: its whole eighth), also loaded before
    // the query is staged.
    const bool quads = (head_dim & 31) == 0;
    const int piece = (head_dim + 7) / 8, p8 = threadIdx.x & 7;
    const int j_lo = min(head_dim, p8 * piece), j_hi = min(head_dim, j_lo + piece);
    const int ts = has_new ? t1 - 1 : t1;  // scores of cached rows
    const bool kfirst = quads && piece <= 16 && t0 + (threadIdx.x >> 3) < ts;
    f32x4 kpre[4];
    if (kfirst) {
        const float* kp = k + static_cast<int64_t>(t0 + (threadIdx.x >> 3)) * kv_width + kv_head * head_dim + j_lo;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * i < piece) {
                const u32x4 raw = load16_a4(reinterpret_cast<const uint8_t*>(kp + 4 * i));
                kpre[i] = f32x4{__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                                __uint_as_float(raw[3])};
            }
    }
    if (INPUTS && has_new) {  // the new row's key and value lanes, in the workgroups whose split holds it
        const int kb = kv_head * head_dim;
        kx = in.k_new[kb + ia];
        ky = in.k_new[kb + ib];
        if (in.k_bias) {
            kxb = in.k_bias[kb + ia];
            kyb = in.k_bias[kb + ib];
        }
        vl = in.v_new[kb + jl];
        if (in.v_bias) vlb = in.v_bias[kb + jl];
    }
    if (INPUTS) {
        if (static_cast<int>(threadIdx.x) < head_dim) {
            // The attention-input transform of lane j (as attention_inputs_kernel: biased, then rotated).
            if (rot && !in.rope) rope_angle(kk, in.position, in.base, in.rotary, sn, cs);
            auto lane = [&](float x, float y, float xb, float yb, bool bias) {
                const float xv = bias ? __fadd_rn(x, xb) : x, yv = bias ? __fadd_rn(y, yb) : y;
                if (!rot) return xv;
                float a, b;
                rope_apply(xv, yv, sn, cs, a, b);
                return jl < pairs ? a : b;
            };
            const float qj = lane(qx, qy, qxb, qyb, in.q_bias != nullptr);
            qs[jl] = qj;
            if (split == 0) {  // the rotated query, for the combine launch to store in place
                float* q_rot =
                    reinterpret_cast<float*>(partial + static_cast<int64_t>(query_heads) * splits * (2 + head_dim));
                q_rot[head * head_dim + jl] = qj;
            }
            if (has_new) {
                const float kj = lane(kx, ky, kxb, kyb, in.k_bias != nullptr);
                const float vj = in.v_bias ? __fadd_rn(vl, vlb) : vl;
                ks_new[jl] = kj;
                vs_new[jl] = vj;
                if (head % group == 0) {  // one workgroup of the key/value head writes the cache row
                    k_cache[static_cast<int64_t>(in.position) * kv_width + kv_head * head_dim + jl] = kj;
                    v_cache[static_cast<int64_t>(in.position) * kv_width + kv_head * head_dim + jl] = vj;
                }
            }
        }
    } else if (staged) {
        for (int j = threadIdx.x; j < head_dim; j += THREADS) qs[j] = qh[j];
    }
    __syncthreads();
    // Scores: eight threads per token, thread p summing lanes [p * piece, (p + 1) * piece) of the key row in
    // order (16-byte loads, all in flight, when the eighths are whole quads), the eight partial sums then
    // added in order.
    double local_max = -INFINITY;
    for (int base = t0; base < ts; base += THREADS / 8) {
        const int t = base + (threadIdx.x >> 3);
        double dot = 0;
        if (t < ts) {
            const float* kt = k + static_cast<int64_t>(t) * kv_width + kv_head * head_dim;
            if (quads) {
                const float* kp = kt + j_lo;
                const float* qp = qsrc + j_lo;
                for (int j0 = 0; j0 < piece; j0 += 16) {
                    f32x4 kv[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (base == t0 && kfirst)
                            kv[i] = kpre[i];
                        else if (j0 + 4 * i < piece) {
                            const u32x4 raw = load16_a4(reinterpret_cast<const uint8_t*>(kp + j0 + 4 * i));
                            kv[i] = f32x4{__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                                          __uint_as_float(raw[3])};
                        }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (j0 + 4 * i >= piece) break;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            dot = dot + static_cast<double>(qp[j0 + 4 * i + e]) * static_cast<double>(kv[i][e]);
                    }
                }
            } else {
                for (int j = j_lo; j < j_hi; ++j) dot = dot + static_cast<double>(qsrc[j]) * static_cast<double>(kt[j]);
            }
        }
        red[threadIdx.x] = dot;
        __syncthreads();
        if (p8 == 0 && t < ts) {
            double total = red[threadIdx.x];
#pragma unroll
            for (int i = 1; i < 8; ++i) total = total + red[threadIdx.x + i];
            const double sc = total * scale;
            es[t - t0] = sc;
            local_max = fmax(local_max, sc);
        }
        __syncthreads();
    }
    if (INPUTS && has_new) {
        // The new row's score, by eight threads over the same lane ranges, in the same order, as a cached row.
        double dot = 0;
        if (threadIdx.x < 8)
            for (int j = j_lo; j < j_hi; ++j) dot = dot + static_cast<double>(qsrc[j]) * static_cast<double>(ks_new[j]);
        red[threadIdx.x] = dot;
        __syncthreads();
        if (threadIdx.x == 0) {
            double total = red[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) total = total + red[i];
            const double sc = total * scale;
            es[t1 - 1 - t0] = sc;
            local_max = fmax(local_max, sc);
        }
        __syncthreads();
    }
    const double m = split_reduce<THREADS>(local_max, red, true);
    double part = 0;
    for (int t = t0 + threadIdx.x; t < t1; t += THREADS) {
        const double e = exp(es[t - t0] - m);
        es[t - t0] = e;
        part = part + e;
    }
    const double l = split_reduce<THREADS>(part, red, false);
    double* out = partial + (static_cast<int64_t>(head) * splits + split) * (2 + head_dim);
    if (threadIdx.x == 0) {
        out[0] = m;
        out[1] = l;
    }
    // Unnormalised sums: lane j of the head over its token parts (threads j, j + 128, ...), added in order.
    for (int j0 = 0; j0 < head_dim; j0 += 128) {
        const int j = j0 + vj0;
        double sum = 0;
        if (j < head_dim) {
            const float* vj = v + kv_head * head_dim + j;
            int t = va;
            if (j0 == 0) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (va + i < vbc) sum = sum + es[va + i - t0] * static_cast<double>(vpre[i]);
                t = min(vbc, va + 16);
            }
            for (; t + 16 <= vbc; t += 16) {
                float vt[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) vt[i] = vj[static_cast<int64_t>(t + i) * kv_width];
#pragma unroll
                for (int i = 0; i < 16; ++i) sum = sum + es[t + i - t0] * static_cast<double>(vt[i]);
            }
            for (; t < vbc; ++t) sum = sum + es[t - t0] * static_cast<double>(vj[static_cast<int64_t>(t) * kv_width]);
            if (v_new_here) sum = sum + es[t1 - 1 - t0] * static_cast<double>(vs_new[j]);  // the last row, last
        }
        red[threadIdx.x] = sum;
        __syncthreads();
        if (threadIdx.x < 128 && j < head_dim) {
            double total = red[threadIdx.x] + red[threadIdx.x + 128];
#pragma unroll
            for (int k = 2; k < kParts; ++k) total = total + red[threadIdx.x + 128 * k];
            out[2 + j] = total;
        }
        __syncthreads();
    }
}

// One workgroup per head. The head's maximum M over the splits' maxima and the rescaled total
// sum_s exp(m_s - M) l_s are workgroup reductions (each thread takes a strided share of the splits, then wave
// shuffles); the splits' weights exp(m_s - M) are formed once per split into LDS. Output lane j is summed over
// the splits in split order by `lanes_per` threads, each over a contiguous share of the splits with 16 loads
// in flight, their partial sums then added in share order, and divided by the total.
template <bool INPUTS>
__global__ __launch_bounds__(kSplitThreads) void attention_combine_kernel(const double* __restrict__ partial,
                                                                          int splits, int head_dim,
                                                                          float* __restrict__ out, float* q,
                                                                          DecodeInputs in) {
    if (INPUTS) {
        // The query rotated in place, as the separate attention-inputs launch leaves it (the split workgroups
        // have all read the original by now): split 0 of each head left it after the partials.
        const float* q_rot =
            reinterpret_cast<const float*>(partial + static_cast<int64_t>(gridDim.x) * splits * (2 + head_dim));
        for (int j = threadIdx.x; j < head_dim; j += kSplitThreads)
            q[blockIdx.x * head_dim + j] = q_rot[blockIdx.x * head_dim + j];
    }
    __shared__ double weight[kCombineWeights];
    __shared__ double lane_part[kSplitThreads];
    __shared__ double red4[kSplitThreads / 64];
    const int head = blockIdx.x;
    const int64_t stride = 2 + head_dim;
    const double* p = partial + static_cast<int64_t>(head) * splits * stride;
    // Threads per output lane: up to 8 while the head's lanes fit the workgroup that many times.
    int lanes_per = 1;
    while (lanes_per < 8 && 2 * lanes_per * head_dim <= kSplitThreads) lanes_per *= 2;
    const int width = kSplitThreads / lanes_per;
    const int share = threadIdx.x / width;
    const int split_share = (splits + lanes_per - 1) / lanes_per;  // splits per thread of an output lane
    if (splits <= kSplitThreads && head_dim <= width && split_share <= kCombineChunk) {
        // A decode-sized head (one split per thread, one pass over the lanes): every global read is issued
        // before the first reduction, so the kernel waits on memory once. The same operations in the same
        // order as the general path below.
        const int j = threadIdx.x % width;
        const int s_lo = min(splits, share * split_share), s_hi = min(splits, s_lo + split_share);
        double m_s = -INFINITY, l_s = 0.0;
        if (threadIdx.x < splits) {
            m_s = p[threadIdx.x * stride];
            l_s = p[threadIdx.x * stride + 1];
        }
        double o[kCombineChunk];
#pragma unroll
        for (int i = 0; i < kCombineChunk; ++i)
            o[i] = j < head_dim && s_lo + i < s_hi ? p[(s_lo + i) * stride + 2 + j] : 0.0;
        const double m = wave_reduce_256(m_s, red4, true);
        double total_part = 0;
        if (threadIdx.x < splits) {
            const double w = l_s > 0 ? exp(m_s - m) : 0.0;
            weight[threadIdx.x] = w;
            total_part = total_part + w * l_s;
        }
        const double total = wave_reduce_256(total_part, red4, false);  // its barrier publishes the weights
        double sum = 0;
#pragma unroll
        for (int i = 0; i < kCombineChunk; ++i)
            if (s_lo + i < s_hi) sum = sum + weight[s_lo + i] * o[i];
        lane_part[threadIdx.x] = sum;
        __syncthreads();
        if (share == 0 && j < head_dim) {
            double lane_sum = lane_part[threadIdx.x];
            for (int i = 1; i < lanes_per; ++i) lane_sum = lane_sum + lane_part[threadIdx.x + i * width];
            out[static_cast<int64_t>(head) * head_dim + j] = static_cast<float>(lane_sum / total);
        }
        return;
    }
    double big = -INFINITY;
    for (int s = threadIdx.x; s < splits; s += kSplitThreads) big = fmax(big, p[s * stride]);
    big = wave_reduce_256(big, red4, true);
    const int chunks = (splits + kCombineWeights - 1) / kCombineWeights;
    double total_part = 0;
    double total = 0;
    for (int j0 = 0; j0 < head_dim; j0 += width) {
        const int j = j0 + threadIdx.x % width;
        double sum = 0;
        for (int chunk = 0; chunk < chunks; ++chunk) {
            const int c0 = chunk * kCombineWeights, n = min(kCombineWeights, splits - c0);
            if (chunks > 1 || j0 == 0) {  // this chunk's weights (once when they all fit)
                __syncthreads();           // the previous chunk's weights are no longer read
                for (int s = threadIdx.x; s < n; s += kSplitThreads) {
                    const double* ps = p + (c0 + s) * stride;
                    const double w = ps[1] > 0 ? exp(ps[0] - big) : 0.0;
                    weight[s] = w;
                    if (j0 == 0) total_part = total_part + w * ps[1];
                }
                __syncthreads();
            }
            if (j < head_dim) {
                const int each = (n + lanes_per - 1) / lanes_per;
                const int s_lo = min(n, share * each), s_hi = min(n, s_lo + each);
                for (int s0 = s_lo; s0 < s_hi; s0 += kCombineChunk) {
                    double o[kCombineChunk];
#pragma unroll
                    for (int i = 0; i < kCombineChunk; ++i) o[i] = s0 + i < s_hi ? p[(c0 + s0 + i) * stride + 2 + j] : 0.0;
#pragma unroll
                    for (int i = 0; i < kCombineChunk; ++i)
                        if (s0 + i < s_hi) sum = sum + weight[s0 + i] * o[i];
                }
            }
        }
        if (j0 == 0) total = wave_reduce_256(total_part, red4, false);
        lane_part[threadIdx.x] = sum;
        __syncthreads();
        if (share == 0 && j < head_dim) {
            double lane_sum = lane_part[threadIdx.x];
            for (int i = 1; i < lanes_per; ++i) lane_sum = lane_sum + lane_part[threadIdx.x + i * width];
            out[static_cast<int64_t>(head) * head_dim + j] = static_cast<float>(lane_sum / total);
        }
        __syncthreads();
    }
}

__device__ __forceinline__ uint32_t byte_at(const uint8_t* p) { return *(const SATORI_GLOBAL uint8_t*)(p); }
__device__ __forceinline__ uint32_t half_bits_at(const uint8_t* p) { return byte_at(p) | (byte_at(p + 1) << 8); }

// One row of a resident Q8_0 / Q4_K / Q6_K matrix decoded to FP32 (QuantizedRow.DecodeQ8Block,
// Q4KCodec.DecodeBlock, Q6KCodec.DecodeBlock), one thread per element, reading the device layout (Q8_0 and
// Q6_K regrouped as at upload).
__global__ __launch_bounds__(kThreads) void decode_row_kernel(const uint8_t* __restrict__ w, int format, int rows,
                                                              int columns, int row, float* __restrict__ out) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= columns) return;
    float value;
    if (format == kQ8_0) {  // regrouped: 32-byte code records, then the FP16 scales
        const int64_t count = static_cast<int64_t>(rows) * (columns / 32);
        const int64_t index = static_cast<int64_t>(row) * (columns / 32) + i / 32;
        const float scale = half_bits_to_float(half_bits_at(w + count * 32 + index * 2));
        value = scale * static_cast<float>(static_cast<int8_t>(byte_at(w + index * 32 + i % 32)));
    } else if (format == kQ4_K) {
        const uint8_t* block = w + (static_cast<int64_t>(row) * (columns / 256) + i / 256) * 144;
        const int e = i % 256, group = e / 64, high = (e % 64) / 32, l = e % 32;
        const u32x4 head = load16_a4(block);
        int s, m;
        q4k_scale_min(2 * group + high, head, s, m);
        const float d = half_bits_to_float(head[0] & 0xFFFFu), dmin = half_bits_to_float(head[0] >> 16);
        const uint32_t q = (byte_at(block + 16 + 32 * group + l) >> (4 * high)) & 0xF;
        value = __fsub_rn(__fmul_rn(__fmul_rn(d, static_cast<float>(s)), static_cast<float>(q)),
                          __fmul_rn(dmin, static_cast<float>(m)));
    } else {  // Q6_K, regrouped: records of 192 bytes, then 16 scale bytes per block, then the FP16 d values
        const int64_t count = static_cast<int64_t>(rows) * (columns / 256);
        const int64_t index = static_cast<int64_t>(row) * (columns / 256) + i / 256;
        const int e = i % 256, hh = e / 128, kk = (e % 128) / 32, t = (e % 32) / 16, x = e % 16;
        const int c = 2 * hh + t;
        const uint8_t* q = w + index * 192 + 48 * c;
        const uint32_t low = kk & 1 ? byte_at(q + 16 + x) : byte_at(q + x);
        const uint32_t nib = kk < 2 ? (low & 0xF) : (low >> 4);
        const uint32_t hb = (byte_at(q + 32 + x) >> (2 * kk)) & 3;
        const int code = static_cast<int>(nib | (hb << 4)) - 32;
        const int sc = static_cast<int8_t>(byte_at(w + count * 192 + index * 16 + 4 * c + kk));
        const float d = half_bits_to_float(half_bits_at(w + count * 208 + index * 2));
        value = __fmul_rn(__fmul_rn(d, static_cast<float>(sc)), static_cast<float>(code));
    }
    out[i] = value;
}

int grid_for(int64_t n) { return static_cast<int>((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_rms_norm(const float* x, const float* w, float epsilon, int length, int count, float* y,
                           hipStream_t stream) {
    rms_norm_kernel<<<count, kThreads, 0, stream>>>(x, w, epsilon, length, y);
    return hipGetLastError();
}

hipError_t launch_rms_norm_heads(float* v, const float* w, float epsilon, int head_dim, int heads, hipStream_t stream) {
    rms_norm_heads_kernel<<<heads, kThreads, 0, stream>>>(v, w, epsilon, head_dim);
    return hipGetLastError();
}

hipError_t launch_rope(float* v, int heads, int head_dim, int position, double base, int rotary, bool half_split,
                       hipStream_t stream) {
    rope_kernel<<<grid_for(static_cast<int64_t>(heads) * (rotary / 2)), kThreads, 0, stream>>>(
        v, heads, head_dim, position, base, rotary, half_split ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* gate, const float* up, int length, float* out, hipStream_t stream) {
    swiglu_kernel<<<grid_for(length), kThreads, 0, stream>>>(gate, up, length, out);
    return hipGetLastError();
}

hipError_t launch_swiglu_q8k(const float* gate, const float* up, int length, float* out, uint8_t* q8k,
                             hipStream_t stream) {
    if (length <= 0 || length % 256 != 0) return hipErrorInvalidValue;
    swiglu_q8k_kernel<<<length / 256, 64, 0, stream>>>(gate, up, out, q8k);
    return hipGetLastError();
}

hipError_t launch_add(const float* left, const float* right, int length, float* out, hipStream_t stream) {
    add_kernel<<<grid_for(length), kThreads, 0, stream>>>(left, right, length, out);
    return hipGetLastError();
}

hipError_t launch_add_rms_norm(float* residual, const float* addend, const float* w, float epsilon, int length,
                               float* normed, hipStream_t stream) {
    add_rms_norm_kernel<<<1, kThreads, 0, stream>>>(residual, addend, w, epsilon, length, normed);
    return hipGetLastError();
}

hipError_t launch_add_rms_norm_q8k(float* residual, const float* addend, const float* w, float epsilon, int length,
                                   float* normed, uint8_t* q8k, hipStream_t stream) {
    if (length <= 0 || length % 256 != 0) return hipErrorInvalidValue;
    if (length > kNormQ8KStaged) {
        const hipError_t e = launch_add_rms_norm(residual, addend, w, epsilon, length, normed, stream);
        if (e != hipSuccess) return e;
        return launch_q8k_quantize(normed, length, 1, q8k, stream);
    }
    add_rms_norm_q8k_kernel<<<1, kThreads, static_cast<size_t>(length) * sizeof(float), stream>>>(
        residual, addend, w, epsilon, length, normed, q8k);
    return hipGetLastError();
}

hipError_t launch_attention_inputs(float* q, const float* q_bias, const float* k, const float* k_bias, float* k_out,
                                   const float* v, const float* v_bias, float* v_out, int heads, int kv_heads,
                                   int head_dim, int position, double base, int rotary, hipStream_t stream) {
    const int64_t items = static_cast<int64_t>(heads + kv_heads) * (rotary / 2) +
                          static_cast<int64_t>(heads + kv_heads) * (head_dim - rotary) +
                          static_cast<int64_t>(kv_heads) * head_dim;
    attention_inputs_kernel<<<grid_for(items), kThreads, 0, stream>>>(q, q_bias, k, k_bias, k_out, v, v_bias, v_out,
                                                                     heads, kv_heads, head_dim, position, base, rotary);
    return hipGetLastError();
}

int attention_splits(int tokens) {
    // One workgroup per head up to 32 tokens; then at least 32 tokens per split and at most 32 splits (a
    // 4096-token context: 128 tokens per split, 384 workgroups for 12 heads; 16 splits measured slower, 64
    // no faster alone and slower once the decode fuses its inputs at 64 tokens per split); beyond 4,096
    // tokens 128 tokens per split up to 64 splits (8,192 tokens: 21.5 against 26.0 us per layer with 32
    // splits); and beyond that as many splits as keep each at most 2,048 tokens.
    if (tokens <= 32) return 1;
    int splits = std::min(kMinSplits, (tokens + 31) / 32);
    splits = std::max(splits, std::min(kLongSplits, (tokens + 127) / 128));
    splits = std::max(splits, (tokens + kMaxSplitTokens - 1) / kMaxSplitTokens);
    return std::min(splits, kMaxSplitsPerLaunch);
}

size_t attention_scratch_bytes(int query_heads, int head_dim, int tokens) {
    const int splits = std::max(kMinSplits, attention_splits(tokens));
    // The partials, then the rotated query of the fused decode form.
    return static_cast<size_t>(query_heads) * splits * (2 + head_dim) * sizeof(double) +
           static_cast<size_t>(query_heads) * head_dim * sizeof(float);
}

namespace {

// Threads of a split workgroup: 512 once a split holds at least kWideSplitTokens tokens (its score passes and
// value loops, each a dependent round of key / value loads, then half as long: a 128-token split's value parts
// are its 16 preloaded rows and one round of 16) while the launch's workgroups fit the CUs at two each (16
// waves: more would run in a second round), else 256. Measured on the whole Qwen-1.5B-shaped token (12 / 2 heads
// of 128 lanes): 1,420 against 1,460 us at 4,095 tokens (32 splits of 128); 512 threads at 96-token splits
// (3,072 tokens) measured slower, 1,514 against 1,462 (their 24-row value parts end in 8 rows read one at a
// time), and at 8,191 tokens (768 workgroups) 1,648 against 1,556.
constexpr int kWideSplitTokens = 128;

int device_cus() {
    int device = 0, cus = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

int split_threads(int per, int workgroups) {
    return per >= kWideSplitTokens && workgroups <= 2 * device_cus() ? 512 : 256;
}

size_t split_lds_bytes(int per, int head_dim) {
    return static_cast<size_t>(per) * sizeof(double) +
           (head_dim <= kStagedQuery ? static_cast<size_t>(head_dim) * sizeof(float) : 0);
}

}  // namespace

bool attention_supported(int tokens, int head_dim) {
    const int splits = attention_splits(tokens);
    if (splits == 1) return true;
    const int per = (tokens + splits - 1) / splits;
    return split_lds_bytes(per, head_dim) + 512 * sizeof(double) <= 64 * 1024;  // either workgroup size
}

namespace {

size_t split_lds_bytes_inputs(int per, int head_dim) {
    return static_cast<size_t>(per) * sizeof(double) + static_cast<size_t>(3) * head_dim * sizeof(float);
}

// The fused form needs the split path, one thread per lane of the head (at most 256 lanes) and room for the new
// row's key and value. It is taken while splits hold at most 80 tokens: measured per layer of a Qwen-1.5B
// token (12 / 2 heads of 128 lanes, 28 layers' caches, attention and combine), fused against the separate
// input launch, 11.1 vs 12.2 us at 512 tokens (16 splits of 32), 15.1 vs 17.0 at 2,049 (65 per split), 17.5
// vs 18.5 at 2,560 (80), but 19.1 vs 16.9 at 3,072 (96) and 20.7 vs 18.6 at 4,096 (128), where the fused
// split launch's longer score and value loops cost more than the launch it saves.
constexpr int kFusedSplitTokens = 80;

bool decode_fusable(int tokens, int head_dim) {
    const int splits = attention_splits(tokens);
    if (splits == 1 || head_dim > kSplitThreads || (tokens + splits - 1) / splits > kFusedSplitTokens) return false;
    const int per = (tokens + splits - 1) / splits;
    return split_lds_bytes_inputs(per, head_dim) + 512 * sizeof(double) <= 64 * 1024;  // either workgroup size
}

}  // namespace

hipError_t launch_rope_table(int positions, int rotary, double base, double* table, hipStream_t stream) {
    const int64_t n = static_cast<int64_t>(positions) * (rotary / 2);
    if (n <= 0) return hipSuccess;
    rope_table_kernel<<<grid_for(n), kThreads, 0, stream>>>(positions, rotary, base, table);
    return hipGetLastError();
}

hipError_t launch_attention_decode(float* q, const float* q_bias, const float* k_new, const float* k_bias,
                                   const float* v_new, const float* v_bias, float* k_cache, float* v_cache,
                                   int query_heads, int kv_heads, int head_dim, int position, double base, int rotary,
                                   const double* rope, float* out, double* partials, hipStream_t stream) {
    const int tokens = position + 1;
    const int64_t kv_width = static_cast<int64_t>(kv_heads) * head_dim;
    if (!decode_fusable(tokens, head_dim)) {  // the two launches it stands for
        hipError_t e = launch_attention_inputs(q, q_bias, k_new, k_bias, k_cache + position * kv_width, v_new, v_bias,
                                               v_cache + position * kv_width, query_heads, kv_heads, head_dim,
                                               position, base, rotary, stream);
        if (e != hipSuccess) return e;
        return launch_attention(q, k_cache, v_cache, query_heads, kv_heads, head_dim, tokens, out, partials, stream);
    }
    if (!partials) return hipErrorInvalidValue;
    const int splits = attention_splits(tokens);
    const int per = (tokens + splits - 1) / splits;
    const DecodeInputs in{q_bias, k_new, k_bias, v_new, v_bias, rope, position, rotary, base};
    const int grid = split_grid(query_heads, kv_heads, splits);
    const size_t lds = split_lds_bytes_inputs(per, head_dim);
    if (split_threads(per, grid) == 512)
        attention_split_kernel<true, 512><<<grid, 512, lds, stream>>>(q, k_cache, v_cache, query_heads, kv_heads, head_dim,
                                                                    tokens, per, splits, partials, in, k_cache, v_cache);
    else
        attention_split_kernel<true, 256><<<grid, 256, lds, stream>>>(q, k_cache, v_cache, query_heads, kv_heads, head_dim,
                                                                    tokens, per, splits, partials, in, k_cache, v_cache);
    attention_combine_kernel<true><<<query_heads, kSplitThreads, 0, stream>>>(partials, splits, head_dim, out, q, in);
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const float* k, const float* v, int query_heads, int kv_heads,
                            int head_dim, int tokens, float* out, double* partials, hipStream_t stream) {
    if (!attention_supported(tokens, head_dim)) return hipErrorInvalidValue;
    const int splits = attention_splits(tokens);
    if (splits == 1) {
        attention_kernel<<<query_heads, kAttnThreads, static_cast<size_t>(tokens) * sizeof(double), stream>>>(
            q, k, v, query_heads, kv_heads, head_dim, tokens, out);
        return hipGetLastError();
    }
    if (!partials) return hipErrorInvalidValue;
    const int per = (tokens + splits - 1) / splits;
    const int grid = split_grid(query_heads, kv_heads, splits);
    const size_t lds = split_lds_bytes(per, head_dim);
    if (split_threads(per, grid) == 512)
        attention_split_kernel<false, 512><<<grid, 512, lds, stream>>>(q, k, v, query_heads, kv_heads, head_dim, tokens,
                                                                     per, splits, partials, DecodeInputs{}, nullptr,
                                                                     nullptr);
    else
        attention_split_kernel<false, 256><<<grid, 256, lds, stream>>>(q, k, v, query_heads, kv_heads, head_dim, tokens,
                                                                     per, splits, partials, DecodeInputs{}, nullptr,
                                                                     nullptr);
    attention_combine_kernel<false><<<query_heads, kSplitThreads, 0, stream>>>(partials, splits, head_dim, out,
                                                                              nullptr, DecodeInputs{});
    return hipGetLastError();
}

size_t attention_partials_bytes(int query_heads, int head_dim, int tokens) {
    const int splits = attention_splits(tokens);
    return splits == 1 ? 0 : static_cast<size_t>(query_heads) * splits * (2 + head_dim) * sizeof(double);
}

hipError_t launch_decode_row(const uint8_t* w, int format, int rows, int columns, int row, float* out,
                             hipStream_t stream) {
    decode_row_kernel<<<grid_for(columns), kThreads, 0, stream>>>(w, format, rows, columns, row, out);
    return hipGetLastError();
}

hipError_t static_attention_partials(double** partials) {
    void* address = nullptr;
    const hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    *partials = static_cast<double*>(address);
    return hipSuccess;
}

}  // namespace satori
