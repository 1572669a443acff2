// Device arithmetic shared by the decode-step operators (transformer_ops.hip) and the K-format launches that
// compute their input from those operators' operands (gemv_kint.hip), so that both produce the same FP32
// values bit for bit: the RmsNorm reduction over 256 threads (TransformerOps.RmsNorm, TransformerOps.cs:13-21)
// and the SwiGlu element (TransformerOps.cs:40-50), each in FP64 with one FP32 rounding.
#pragma once

#include <cmath>

#include "device_common.hpp"

namespace satori {

constexpr int kOpsThreads = 256;

// Reduction (sum or maximum) of one double per thread over a 256-thread workgroup in a fixed pairwise tree
// (deterministic): at stride s = 128, 64, ..., 1, value t < s becomes op(value t, value t + s). The first
// wave forms the strides 128 and 64 from the LDS copy, then the strides 32 to 1 in registers with lane
// shuffles (lane t < s combines lane t + s: the same operations in the same order as the tree in LDS), so
// the tree costs three barriers instead of ten. `red` holds 256 doubles; every thread of the workgroup must
// call it, and every thread gets the result.
__device__ __forceinline__ double block_tree_256(double v, double* red, bool take_max) {
    const int t = threadIdx.x;
    auto op = [take_max](double a, double b) { return take_max ? fmax(a, b) : a + b; };
    red[t] = v;
    __syncthreads();
    if (t < 64) {
        double x = op(op(red[t], red[t + 128]), op(red[t + 64], red[t + 192]));
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) x = op(x, __shfl_down(x, s, 64));
        if (t == 0) red[0] = x;
    }
    __syncthreads();
    const double r = red[0];
    __syncthreads();
    return r;
}

__device__ __forceinline__ double block_sum_256(double v, double* red) { return block_tree_256(v, red, false); }

// 1 / sqrt(mean of squares + epsilon) from the sum of squares of `length` values.
__device__ __forceinline__ double rms_scale(double sum, int length, float epsilon) {
    return 1.0 / __dsqrt_rn(sum / length + static_cast<double>(epsilon));
}

// One RmsNorm output: value * scale * weight in FP64, rounded once.
__device__ __forceinline__ float rms_value(float value, double scale, float weight) {
    return static_cast<float>(static_cast<double>(value) * scale * static_cast<double>(weight));
}

// One SwiGlu output: silu(gate) * up in FP64 (the sigmoid in the overflow-safe form for negative gates).
__device__ __forceinline__ float swiglu_value(float gate, float up) {
    const double x = gate;
    const double sigmoid = x >= 0 ? 1.0 / (1.0 + exp(-x)) : exp(x) / (1.0 + exp(x));
    return static_cast<float>(x * sigmoid * static_cast<double>(up));
}

}  // namespace satori
