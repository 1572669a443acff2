// Device arithmetic shared by the decode-step operators (transformer_ops.hip) and the K-format launches that
// compute their input from those operators' operands (gemv_kint.hip), so that both produce the same FP32
// values bit for bit: the RmsNorm reduction over 256 threads (TransformerOps.RmsNorm, TransformerOps.cs:13-21)
// and the SwiGlu element (TransformerOps.cs:40-50), each in FP64 with one FP32 rounding.
#pragma once

#include <cmath>

#include "device_common.hpp"

namespace satori {

constexpr int kOpsThreads = 256;

// Sum of one double per thread over a 256-thread workgroup (tree in LDS, fixed order: deterministic).
// `red` holds 256 doubles; every thread of the workgroup must call it.
__device__ __forceinline__ double block_sum_256(double v, double* red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int s = kOpsThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + s];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

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
