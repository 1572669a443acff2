// Q8_K quantization of one 256-element block by one wave (Q8KCodec.QuantizeBlock, src/Satori.Core/Q8KCodec.cs:44-76),
// shared by the Q8_K kernels: first-largest |x| with a strict comparison, -127/max and 1/inverse as correctly
// rounded divisions, the product and the 12582912 add rounded separately.
#pragma once

#include "device_common.hpp"

namespace satori {

// One wave per 256-element block, four consecutive elements per lane.
struct Q8KLane {
    uint32_t packed;  // this lane's four codes (elements 4 * lane .. 4 * lane + 3)
    int group_sum;    // sum of the 16 codes of group lane / 4 (every lane of the group holds it)
    float scale;      // 1 / inverse (the block's float scale)
    bool zero;        // the block is all zero: every byte of it is zero
};

// One block from this lane's four values v = src[4 * lane .. 4 * lane + 3]. The first-largest magnitude
// (Q8KCodec.cs:50-56: strict comparison, so the lowest index wins ties and NaN never wins) is found as the
// wave maximum of the magnitudes' bit patterns (NaN mapped to 0; non-negative floats order like their
// bits), then the wave minimum of the indices holding it; the signed value is read from its lane.
__device__ __forceinline__ Q8KLane q8k_quantize_values(const float (&v)[4], int lane) {
    uint32_t key = 0;
    int index = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = __builtin_fabsf(v[i]);
        const uint32_t k = a == a ? __float_as_uint(a) : 0u;  // NaN never wins
        if (k > key) {
            key = k;
            index = 4 * lane + i;
        }
    }
    const uint32_t best = wave_extreme_u32<true>(key);
    Q8KLane r{0u, 0, 0.0f, best == 0u};  // magnitude 0: the block is all zero bytes (Q8KCodec.cs:59-63)
    if (r.zero) return r;
    const int first = static_cast<int>(wave_extreme_u32<false>(key == best ? static_cast<uint32_t>(index) : 0xFFFFFFFFu));
    const float candidate = (first & 3) == 0 ? v[0] : (first & 3) == 1 ? v[1] : (first & 3) == 2 ? v[2] : v[3];
    const float max = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(candidate), first >> 2));
    const float inverse = __fdiv_rn(-127.0f, max);
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float shifted = __fadd_rn(__fmul_rn(inverse, v[i]), 12582912.0f);
        int n = static_cast<int>(__float_as_uint(shifted) & 0x007FFFFFu) - 0x00400000;  // NearestInteger, :120-125
        n = n < 127 ? n : 127;
        const int8_t code = static_cast<int8_t>(n);
        sum += code;
        r.packed |= (static_cast<uint32_t>(static_cast<uint8_t>(code))) << (8 * i);
    }
    r.group_sum = quad_sum_int(sum);  // group sums of 16 codes = 4 lanes (Q8KCodec.cs:68-74)
    r.scale = __fdiv_rn(1.0f, inverse);
    return r;
}

__device__ __forceinline__ void q8k_load_values(const float* __restrict__ src, int lane, float (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = load_f32(src + 4 * lane + i);
}

}  // namespace satori
