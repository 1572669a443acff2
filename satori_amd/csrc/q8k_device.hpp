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

namespace satori {

// The same quantization with 16 lanes per block (one DPP row), sixteen elements per lane: lane j of the
// row holds elements 16j .. 16j + 15, which are exactly Q8_K group j, so its group sum needs no cross-lane
// step. The row maximum of the magnitude keys is an all-reduce by rotation within the row (row_ror 1, 2,
// 4, 8); the first index holding it is the lowest row lane whose own first maximal element has the key
// (ballot), and that element's signed value is read from its lane (bpermute). Four blocks per wave.
struct Q8KRow16 {
    uint32_t packed[4];  // codes 16j .. 16j + 15
    int group_sum;       // sum of those 16 codes
    float scale;         // 1 / inverse, or 0 for an all-zero block
};

__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xF, 0xF, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xF, 0xF, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xF, 0xF, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xF, 0xF, false)));
    return v;
}

// `lane` is the lane within the wave (0..63); all 16 lanes of its row must be active together.
__device__ __forceinline__ Q8KRow16 q8k_quantize_row16(const float (&v)[16], int lane) {
    uint32_t key = 0;
    float first = 0.0f;  // the lane's first element of maximal magnitude (strict >: the lowest index wins)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float a = __builtin_fabsf(v[i]);
        const uint32_t k = a == a ? __float_as_uint(a) : 0u;  // NaN never wins
        if (k > key) {
            key = k;
            first = v[i];
        }
    }
    const uint32_t best = row_max_u32(key);
    Q8KRow16 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r.packed[w] = 0u;
    r.group_sum = 0;
    r.scale = 0.0f;
    if (best == 0u) return r;  // magnitude 0: the block is all zero bytes (Q8KCodec.cs:59-63)
    const int base = lane & ~15;
    const uint64_t holders = __ballot(key == best);
    const uint32_t row_bits = static_cast<uint32_t>(holders >> base) & 0xFFFFu;
    const int src = base + __builtin_ctz(row_bits);
    const float max = __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(first)));
    const float inverse = __fdiv_rn(-127.0f, max);
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float shifted = __fadd_rn(__fmul_rn(inverse, v[i]), 12582912.0f);
        int n = static_cast<int>(__float_as_uint(shifted) & 0x007FFFFFu) - 0x00400000;  // NearestInteger, :120-125
        n = n < 127 ? n : 127;
        sum += static_cast<int8_t>(n);
        r.packed[i >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(n)) << (8 * (i & 3));
    }
    r.group_sum = sum;
    r.scale = __fdiv_rn(1.0f, inverse);
    return r;
}

}  // namespace satori
