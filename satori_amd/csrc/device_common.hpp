// Device helpers shared by the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace satori {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte load from a 4-byte aligned global address (one global_load_dwordx4).
__device__ __forceinline__ u32x4 load16_a4(const uint8_t* p) {
    return *reinterpret_cast<const u32x4_a4*>(p);
}

__device__ __forceinline__ uint32_t load4_a4(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}

// N little-endian dwords starting at a 2-byte aligned address, assembled from N + 1 aligned dword loads
// and v_alignbyte. Reads up to 4 bytes past p + 4N; every payload allocation carries slack for that.
template <int N>
__device__ __forceinline__ void load_unaligned(const uint8_t* p, uint32_t (&out)[N]) {
    const uintptr_t address = reinterpret_cast<uintptr_t>(p);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(address & ~uintptr_t(3));
    const uint32_t shift = static_cast<uint32_t>(address & 3);
    uint32_t d[N + 1];
#pragma unroll
    for (int i = 0; i <= N; ++i) d[i] = base[i];
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], shift);
}

// binary16 -> binary32, exact (v_cvt_f32_f16; FP16 denormals are kept by the kernel float mode).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    _Float16 h;
    const uint16_t b = static_cast<uint16_t>(bits16);
    __builtin_memcpy(&h, &b, 2);
    return static_cast<float>(h);
}

__device__ __forceinline__ float byte_to_float(uint32_t word, int index) {
    return static_cast<float>((word >> (8 * index)) & 0xFFu);
}

__device__ __forceinline__ float sbyte_to_float(uint32_t word, int index) {
    return static_cast<float>(static_cast<int8_t>(word >> (8 * index)));
}

// Sum over aligned groups of L lanes (L a power of two <= 64); every lane of a group gets the sum.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int offset = L / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

template <int L>
__device__ __forceinline__ int group_sum_int(int v) {
#pragma unroll
    for (int offset = L / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

}  // namespace satori
