// Device helpers shared by the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#define SATORI_GLOBAL __attribute__((address_space(1)))

namespace satori {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Loads through the global address space (global_load_* rather than flat_*): every pointer the kernels
// dereference with these helpers is device memory returned by hipMalloc.
__device__ __forceinline__ u32x4 load16_a4(const uint8_t* p) {
    return *(const SATORI_GLOBAL u32x4_a4*)(p);
}

__device__ __forceinline__ uint32_t load4_a4(const uint8_t* p) {
    return *(const SATORI_GLOBAL uint32_t*)(p);
}

__device__ __forceinline__ uint64_t load8_a8(const uint8_t* p) { return *(const SATORI_GLOBAL uint64_t*)(p); }

__device__ __forceinline__ uint32_t load2_a2(const uint8_t* p) { return *(const SATORI_GLOBAL uint16_t*)(p); }

__device__ __forceinline__ float load_f32(const float* p) { return *(const SATORI_GLOBAL float*)(p); }

// Non-temporal loads for data that one instruction reads exactly once per launch (the Ternary2 panel
// layout): streamed past the caches instead of evicting the activations and partial sums that are reused.
// Layouts whose lines are touched again by later instructions (block headers shared by several chunks,
// misaligned blocks) must use the plain loads above.
__device__ __forceinline__ u32x4 stream16(const uint8_t* p) {  // 16-byte aligned
    return __builtin_nontemporal_load((const SATORI_GLOBAL u32x4*)(p));
}

__device__ __forceinline__ uint32_t stream4(const uint8_t* p) {
    return __builtin_nontemporal_load((const SATORI_GLOBAL uint32_t*)(p));
}

__device__ __forceinline__ void store_f32(float* p, float v) { *(SATORI_GLOBAL float*)(p) = v; }
__device__ __forceinline__ void store_u32(uint32_t* p, uint32_t v) { *(SATORI_GLOBAL uint32_t*)(p) = v; }

// N little-endian dwords starting at a 2-byte aligned address, assembled from N + 1 aligned dword loads
// and v_alignbyte. Reads up to 4 bytes past p + 4N; every payload allocation carries slack for that.
// (Plain loads: neighbouring lanes and the next instruction read the same lines again.)
template <int N>
__device__ __forceinline__ void load_unaligned(const uint8_t* p, uint32_t (&out)[N]) {
    const uintptr_t address = reinterpret_cast<uintptr_t>(p);
    const SATORI_GLOBAL uint32_t* base = (const SATORI_GLOBAL uint32_t*)(address & ~uintptr_t(3));
    const uint32_t shift = static_cast<uint32_t>(address & 3);
    uint32_t d[N + 1];
#pragma unroll
    for (int i = 0; i <= N; ++i) d[i] = base[i];
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], shift);
}

// One quarter (c = 2h + t) of Q6_K block `index` from the regrouped device layout of a matrix of `blocks`
// blocks (Q6KLayout): 48 code bytes (ql[64h + 16t, +16), ql[64h + 32 + 16t, +16), qh[32h + 16t, +16)), the
// quarter's four scales sc[8h + 2k + t] (byte k), and d.
struct Q6KQuarter {
    u32x4 qla, qlb, qh;
    uint32_t sc;
    uint32_t dpair;   // the aligned dword holding d (kept raw: converting it at load time would wait for it)
    uint32_t dshift;  // 0 or 16: d's half of dpair
};

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16);

__device__ __forceinline__ void q6k_load_quarter(const uint8_t* w, int64_t blocks, int64_t index, int c,
                                                 Q6KQuarter& r) {
    const uint8_t* record = w + index * 192 + 48 * c;
    r.qla = *(const SATORI_GLOBAL u32x4*)(record);
    r.qlb = *(const SATORI_GLOBAL u32x4*)(record + 16);
    r.qh = *(const SATORI_GLOBAL u32x4*)(record + 32);
    r.sc = load4_a4(w + blocks * 192 + index * 16 + 4 * c);
    // d array: 2 bytes per block from offset blocks * 208 (a multiple of 16); read the aligned dword.
    r.dpair = load4_a4(w + blocks * 208 + (index & ~int64_t(1)) * 2);
    r.dshift = 16 * static_cast<uint32_t>(index & 1);
}

// The quarter's block scale d (FP16 -> FP32, exact), read where it is used.
__device__ __forceinline__ float q6k_d(const Q6KQuarter& r) { return half_bits_to_float(r.dpair >> r.dshift); }

// Q4KCodec.GetScaleMin (src/Satori.Core/Q4KCodec.cs:24-36) for sub-block j (0..7), from the dwords holding
// scales[12] (head[1..3]). Both forms are computed from fixed dwords with a per-lane shift and one is
// selected, so no register vector is indexed by a per-lane value.
__device__ __forceinline__ void q4k_scale_min(int j, const u32x4& head, int& scale, int& min) {
    const int shift = 8 * (j & 3);
    const uint32_t a = head[1] >> shift, b = head[2] >> shift, c = head[3] >> shift;  // bytes j&3, 4+(j&3), 8+(j&3)
    const int low_scale = static_cast<int>(a & 63), low_min = static_cast<int>(b & 63);
    const int high_scale = static_cast<int>((c & 0xFu) | (((a >> 6) & 3u) << 4));
    const int high_min = static_cast<int>(((c >> 4) & 0xFu) | (((b >> 6) & 3u) << 4));
    scale = j < 4 ? low_scale : high_scale;
    min = j < 4 ? low_min : high_min;
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

// DPP lane moves within 16-lane rows (row_shr:n) and across rows (row_bcast:15 / row_bcast:31).
template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, BOUND_ZERO);
}

// Sum over aligned groups of L lanes (L a power of two, 2..64) with DPP adds: the total of each group is
// valid in the group's LAST lane (lane % L == L - 1); other lanes hold partial sums.
template <int L>
__device__ __forceinline__ float group_sum_last(float v) {
    if constexpr (L >= 2) v += __int_as_float(dpp<0x111, 0xF, true>(__float_as_int(v)));
    if constexpr (L >= 4) v += __int_as_float(dpp<0x112, 0xF, true>(__float_as_int(v)));
    if constexpr (L >= 8) v += __int_as_float(dpp<0x114, 0xF, true>(__float_as_int(v)));
    if constexpr (L >= 16) v += __int_as_float(dpp<0x118, 0xF, true>(__float_as_int(v)));
    if constexpr (L >= 32) v += __int_as_float(dpp<0x142, 0xA, false>(__float_as_int(v)));
    if constexpr (L >= 64) v += __int_as_float(dpp<0x143, 0xC, false>(__float_as_int(v)));
    return v;
}

// Maximum (MAX) or minimum of an unsigned value over the whole wave, returned to every lane: DPP steps
// within rows and across rows, then a read of lane 63. Lanes outside a step's source range contribute the
// identity.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_extreme_u32(uint32_t v) {
    constexpr uint32_t kIdentity = MAX ? 0u : 0xFFFFFFFFu;
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    auto step = [&](auto ctrl, auto row_mask) {
        const uint32_t other = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            static_cast<int>(kIdentity), static_cast<int>(v), decltype(ctrl)::value, decltype(row_mask)::value,
            0xF, false));
        v = op(v, other);
    };
    step(std::integral_constant<int, 0x111>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x112>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xA>{});
    step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xC>{});
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Sum over each aligned group of 4 lanes, in every lane of the group (DPP quad permutes).
__device__ __forceinline__ int quad_sum_int(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    return v;
}

template <int L>
__device__ __forceinline__ int group_sum_last_int(int v) {
    if constexpr (L >= 2) v += dpp<0x111, 0xF, true>(v);
    if constexpr (L >= 4) v += dpp<0x112, 0xF, true>(v);
    if constexpr (L >= 8) v += dpp<0x114, 0xF, true>(v);
    if constexpr (L >= 16) v += dpp<0x118, 0xF, true>(v);
    if constexpr (L >= 32) v += dpp<0x142, 0xA, false>(v);
    if constexpr (L >= 64) v += dpp<0x143, 0xC, false>(v);
    return v;
}

}  // namespace satori
