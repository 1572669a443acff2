// Upload-time regrouping on the device. A packed payload is copied unchanged into a device staging buffer
// and rearranged there into the device layout the MatVec kernels read (kernels.hpp: the Ternary2 panel
// layout, the Q6_K quarter records, the Q8_0 / Q4_0 aligned code records), so the host only copies bytes.
// The Ternary2 kernel also applies the payload rule of Ternary2Matrix.ValidatePayload
// (src/Satori.Core/Ternary2Matrix.cs:83-101) to every block and raises a flag on the first failure it sees;
// the host then names the failure with its own restatement of that rule (the reference's order and message).
// Each kernel covers one chunk of whole units (64-row panels or blocks) of the payload; the caller zeroes the
// destination first, so padding rows, chunks and scale slots stay zero.
#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

__device__ __forceinline__ uint32_t load_u32(const uint8_t* p) { return *(const SATORI_GLOBAL uint32_t*)(p); }
__device__ __forceinline__ uint32_t load_u16(const uint8_t* p) { return *(const SATORI_GLOBAL uint16_t*)(p); }

// Bits 0..15 of v moved to the even bit positions 0, 2, ..., 30.
__device__ __forceinline__ uint32_t spread16(uint32_t v) {
    v &= 0xFFFFu;
    v = (v | (v << 8)) & 0x00FF00FFu;
    v = (v | (v << 4)) & 0x0F0F0F0Fu;
    v = (v | (v << 2)) & 0x33333333u;
    v = (v | (v << 1)) & 0x55555555u;
    return v;
}

// Thread (panel, block, lane) of the chunk: row lane of the panel, one block of it. The source rows of the
// chunk start at `packed` (row row0 = first_panel * 64). With r.bitplanes the source blocks are ternary
// bitplane blocks (the scale, then B/8 bytes of positive-plane bits and B/8 of negative-plane bits, bit i of
// the plane is weight i), converted to their Ternary2 codes (code = positive bit | negative bit << 1,
// TernaryBitplaneMatrix.ToTernary2, src/Satori.Core/TernaryBitplaneMatrix.cs:38-54). A bitplane block breaks
// TernaryBitplaneMatrix.Validate (:64-85) exactly when its codes break the Ternary2 rule checked here.
__global__ __launch_bounds__(256) void t2_panels_kernel(const uint8_t* __restrict__ packed, T2Regroup r,
                                                         uint8_t* __restrict__ out, uint32_t* __restrict__ bad) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int lane = static_cast<int>(t & 63);
    const int64_t pb = t >> 6;
    const int block = static_cast<int>(pb % r.blocks);
    const int local_panel = static_cast<int>(pb / r.blocks);
    const int local_row = local_panel * kT2PanelRows + lane;
    if (local_row >= r.chunk_rows) return;
    const int64_t panel = static_cast<int64_t>(r.first_panel) + local_panel;
    const uint8_t* src = packed + static_cast<int64_t>(local_row) * r.row_bytes + static_cast<int64_t>(block) * r.block_bytes;
    const uint32_t bits = load_u32(src);
    *(SATORI_GLOBAL uint32_t*)(out + r.codes_bytes + ((panel * r.slots + block) * 64 + lane) * 4) = bits;

    // Ternary2Matrix.ValidatePayload for this block: a finite, non-negative scale that is not -0; no code 3;
    // zero codes past the last column and everywhere in a block of scale 0.
    const float scale = __uint_as_float(bits);
    bool invalid = !isfinite(scale) || scale < 0.0f || bits == 0x80000000u;
    const int count = min(r.block_size, r.columns - block * r.block_size);
    const int per_block = r.block_size / 64;  // 16-byte code records in a block
    for (int i = 0; i < per_block; ++i) {
        uint32_t w[4];
        if (r.bitplanes) {
            const uint8_t* pos = src + 4 + 8 * i;
            const uint8_t* neg = pos + r.block_size / 8;
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // weights 32h .. 32h + 31 of the record
                const uint32_t p = load_u32(pos + 4 * h), q = load_u32(neg + 4 * h);
                w[2 * h] = spread16(p) | (spread16(q) << 1);
                w[2 * h + 1] = spread16(p >> 16) | (spread16(q >> 16) << 1);
            }
        } else {
#pragma unroll
            for (int d = 0; d < 4; ++d) w[d] = load_u32(src + 4 + 16 * i + 4 * d);
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int first = count - 64 * i - 16 * d;  // fields of this dword before the last column
            uint32_t must_be_zero;
            if (scale == 0.0f || first <= 0)
                must_be_zero = 0x55555555u;
            else if (first >= 16)
                must_be_zero = 0u;
            else
                must_be_zero = 0x55555555u & ~((1u << (2 * first)) - 1u);
            const uint32_t code3 = w[d] & (w[d] >> 1) & 0x55555555u;
            const uint32_t nonzero = (w[d] | (w[d] >> 1)) & 0x55555555u;
            invalid = invalid || code3 != 0u || (nonzero & must_be_zero) != 0u;
        }
        // The record rotated left by 2 bits as one 128-bit little-endian integer.
        u32x4 rot;
#pragma unroll
        for (int d = 0; d < 4; ++d) rot[d] = (w[d] << 2) | (w[(d + 3) & 3] >> 30);
        const int64_t chunk = static_cast<int64_t>(block) * per_block + i;
        *(SATORI_GLOBAL u32x4*)(out + ((panel * r.chunks + chunk) * 64 + lane) * 16) = rot;
    }
    if (invalid) *(SATORI_GLOBAL uint32_t*)(bad) = 1u;
}

// Q6_K: thread per block of the chunk (blocks first .. first + count - 1 of the matrix's n). 210-byte blocks
// are 2-byte aligned, so the source is read as 16-bit words.
__global__ __launch_bounds__(256) void q6k_regroup_kernel(const uint8_t* __restrict__ packed, int64_t first,
                                                          int64_t count, int64_t n, uint8_t* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint8_t* block = packed + i * 210;
    const int64_t b = first + i;
    uint8_t* codes = out + b * 192;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int h = c >> 1, t = c & 1;
        // ql[64h + 16t, +16), ql[64h + 32 + 16t, +16), qh[32h + 16t, +16)
        const int starts[3] = {64 * h + 16 * t, 64 * h + 32 + 16 * t, 128 + 32 * h + 16 * t};
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            u32x4 v;
#pragma unroll
            for (int d = 0; d < 4; ++d)
                v[d] = load_u16(block + starts[s] + 4 * d) | (load_u16(block + starts[s] + 4 * d + 2) << 16);
            *(SATORI_GLOBAL u32x4*)(codes + 48 * c + 16 * s) = v;
        }
    }
    // Quarter c's scales sc[8h + 2k + t], k = 0..3, at 4c + k.
    u32x4 sc;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int h = c >> 1, t = c & 1;
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int at = 192 + 8 * h + 2 * k + t;  // byte at an even or odd offset of its 16-bit word
            const uint32_t pair = load_u16(block + (at & ~1));
            word |= ((at & 1) ? (pair >> 8) : (pair & 0xFFu)) << (8 * k);
        }
        sc[c] = word;
    }
    *(SATORI_GLOBAL u32x4*)(out + n * 192 + b * 16) = sc;
    *(SATORI_GLOBAL uint16_t*)(out + n * 208 + b * 2) = static_cast<uint16_t>(load_u16(block + 208));
}

// Q8_0 / Q4_0: thread per block of the chunk; the FP16 scale to the scale array, the codes to an aligned
// record (Q4_0 bytes XOR 0x88).
__global__ __launch_bounds__(256) void legacy_regroup_kernel(const uint8_t* __restrict__ packed, int64_t first,
                                                             int64_t count, int64_t n, int format,
                                                             uint8_t* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int record = legacy_record_bytes(format);
    const int block_bytes = record + 2;
    const uint8_t* block = packed + i * block_bytes;
    const int64_t b = first + i;
    const uint32_t flip = format == kQ4_0 ? 0x88888888u : 0u;
    for (int s = 0; s < record; s += 16) {
        u32x4 v;
#pragma unroll
        for (int d = 0; d < 4; ++d)
            v[d] = (load_u16(block + 2 + s + 4 * d) | (load_u16(block + 4 + s + 4 * d) << 16)) ^ flip;
        *(SATORI_GLOBAL u32x4*)(out + b * record + s) = v;
    }
    *(SATORI_GLOBAL uint16_t*)(out + n * record + b * 2) = static_cast<uint16_t>(load_u16(block));
}

int grid_for(int64_t threads) { return static_cast<int>((threads + 255) / 256); }

}  // namespace

hipError_t launch_t2_regroup(const uint8_t* packed, const T2Regroup& r, uint8_t* out, uint32_t* bad,
                             hipStream_t stream) {
    const int panels = (r.chunk_rows + kT2PanelRows - 1) / kT2PanelRows;
    const int64_t threads = static_cast<int64_t>(panels) * r.blocks * 64;
    if (threads <= 0) return hipSuccess;
    if ((threads + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
    t2_panels_kernel<<<grid_for(threads), 256, 0, stream>>>(packed, r, out, bad);
    return hipGetLastError();
}

hipError_t launch_q6k_regroup(const uint8_t* packed, int64_t first, int64_t count, int64_t n, uint8_t* out,
                              hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    if ((count + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
    q6k_regroup_kernel<<<grid_for(count), 256, 0, stream>>>(packed, first, count, n, out);
    return hipGetLastError();
}

hipError_t launch_legacy_regroup(const uint8_t* packed, int64_t first, int64_t count, int64_t n, int format,
                                 uint8_t* out, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    if ((count + 255) / 256 > INT32_MAX || (format != kQ8_0 && format != kQ4_0)) return hipErrorInvalidValue;
    legacy_regroup_kernel<<<grid_for(count), 256, 0, stream>>>(packed, first, count, n, format, out);
    return hipGetLastError();
}

}  // namespace satori
