// Device check of the GGUF block scales of an uploaded matrix: the finiteness rule of
// QuantizedMatVec.ValidatePayload (src/Satori.Core/QuantizedMatVec.cs:28-42) with Q4KCodec.AreScalesFinite
// (src/Satori.Core/Q4KCodec.cs:91-93) and Q6KCodec.AreScalesFinite (src/Satori.Core/Q6KCodec.cs:84-85),
// run over the device copy so a large tensor is checked at HBM speed instead of by a host pass.
#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

__device__ __forceinline__ bool half_nonfinite(uint32_t h) { return ((h >> 10) & 0x1Fu) == 0x1Fu; }

__device__ __forceinline__ uint32_t load_u16(const uint8_t* p) {
    return *(const SATORI_GLOBAL uint16_t*)(p);
}

// Blocks of the device layout: Q4_K (144 B) as uploaded; Q6_K, Q8_0 and Q4_0 regrouped, with the FP16 scale
// of every block in one array after the codes (and, for Q6_K, the sub-block scales). A block with a non-finite scale
// stores its index + 1 into *flag (any one of them: the caller reports the first from the host copy).
__global__ __launch_bounds__(256) void scale_check_kernel(const uint8_t* __restrict__ payload, int64_t blocks,
                                                          int format, uint32_t* __restrict__ flag) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < blocks; i += stride) {
        bool bad;
        if (format == kQ6_K) {
            bad = half_nonfinite(load_u16(payload + blocks * 208 + 2 * i));
        } else if (format == kQ4_K) {
            const uint8_t* b = payload + 144 * i;
            bad = half_nonfinite(load_u16(b)) || half_nonfinite(load_u16(b + 2));
        } else {  // Q8_0 / Q4_0 regrouped: the FP16 scales follow the code records
            bad = half_nonfinite(load_u16(payload + blocks * legacy_record_bytes(format) + 2 * i));
        }
        if (bad) *(SATORI_GLOBAL uint32_t*)(flag) = static_cast<uint32_t>(i) + 1u;
    }
}

}  // namespace

hipError_t launch_scale_check(const uint8_t* payload, int64_t blocks, int format, uint32_t* flag, hipStream_t stream) {
    if (blocks <= 0) return hipSuccess;
    const int64_t groups = (blocks + 255) / 256;
    const int grid = static_cast<int>(groups < 8192 ? groups : 8192);
    scale_check_kernel<<<grid, 256, 0, stream>>>(payload, blocks, format, flag);
    return hipGetLastError();
}

}  // namespace satori
