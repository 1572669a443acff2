// The host-buffer calls' vector copies as a kernel: the GPU reads the pinned input staging buffer, or writes
// the pinned output staging buffer, over the host link itself (every hipHostMalloc allocation is mapped into
// the device's address space). For the few kilobytes a MatVec moves this is one launch on the call's stream
// instead of a copy-engine transfer.
#include "device_common.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

// Thread i copies words 4i .. 4i + 3 (one 16-byte access when all four are in range).
__global__ __launch_bounds__(256) void copy_words_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                         int64_t words) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i + 4 <= words) {
        *reinterpret_cast<u32x4*>(dst + i) = *reinterpret_cast<const u32x4*>(src + i);
    } else {
        for (int64_t k = i; k < words; ++k) dst[k] = src[k];
    }
}

}  // namespace

hipError_t launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    if (bytes % 4 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0 ||
        bytes > kKernelCopyMaxBytes)
        return hipErrorInvalidValue;
    const int64_t words = static_cast<int64_t>(bytes / 4);
    const int grid = static_cast<int>((words + 1023) / 1024);
    copy_words_kernel<<<grid, 256, 0, stream>>>(static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), words);
    return hipGetLastError();
}

}  // namespace satori
