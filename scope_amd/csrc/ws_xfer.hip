// Transfers of a decode step between HBM and pinned host memory by a copy
// kernel rather than the DMA engines: the query of a layer to the host
// partial.  Pinned host memory (hipHostMalloc) is mapped into the device's
// address space, so the kernel's loads and stores cross the host link
// directly.  Measured on MI355X in a 27-layer two-sided MLA loop (B 32, 590
// KB of query to the host and 1 MB of host partial back per layer, the host
// partial replaced by a 250 us spin): 336 us per layer with DMA copies both
// ways, 314 with this kernel both ways, 312 with this kernel for the query
// and the merge reading the host partial from pinned memory in place (265
// with no transfers).  A DMA copy's set-up latency is paid on every layer's
// critical path.
#include <algorithm>

#include "ws_common.h"

namespace ws {

constexpr int kXferThreads = 256;
constexpr int kXferMaxBlocks = 1024;

// dst[i] = src[i] for 16-byte units i < n16, then the 4-byte tail (n4 words
// after them).
__global__ __launch_bounds__(kXferThreads) void copy_kernel(u32x4* __restrict__ dst,
                                                            const u32x4* __restrict__ src,
                                                            size_t n16, int n4) {
  const size_t stride = (size_t)gridDim.x * kXferThreads;
  for (size_t i = (size_t)blockIdx.x * kXferThreads + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
  if (blockIdx.x == 0 && (int)threadIdx.x < n4)
    ((uint32_t*)(dst + n16))[threadIdx.x] = ((const uint32_t*)(src + n16))[threadIdx.x];
}

}  // namespace ws

using namespace ws;

extern "C" int ws_copy(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return WS_OK;
  if (!dst || !src) return set_error(WS_EINVAL, "ws_copy: null pointer");
  if (((uintptr_t)dst & 15u) || ((uintptr_t)src & 15u) || (bytes & 3u))
    return set_error(WS_EINVAL,
                     "ws_copy: pointers must be 16-byte aligned and bytes a multiple of 4 "
                     "(got %zu)", bytes);
  const char* s = (const char*)src;
  char* d = (char*)dst;
  if ((s < d && s + bytes > d) || (d < s && d + bytes > s) || s == d)
    return set_error(WS_EINVAL, "ws_copy: source and destination overlap");
  const size_t n16 = bytes / 16;
  const int n4 = (int)((bytes % 16) / 4);
  const size_t want = (n16 + kXferThreads - 1) / kXferThreads;
  const int blocks = (int)std::max<size_t>(1, std::min<size_t>(want, kXferMaxBlocks));
  hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(kXferThreads), 0, (hipStream_t)stream,
                     (u32x4*)dst, (const u32x4*)src, n16, n4);
  return check_launch("ws_copy");
}
