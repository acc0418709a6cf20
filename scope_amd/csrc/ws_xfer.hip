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

namespace ws {

constexpr int kPageChunk = kXferThreads * 8 * 16;  // bytes of a page one workgroup moves
// Default bound of a page copy's grid: eight workgroups per CU keep an
// HBM-to-HBM copy at the memory rate; each loops over the units beyond it.
constexpr int kCopyPagesMaxBlocks = 2048;

// Page copies of a boundary move: for every layer l and listed page i,
// dst page dst_ids[i] of layer l = src page src_ids[i] of layer l, in units
// of one kPageChunk-byte chunk of one page of one layer (unit u: layer
// u / (n_pages * chunks), then page, then chunk), the grid striding over
// the units.  Each thread moves eight 16-byte units of a chunk, all loads in
// flight before the stores.  The ids live in device memory, so the launcher
// cannot check them: a listed id outside [0, num_pages) moves nothing
// (scope_amd/ops.py copy_pages refuses such ids before the launch).
__global__ __launch_bounds__(kXferThreads) void copy_pages_kernel(
    char* __restrict__ dst, long long dst_layer_stride, const int32_t* __restrict__ dst_ids,
    int dst_num_pages, const char* __restrict__ src, long long src_layer_stride,
    const int32_t* __restrict__ src_ids, int src_num_pages, int n_pages, int chunks,
    long long page_bytes, long long units) {
  const long long per_layer = (long long)n_pages * chunks;
  for (long long u = blockIdx.x; u < units; u += gridDim.x) {
    const long long l = u / per_layer;
    const int r = (int)(u - l * per_layer);
    const int i = r / chunks;
    const int c = r - i * chunks;
    const int d = dst_ids[i];
    const int s = src_ids[i];
    if (d < 0 || d >= dst_num_pages || s < 0 || s >= src_num_pages) continue;
    const long long off = (long long)c * kPageChunk;
    const u32x4* sp = (const u32x4*)(src + l * src_layer_stride + s * page_bytes + off);
    u32x4* dp = (u32x4*)(dst + l * dst_layer_stride + d * page_bytes + off);
    const int n16 = (int)(std::min<long long>(kPageChunk, page_bytes - off) / 16);
    u32x4 v[8];
#pragma unroll
    for (int k8 = 0; k8 < 8; ++k8) {
      const int k = k8 * kXferThreads + threadIdx.x;
      if (k < n16) v[k8] = sp[k];
    }
#pragma unroll
    for (int k8 = 0; k8 < 8; ++k8) {
      const int k = k8 * kXferThreads + threadIdx.x;
      if (k < n16) dp[k] = v[k8];
    }
  }
}

}  // namespace ws

extern "C" int ws_copy_pages(void* dst, long long dst_layer_stride, const int32_t* dst_ids,
                             int dst_num_pages, const void* src, long long src_layer_stride,
                             const int32_t* src_ids, int src_num_pages, int n_pages,
                             int n_layers, long long page_bytes, int max_workgroups,
                             void* stream) {
  static const char* name = "ws_copy_pages";
  if (n_pages == 0 || n_layers == 0) return WS_OK;
  if (!dst || !src || !dst_ids || !src_ids)
    return set_error(WS_EINVAL, "%s: null pointer", name);
  if (n_pages < 0 || n_layers < 0 || page_bytes <= 0 || page_bytes % 16 ||
      dst_num_pages <= 0 || src_num_pages <= 0 || max_workgroups < 0)
    return set_error(WS_EINVAL,
                     "%s: bad sizes n_pages=%d n_layers=%d page_bytes=%lld max_workgroups=%d",
                     name, n_pages, n_layers, page_bytes, max_workgroups);
  if (((uintptr_t)dst & 15u) || ((uintptr_t)src & 15u) || dst_layer_stride % 16 ||
      src_layer_stride % 16)
    return set_error(WS_EINVAL, "%s: pools and layer strides must be 16-byte aligned", name);
  const long long chunks = (page_bytes + kPageChunk - 1) / kPageChunk;
  if ((long long)n_pages * chunks > 0x7fffffffLL)
    return set_error(WS_EINVAL, "%s: %d pages of %lld bytes exceed the chunk index range", name,
                     n_pages, page_bytes);
  const long long units = (long long)n_pages * chunks * n_layers;
  const int cap = max_workgroups > 0 ? max_workgroups : kCopyPagesMaxBlocks;
  const int grid = (int)std::min<long long>(units, cap);
  hipLaunchKernelGGL(copy_pages_kernel, dim3(grid), dim3(kXferThreads), 0, (hipStream_t)stream,
                     (char*)dst, dst_layer_stride, dst_ids, dst_num_pages, (const char*)src,
                     src_layer_stride, src_ids, src_num_pages, n_pages, (int)chunks, page_bytes,
                     units);
  return check_launch(name);
}
