// Append kernels: copy each sequence's new token(s) into its HBM page slot.
//
// Grid (sequence, chunk of kChunkVecs 16-byte vectors).  A decode step's
// append (one token) is one chunk per sequence: that workgroup is the only
// reader of gpu_len[b], so it bumps the length after a barrier.  A longer
// append (prefill into the partition) spreads over many chunks, which all
// read the old length, and len_add_kernel bumps it afterwards on the same
// stream.
//
// A sequence's append is all or nothing: if its length is negative (an
// earlier error) or any slot [len, len + n_new) lies past the page table's
// capacity or in a page id outside the pool, none of its tokens is written
// and its length becomes -1 (with update_len), which every later decode
// call turns into NaN outputs for that sequence.
#include "ws_common.h"

namespace ws {

constexpr int kChunkVecs = 256 * 8;  // 32 KB of each tensor per workgroup

// Whether every slot [len, len + n_new) of the sequence whose page-table row
// is pt_row lies in a page of the pool.  Every thread of the workgroup must
// call it; the result is the same in all of them.
__device__ __forceinline__ bool append_ok(const int32_t* __restrict__ pt_row, int len,
                                          int n_new, int page_size, int max_pages,
                                          int num_pages) {
  if (len < 0 || (long long)len + n_new > (long long)page_size * max_pages) return false;
  const int p0 = len / page_size;
  const int p1 = (len + n_new - 1) / page_size;
  int bad = 0;
  for (int pg = p0 + (int)threadIdx.x; pg <= p1; pg += blockDim.x) {
    const int pid = pt_row[pg];
    bad |= (pid < 0 || pid >= num_pages);
  }
  return !__syncthreads_or(bad);
}

// Length update of a multi-chunk append: one workgroup per sequence.
__global__ __launch_bounds__(256) void len_add_kernel(int32_t* __restrict__ gpu_len,
                                                      const int32_t* __restrict__ page_table,
                                                      int n_new, int page_size, int max_pages,
                                                      int num_pages) {
  const int b = blockIdx.x;
  const int len = gpu_len[b];
  const bool ok = append_ok(page_table + (size_t)b * max_pages, len, n_new, page_size,
                            max_pages, num_pages);
  __syncthreads();  // every thread has read gpu_len[b]
  if (threadIdx.x == 0) gpu_len[b] = ok ? len + n_new : -1;
}

__global__ __launch_bounds__(256) void kv_append_kernel(
    const u32x4* __restrict__ k_new, const u32x4* __restrict__ v_new,
    u32x4* __restrict__ k_pages, u32x4* __restrict__ v_pages,
    const int32_t* __restrict__ page_table, int32_t* __restrict__ gpu_len,
    int Hkv, int dvec, int n_new, int page_size, int max_pages, int num_pages,
    int update_len) {
  const int b = blockIdx.x;
  const int len = gpu_len[b];
  const bool ok = append_ok(page_table + (size_t)b * max_pages, len, n_new, page_size,
                            max_pages, num_pages);
  const int per_token = Hkv * dvec;     // vectors of one token of one tensor
  const int total = ok ? n_new * per_token : 0;  // vectors of one tensor
  const int end = min(total, (int)(blockIdx.y + 1) * kChunkVecs);
  for (int idx = blockIdx.y * kChunkVecs + threadIdx.x; idx < end; idx += blockDim.x) {
    // source order [Hkv][n_new][dvec]
    const int dv = idx % dvec;
    const int rest = idx / dvec;
    const int i = rest % n_new;
    const int h = rest / n_new;
    const int pos = len + i;
    const int page = pos / page_size;
    const int pid = page_table[(size_t)b * max_pages + page];  // checked by append_ok
    const size_t src = (((size_t)b * Hkv + h) * n_new + i) * dvec + dv;
    const size_t dst =
        (((size_t)pid * Hkv + h) * page_size + (pos % page_size)) * dvec + dv;
    k_pages[dst] = k_new[src];
    v_pages[dst] = v_new[src];
  }
  if (update_len) {
    __syncthreads();
    if (threadIdx.x == 0) gpu_len[b] = ok ? len + n_new : -1;
  }
}

constexpr int kLatent = 576;
constexpr int kLatentC = 512;

__global__ __launch_bounds__(256) void latent_append_kernel(
    const u32x4* __restrict__ c_new, int64_t c_stride_vec,
    const u32x4* __restrict__ pe_new, int64_t pe_stride_vec,
    u32x4* __restrict__ latent_pages, const int32_t* __restrict__ page_table,
    int32_t* __restrict__ gpu_len, int n_new, int page_size, int max_pages,
    int num_pages, int update_len) {
  const int b = blockIdx.x;
  const int len = gpu_len[b];
  const bool ok = append_ok(page_table + (size_t)b * max_pages, len, n_new, page_size,
                            max_pages, num_pages);
  constexpr int vec_row = kLatent / 8;    // 72 vectors per token
  constexpr int vec_c = kLatentC / 8;     // 64 of them from c_kv
  const int total = ok ? n_new * vec_row : 0;
  const int end = min(total, (int)(blockIdx.y + 1) * kChunkVecs);
  for (int idx = blockIdx.y * kChunkVecs + threadIdx.x; idx < end; idx += blockDim.x) {
    const int v = idx % vec_row;
    const int i = idx / vec_row;
    const int pos = len + i;
    const int page = pos / page_size;
    const int pid = page_table[(size_t)b * max_pages + page];  // checked by append_ok
    const size_t row = (size_t)b * n_new + i;
    const u32x4 val = (v < vec_c) ? c_new[row * c_stride_vec + v]
                                  : pe_new[row * pe_stride_vec + (v - vec_c)];
    latent_pages[((size_t)pid * page_size + (pos % page_size)) * vec_row + v] =
        val;
  }
  if (update_len) {
    __syncthreads();
    if (threadIdx.x == 0) gpu_len[b] = ok ? len + n_new : -1;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Chunks per sequence of an append moving `vecs` vectors per sequence; 0 if
// the grid would be too tall.
static int append_chunks(long long vecs) {
  const long long c = (vecs + kChunkVecs - 1) / kChunkVecs;
  return c > 65535 ? 0 : (int)c;
}

}  // namespace ws

using namespace ws;

extern "C" int ws_kv_append(const uint16_t* k_new, const uint16_t* v_new,
                            uint16_t* k_pages, uint16_t* v_pages,
                            const int32_t* page_table, int32_t* gpu_len, int B,
                            int Hkv, int D, int n_new, int page_size,
                            int max_pages, int num_pages, int update_len,
                            void* stream) {
  if (!k_new || !v_new || !k_pages || !v_pages || !page_table || !gpu_len)
    return set_error(WS_EINVAL, "ws_kv_append: null pointer");
  if (B < 0 || Hkv <= 0 || D <= 0 || D % 8 != 0 || n_new < 0 ||
      page_size <= 0 || max_pages <= 0 || num_pages <= 0)
    return set_error(WS_EINVAL,
                     "ws_kv_append: bad sizes B=%d Hkv=%d D=%d n_new=%d "
                     "page_size=%d max_pages=%d num_pages=%d",
                     B, Hkv, D, n_new, page_size, max_pages, num_pages);
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_pages) ||
      !aligned16(v_pages))
    return set_error(WS_EINVAL, "ws_kv_append: bf16 buffers must be 16-byte aligned");
  if (B == 0 || n_new == 0) return WS_OK;
  const int chunks = append_chunks((long long)n_new * Hkv * (D / 8));
  if (chunks == 0) return set_error(WS_EINVAL, "ws_kv_append: %d tokens in one call", n_new);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(kv_append_kernel, dim3(B, chunks), dim3(256), 0, s, (const u32x4*)k_new,
                     (const u32x4*)v_new, (u32x4*)k_pages, (u32x4*)v_pages, page_table,
                     gpu_len, Hkv, D / 8, n_new, page_size, max_pages, num_pages,
                     chunks == 1 ? update_len : 0);
  if (update_len && chunks > 1)
    hipLaunchKernelGGL(len_add_kernel, dim3(B), dim3(256), 0, s, gpu_len, page_table, n_new,
                       page_size, max_pages, num_pages);
  return check_launch("ws_kv_append");
}

extern "C" int ws_latent_append(const uint16_t* c_new, int64_t c_stride,
                                const uint16_t* pe_new, int64_t pe_stride,
                                uint16_t* latent_pages,
                                const int32_t* page_table, int32_t* gpu_len,
                                int B, int n_new, int page_size, int max_pages,
                                int num_pages, int update_len, void* stream) {
  if (!c_new || !pe_new || !latent_pages || !page_table || !gpu_len)
    return set_error(WS_EINVAL, "ws_latent_append: null pointer");
  if (B < 0 || n_new < 0 || page_size <= 0 || max_pages <= 0 ||
      num_pages <= 0 || c_stride < 512 || pe_stride < 64 || c_stride % 8 ||
      pe_stride % 8)
    return set_error(WS_EINVAL,
                     "ws_latent_append: bad sizes B=%d n_new=%d page_size=%d "
                     "max_pages=%d num_pages=%d c_stride=%lld pe_stride=%lld",
                     B, n_new, page_size, max_pages, num_pages,
                     (long long)c_stride, (long long)pe_stride);
  if (!aligned16(c_new) || !aligned16(pe_new) || !aligned16(latent_pages))
    return set_error(WS_EINVAL,
                     "ws_latent_append: bf16 buffers must be 16-byte aligned");
  if (B == 0 || n_new == 0) return WS_OK;
  const int chunks = append_chunks((long long)n_new * (kLatent / 8));
  if (chunks == 0) return set_error(WS_EINVAL, "ws_latent_append: %d tokens in one call", n_new);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(latent_append_kernel, dim3(B, chunks), dim3(256), 0, s,
                     (const u32x4*)c_new, c_stride / 8, (const u32x4*)pe_new, pe_stride / 8,
                     (u32x4*)latent_pages, page_table, gpu_len, n_new, page_size, max_pages,
                     num_pages, chunks == 1 ? update_len : 0);
  if (update_len && chunks > 1)
    hipLaunchKernelGGL(len_add_kernel, dim3(B), dim3(256), 0, s, gpu_len, page_table, n_new,
                       page_size, max_pages, num_pages);
  return check_launch("ws_latent_append");
}
