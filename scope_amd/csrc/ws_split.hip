// Workgroup count choice and the standalone split reduction.
//
// split_reduce_kernel combines per-split partials [split][row][Dv] for
// callers that schedule their own splits, with one 64-thread workgroup per
// (row, 256-column chunk): the row's split weights are computed once per
// workgroup from the lse values, then every lane accumulates one float4
// column over the splits with eight loads in flight.
#include <math.h>

#include "ws_reduce.h"

namespace ws {

constexpr int kSplitChunk4 = 64;  // float4 columns per workgroup

__global__ __launch_bounds__(64) void split_reduce_kernel(
    const float* __restrict__ part_out, const float* __restrict__ part_lse,
    const int32_t* __restrict__ gpu_len, int len_add, int rows, int heads_per_len,
    int Dv, int n_splits, int tokens_per_split, int untouched_single,
    float* __restrict__ out, float* __restrict__ lse) {
  __shared__ float s_w[kReduceMaxWeights];
  __shared__ float s_ML[2];
  const int row = blockIdx.x;
  const int chunk = blockIdx.y;
  const int t = threadIdx.x;
  const int c4 = Dv >> 2;
  const int c = chunk * kSplitChunk4 + t;
  const int len0 = gpu_len[row / heads_per_len];
  const int len = len0 + len_add;
  int n = len > 0 ? (len + tokens_per_split - 1) / tokens_per_split : 0;
  if (n > n_splits) n = n_splits;
  if (n == 1 && untouched_single) return;
  if (n == 0) {  // empty: (0, -inf); a negative length is an error: NaN
    const float v = len0 < 0 ? qnan() : 0.f;
    if (c < c4) ((float4*)out)[(size_t)row * c4 + c] = make_float4(v, v, v, v);
    if (chunk == 0 && t == 0) lse[row] = len0 < 0 ? qnan() : neg_inf();
    return;
  }
  float mx = neg_inf();
  for (int s = t; s < n; s += 64) {
    const float v = part_lse[(size_t)s * rows + row];
    s_w[s] = v;
    mx = max_nan(mx, v);
  }
  for (int o = 1; o < 64; o <<= 1) mx = max_nan(mx, __shfl_xor(mx, o));
  float sum = 0.f;
  for (int s = t; s < n; s += 64) {
    const float w = __expf(s_w[s] - mx);
    s_w[s] = w;
    sum += w;
  }
  for (int o = 1; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
  if (t == 0) {
    s_ML[0] = mx;
    s_ML[1] = sum;
  }
  __syncthreads();
  if (chunk == 0 && t == 0) lse[row] = mx + __logf(sum);
  if (c >= c4) return;
  const float4* src = (const float4*)part_out + (size_t)row * c4 + c;
  const size_t sstride = (size_t)rows * c4;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  int s = 0;
  for (; s + 8 <= n; s += 8) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[(size_t)(s + u) * sstride];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float w = s_w[s + u];
      a.x += w * v[u].x; a.y += w * v[u].y; a.z += w * v[u].z; a.w += w * v[u].w;
    }
  }
  for (; s < n; ++s) {
    const float w = s_w[s];
    const float4 v = src[(size_t)s * sstride];
    a.x += w * v.x; a.y += w * v.y; a.z += w * v.z; a.w += w * v.w;
  }
  const float inv = 1.f / s_ML[1];
  ((float4*)out)[(size_t)row * c4 + c] =
      make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
}

// Compute units of each device, read once (a device property, not state).
static int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int choose_workgroups(int n_workgroups, int per_cu, long long max_blocks, int min_blocks) {
  if (n_workgroups > 0) return n_workgroups;
  long long n = (long long)per_cu * cu_count();
  const long long feed = (max_blocks + min_blocks - 1) / min_blocks;
  if (feed < n) n = feed;
  return n < 1 ? 1 : (int)n;
}

static int launch_split_reduce(const float* part_out, const float* part_lse,
                               const int32_t* gpu_len, int len_add, int rows,
                               int heads_per_len, int Dv, int n_splits, int tps,
                               int untouched_single, float* out, float* lse,
                               hipStream_t stream) {
  const int chunks = ((Dv >> 2) + kSplitChunk4 - 1) / kSplitChunk4;
  hipLaunchKernelGGL(split_reduce_kernel, dim3(rows, chunks), dim3(64), 0, stream,
                     part_out, part_lse, gpu_len, len_add, rows, heads_per_len, Dv,
                     n_splits, tps, untouched_single, out, lse);
  return check_launch("split_reduce");
}

}  // namespace ws

using namespace ws;

extern "C" int ws_split_reduce(const float* part_out, const float* part_lse,
                               const int32_t* gpu_len, int rows, int heads_per_len,
                               int Dv, int n_splits, int tokens_per_split, float* out,
                               float* lse, void* stream) {
  if (!part_out || !part_lse || !gpu_len || !out || !lse)
    return set_error(WS_EINVAL, "ws_split_reduce: null pointer");
  if (rows < 0 || heads_per_len <= 0 || Dv <= 0 || Dv % 4 || n_splits <= 0 ||
      n_splits > kReduceMaxWeights || tokens_per_split <= 0)
    return set_error(WS_EINVAL, "ws_split_reduce: bad sizes");
  if (((uintptr_t)part_out | (uintptr_t)out) & 15u)
    return set_error(WS_EINVAL, "ws_split_reduce: buffers must be 16-byte aligned");
  if (rows == 0) return WS_OK;
  return launch_split_reduce(part_out, part_lse, gpu_len, 0, rows, heads_per_len, Dv,
                             n_splits, tokens_per_split, 1, out, lse,
                             (hipStream_t)stream);
}
