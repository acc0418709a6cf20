// Cross-workgroup split reduction shared by the decode kernels.
//
// A decode call splits every row's tokens into tokens_per_split chunks; each
// chunk's workgroup produces a partial (out normalised fp32, lse natural log).
// When a row has more than one chunk, each workgroup stores its partial in the
// workspace and bumps the row's arrival counter; the workgroup that arrives
// last combines all partials of the row (reduce_rows) and resets the counter
// to zero, so the workspace needs zeroed counters only once, before its first
// use.
//
// Workspace layout (ws_decode_workspace_bytes), for a call over rows_kv rows
// of `heads` output rows each, run by n workgroups:
//   [counters int32 x kCounterSlots]
//   [slot lse f32 x (n + rows_kv) x heads, padded to 256 B]
//   [slot out f32 x (n + rows_kv) x heads x Dv]
// (slot = workgroup + row, ws_plan.h).  The counter block has a fixed size,
// so calls of any shape that share one workspace never write partials over
// another call's counters.
#pragma once

#include "ws_common.h"

namespace ws {

// Most (partial, row) weights one reduction keeps in LDS.
constexpr int kReduceMaxWeights = 4096;
// Arrival counters at the head of every workspace (one per kv row).
constexpr int kCounterSlots = 16384;

__host__ __device__ inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct SplitWorkspace {
  int32_t* counters;
  float* part_lse;
  float* part_out;
};

__host__ __device__ inline size_t workspace_bytes(int rows_kv, int heads, int Dv, int n) {
  const size_t slots = (size_t)n + rows_kv;
  return (size_t)kCounterSlots * 4 + align256(slots * heads * 4) + slots * heads * Dv * 4;
}

__host__ __device__ inline SplitWorkspace carve_workspace(void* base, int rows_kv,
                                                          int heads, int n) {
  SplitWorkspace w;
  char* p = (char*)base;
  const size_t slots = (size_t)n + rows_kv;
  w.counters = (int32_t*)p;
  p += (size_t)kCounterSlots * 4;
  w.part_lse = (float*)p;
  p += align256(slots * heads * 4);
  w.part_out = (float*)p;
  return w;
}

// Workgroups of a decode call: n_workgroups, or the library's choice (0):
// `per_cu` resident workgroups on every CU of the current device, but no more
// than the call's 32-token blocks can feed with `min_blocks` each.
int choose_workgroups(int n_workgroups, int per_cu, long long max_blocks, int min_blocks);
// Workgroups of an MLA call (ws_mla.hip).
int mla_workgroups(int n_workgroups, int B, int max_len);
// Combines the pieces of a split decode step with no host partial: rows held
// by several splits are LSE-combined from the workspace, the others copied;
// lengths are len[b] + len_add; out/lse may alias out_g/lse_g (Dv <= 256).
// Launches on `stream`; returns WS_OK or an error code (ws_merge.hip).
int merge_split_pieces(const int32_t* len, int len_add, int B, int R, int heads, int Dv,
                       int cap, int n, const float* out_g, const float* lse_g,
                       const SplitWorkspace& w, float* out, float* lse, hipStream_t stream);

// Partials travel between workgroups (possibly on different XCDs, whose L2
// caches are not coherent with each other) through device-scope atomic
// stores and loads: each access is coherent by itself, so no cache-wide
// writeback or invalidate is needed.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of a workgroup after it stored its partial with
// st_agent.  Returns true in the workgroup that stored the row's last
// partial; that workgroup then reads every partial with ld_agent.  Each wave
// first waits until its own stores have completed, so the arrival count is
// bumped only after the whole workgroup's partial is visible device-wide.
// `flag` is an LDS int.
__device__ __forceinline__ bool arrive_last(int32_t* counter, int n_arrivals,
                                            int* flag) {
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    *flag = (prev == n_arrivals - 1);
  }
  __syncthreads();
  return *flag != 0;
}

// LSE-combine n partials of nrows rows, stored by other workgroups with
// st_agent: partial s of row r is out po[(s * slot_rows + r) * Dv .. + Dv],
// lse pl[s * slot_rows + r]; the result goes to out[r * Dv ..], lse[r].
// nrows in {1, 2, 4, 8, 16}; Dv % 4 == 0; n * nrows <= kReduceMaxWeights.
// sw: LDS of n * nrows floats; sred: LDS of 32 * (NT / 64) + 32 floats.
// Kept out of line: its 32 loads in flight would otherwise share the register
// budget of the decode loop it is called from.
template <int NT>
__device__ __noinline__ void reduce_rows(const float* __restrict__ po, const float* __restrict__ pl,
                            int slot_rows, int nrows, int Dv, int n,
                            float* __restrict__ out, float* __restrict__ lse,
                            float* sw, float* sred) {
  constexpr int NW = NT / 64;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  float* s_max = sred;                // [NW][16]
  float* s_sum = sred + 16 * NW;      // [NW][16]
  float* s_M = sred + 32 * NW;        // [16]
  float* s_L = s_M + 16;              // [16]
  const int total = n * nrows;

  // Since NT is a multiple of nrows, thread t always meets row t % nrows.
  float mx = neg_inf();
  for (int idx = t; idx < total; idx += NT) {
    const int s = idx / nrows;
    const int r = idx - s * nrows;
    const float v = ld_agent(pl + (size_t)s * slot_rows + r);
    sw[idx] = v;
    mx = fmaxf(mx, v);
  }
  for (int o = nrows; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane < nrows) s_max[wave * 16 + lane] = mx;
  __syncthreads();
  if (t < nrows) {
    float M = neg_inf();
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_max[w * 16 + t]);
    s_M[t] = M;
  }
  __syncthreads();

  float sum = 0.f;
  const float Mr = s_M[t % nrows];
  for (int idx = t; idx < total; idx += NT) {
    const float w = __expf(sw[idx] - Mr);
    sw[idx] = w;
    sum += w;
  }
  for (int o = nrows; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
  if (lane < nrows) s_sum[wave * 16 + lane] = sum;
  __syncthreads();
  if (t < nrows) {
    float L = 0.f;
    for (int w = 0; w < NW; ++w) L += s_sum[w * 16 + t];
    s_L[t] = L;
    lse[t] = s_M[t] + __logf(L);
  }
  __syncthreads();

  const int c4 = Dv >> 2;
  const size_t sstride = (size_t)slot_rows * Dv;
  for (int idx = t; idx < nrows * c4; idx += NT) {
    const int r = idx / c4;
    const int c = idx - r * c4;
    const float* src = po + (size_t)r * Dv + 4 * c;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    int s = 0;
    // eight partials (32 independent loads) in flight per round
    for (; s + 8 <= n; s += 8) {
      float v[8][4];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) v[u][k] = ld_agent(src + (size_t)(s + u) * sstride + k);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float w = sw[(s + u) * nrows + r];
        a.x += w * v[u][0]; a.y += w * v[u][1]; a.z += w * v[u][2]; a.w += w * v[u][3];
      }
    }
    for (; s < n; ++s) {
      const float w = sw[s * nrows + r];
      const float* v = src + (size_t)s * sstride;
      a.x += w * ld_agent(v); a.y += w * ld_agent(v + 1);
      a.z += w * ld_agent(v + 2); a.w += w * ld_agent(v + 3);
    }
    const float inv = 1.f / s_L[r];
    ((float4*)out)[(size_t)r * c4 + c] =
        make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
  }
}

}  // namespace ws
