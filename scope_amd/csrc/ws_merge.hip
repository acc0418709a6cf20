// LSE merge of the GPU partial with a second (host) partial, fused with the
// final normalisation and the bf16 cast.  One workgroup per row, one float4
// of the output per thread.  The second operand may arrive in any of the
// reference CPU kernels' output conventions, so no conversion launch is
// needed after its host-to-device copy.
#include <math.h>

#include "ws_plan.h"
#include "ws_reduce.h"

namespace ws {

template <int FMT>
__device__ __forceinline__ void load_b(const void* b_out, const void* aux0,
                                       const void* aux1, int row, int Dv, int c,
                                       float& lse_b, float4& o_b) {
  if (FMT == WS_PARTIAL_LSE_F32) {
    lse_b = ((const float*)aux0)[row];
    o_b = ((const float4*)((const float*)b_out + (size_t)row * Dv))[c];
  } else if (FMT == WS_PARTIAL_LSE_BF16) {
    lse_b = ((const float*)aux0)[row];
    const uint2 raw = ((const uint2*)((const uint16_t*)b_out + (size_t)row * Dv))[c];
    o_b = make_float4(bf16_to_f32(raw.x & 0xffffu), bf16_to_f32(raw.x >> 16),
                      bf16_to_f32(raw.y & 0xffffu), bf16_to_f32(raw.y >> 16));
  } else if (FMT == WS_TRIPLE_UNNORM_F32 || FMT == WS_TRIPLE_NORM_F32) {
    const float m = ((const float*)aux0)[row];
    const float s = ((const float*)aux1)[row];
    lse_b = (s == 0.f) ? neg_inf() : m + __logf(s);
    o_b = ((const float4*)((const float*)b_out + (size_t)row * Dv))[c];
    if (FMT == WS_TRIPLE_UNNORM_F32) {
      const float inv = (s > 0.f) ? 1.f / s : 0.f;
      o_b.x *= inv;
      o_b.y *= inv;
      o_b.z *= inv;
      o_b.w *= inv;
    }
  } else {  // WS_TRIPLE_NORM_BF16
    const float m = bf16_to_f32(((const uint16_t*)aux0)[row]);
    const float s = bf16_to_f32(((const uint16_t*)aux1)[row]);
    lse_b = (s == 0.f) ? neg_inf() : m + __logf(s);
    const uint2 raw =
        ((const uint2*)((const uint16_t*)b_out + (size_t)row * Dv))[c];
    o_b = make_float4(bf16_to_f32(raw.x & 0xffffu), bf16_to_f32(raw.x >> 16),
                      bf16_to_f32(raw.y & 0xffffu), bf16_to_f32(raw.y >> 16));
  }
}

template <int FMT>
__global__ __launch_bounds__(128) void lse_merge_kernel(
    const float* __restrict__ out_g, const float* __restrict__ lse_g,
    const void* __restrict__ b_out, const void* __restrict__ b_aux0,
    const void* __restrict__ b_aux1, uint16_t* __restrict__ out_bf16,
    float* __restrict__ out_f32, float* __restrict__ lse_out, int Dv) {
  const int row = blockIdx.x;
  const int c = threadIdx.x;
  if (c >= Dv / 4) return;
  const float la = lse_g[row];
  float lb;
  float4 ob;
  load_b<FMT>(b_out, b_aux0, b_aux1, row, Dv, c, lb, ob);
  const float M = max_nan(la, lb);
  float4 r;
  float lse_r;
  if (M == neg_inf()) {
    r = make_float4(0.f, 0.f, 0.f, 0.f);
    lse_r = neg_inf();
  } else {
    const float wa = __expf(la - M);
    const float wb = __expf(lb - M);
    const float inv = 1.f / (wa + wb);
    const float4 oa = ((const float4*)(out_g + (size_t)row * Dv))[c];
    // An empty side has weight 0; its (0) output must not turn into NaN.
    const float fa = wa * inv, fb = wb * inv;
    r = make_float4(fa * oa.x + fb * ob.x, fa * oa.y + fb * ob.y,
                    fa * oa.z + fb * ob.z, fa * oa.w + fb * ob.w);
    lse_r = M + __logf(wa + wb);
  }
  if (out_f32) ((float4*)(out_f32 + (size_t)row * Dv))[c] = r;
  if (out_bf16) {
    uint2 packed;
    packed.x = pack_bf16x2(r.x, r.y);
    packed.y = pack_bf16x2(r.z, r.w);
    ((uint2*)(out_bf16 + (size_t)row * Dv))[c] = packed;
  }
  if (lse_out && c == 0) lse_out[row] = lse_r;
}

// ---------------------------------------------------------------------------
// Split combine + host merge of a deferred-combine decode step.
//
// One 64-lane workgroup per output row (kv row * heads + head) and 256-column
// chunk.  It rebuilds
// the step's plan from the post-step lengths (ws_plan.h) to find the row's
// GPU pieces: the final (out, lse) the step wrote when one workgroup held the
// row, else the partials of the row's workgroups (slots w + kv row), then
// LSE-combines them with the host partial (format FMT, or none when FMT < 0)
// and writes the normalised result.  Runs after the step on the same stream,
// so plain loads see its writes.
struct MergeSplitParams {
  const int32_t* gpu_len;
  // B: plan sequences; ng > 1 for absorbed MLA with H = 16 ng heads, whose
  // plan sequences are (sequence, 16-head group) pairs (ws_plan.h seq_of).
  int B, ng, R, heads, Dv, cap, grid;
  int add;  // lengths are gpu_len[b] + add (1 when gpu_len is a fused step's len_in)
  const float* out_g;
  const float* lse_g;
  const uint16_t* part_out;  // bf16 pieces
  const float* part_lse;
  const void* b_out;
  const void* b_aux0;
  const void* b_aux1;
  uint16_t* out_bf16;
  float* out_f32;
  float* lse_out;
};

// One 64-lane workgroup per (output row, 256-column chunk): lane t owns float4
// column chunk * 64 + t and accumulates it over the pieces with eight loads
// in flight.
constexpr int kMergeChunk4 = 64;

template <int FMT>
__global__ __launch_bounds__(64) void merge_split_kernel(const MergeSplitParams p) {
  __shared__ int s_pref[kMaxSeqs + 1];
  __shared__ int s_wpref[kSeqPlanMax + 1];
  __shared__ int s_scan[2];
  __shared__ float s_w[kReduceMaxWeights];
  const int qrow = blockIdx.x;
  const int t = threadIdx.x;
  const int krow = qrow / p.heads;
  const int h = qrow - krow * p.heads;
  const int b = krow / p.R;
  const int r = krow - b * p.R;
  // The host partial's address depends on nothing the plan computes: its
  // loads go out first.
  const int c = blockIdx.y * kMergeChunk4 + t;  // float4 column
  const bool col_ok = c < (p.Dv >> 2);
  float lb = neg_inf();
  float4 ob = make_float4(0.f, 0.f, 0.f, 0.f);
  if (FMT >= 0)
    load_b<(FMT >= 0 ? FMT : 0)>(p.b_out, p.b_aux0, p.b_aux1, qrow, p.Dv, col_ok ? c : 0, lb,
                                 ob);
  const Plan plan = plan_build<64>(p.gpu_len, p.add, p.cap, p.B, p.R, p.grid, s_pref, s_scan,
                                   nullptr, s_wpref, -1, p.ng);
  const int nbb = (plan_len(p.gpu_len, seq_of(b, p.ng), p.add, p.cap) + 31) >> 5;
  // One piece: the step's final partial (out_g, fp32); several: their bf16
  // workspace slots, piece s at pieces + s * sstride.
  int n = 1;
  const float* src = p.out_g + (size_t)qrow * p.Dv;
  const uint16_t* pieces = nullptr;
  const float* lsrc = p.lse_g + qrow;  // lse of piece s at lsrc[s * lstride]
  size_t sstride = 0, lstride = 0;
  if (nbb > 0 && plan.n > 0) {
    const int row_start = s_pref[b] + r * nbb;
    int w_first, nseg;
    plan_row_splits(plan, b, row_start, nbb, s_wpref, w_first, nseg);
    if (nseg > 1) {
      n = nseg;
      const size_t slot0 = (size_t)(w_first + krow) * p.heads + h;
      pieces = p.part_out + slot0 * p.Dv;
      lsrc = p.part_lse + slot0;
      sstride = (size_t)p.heads * p.Dv;
      lstride = p.heads;
    }
  }
  // The pieces' columns are requested with their lse values.
  const int cc = col_ok ? c : 0;
  uint2 pv[8];
  float4 v1 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (!pieces)
    v1 = ((const float4*)src)[cc];
  else if (n <= 8)
    preload_pieces(pieces + 4 * cc, sstride, n, pv);
  // weights: M over the GPU pieces and the host partial
  float mx = lb;
  for (int s = t; s < n; s += 64) {
    const float v = lsrc[(size_t)s * lstride];
    s_w[s] = v;
    mx = max_nan(mx, v);
  }
  for (int o = 1; o < 64; o <<= 1) mx = max_nan(mx, __shfl_xor(mx, o));
  float sum = 0.f;
  for (int s = t; s < n; s += 64) {
    const float w = mx == neg_inf() ? 0.f : __expf(s_w[s] - mx);
    s_w[s] = w;
    sum += w;
  }
  for (int o = 1; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
  const float wb = (FMT >= 0 && mx != neg_inf()) ? __expf(lb - mx) : 0.f;
  const float L = sum + wb;
  __syncthreads();
  const float inv = L == 0.f ? 0.f : 1.f / L;
  if (blockIdx.y == 0 && t == 0 && p.lse_out)
    p.lse_out[qrow] = L == 0.f ? neg_inf() : mx + __logf(L);
  if (!col_ok) return;
  // an empty host side has weight 0 and must not turn its output into NaN
  float4 a = wb > 0.f ? make_float4(wb * ob.x, wb * ob.y, wb * ob.z, wb * ob.w)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
  if (pieces) {
    if (n <= 8)
      accum_preloaded(pv, n, s_w, a);
    else
      accum_pieces(pieces + 4 * c, sstride, n, s_w, a);
  } else {
    const float w = s_w[0];
    a.x += w * v1.x; a.y += w * v1.y; a.z += w * v1.z; a.w += w * v1.w;
  }
  const float4 o = make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
  if (p.out_f32) ((float4*)(p.out_f32 + (size_t)qrow * p.Dv))[c] = o;
  if (p.out_bf16) {
    uint2 packed;
    packed.x = pack_bf16x2(o.x, o.y);
    packed.y = pack_bf16x2(o.z, o.w);
    ((uint2*)(p.out_bf16 + (size_t)qrow * p.Dv))[c] = packed;
  }
}

// ---------------------------------------------------------------------------
// Split combine + host merge + the W_UV epilogue of absorbed MLA
// (system/deepseek.py:397-407): the merged latent row of (sequence b, head h)
// is normalised, rounded to bf16 as the reference rounds it before its bmm,
// and projected onto W_UV[h] ([Dout][512] bf16), giving out_v[b][h * Dout + v].
//
// One 256-thread workgroup per (b, h) row: threads 0..127 merge one float4
// column each (the same pieces, weights and accumulation order as
// merge_split_kernel, so the optional latent output is bit-identical to it)
// into an LDS row; then eight lanes per W_UV row read it 128 contiguous bytes
// at a time and reduce by shuffles, 32 rows per pass.  W_UV[h] is shared by
// the B rows of head h through L2.
constexpr int kUvThreads = 256;
constexpr int kUvGroup = 2;  // passes of 32 W_UV rows whose loads are in flight together

template <int FMT>
__global__ __launch_bounds__(kUvThreads) void merge_split_uv_kernel(
    const MergeSplitParams p, const uint16_t* __restrict__ w_uv, int Dout,
    uint16_t* __restrict__ out_v) {
  __shared__ int s_pref[kMaxSeqs + 1];
  __shared__ int s_wpref[kSeqPlanMax + 1];
  __shared__ int s_scan[kUvThreads / 64 + 1];
  __shared__ float s_w[kReduceMaxWeights];
  __shared__ float s_row[512];
  __shared__ float s_ml[2];  // M, 1 / L
  const int qrow = blockIdx.x;  // b * heads + h
  const int t = threadIdx.x;
  const int b = qrow / p.heads;
  const int h = qrow - b * p.heads;
  const int hp = p.heads / p.ng;  // heads of a piece: 16, or 128 (wide layout)
  const int pv_seq = qrow / hp;   // plan sequence (b, head group) and head in it
  const int h16 = qrow - pv_seq * hp;
  // The W_UV rows of the first kUvGroup passes do not depend on the merge:
  // their loads go out first and land while the plan and the merge run.
  const int lane8 = t & 7;
  const int rsub = t >> 3;  // 32 rows per pass
  u32x4 wv[kUvGroup][8];
#pragma unroll
  for (int g = 0; g < kUvGroup; ++g) {
    const int v = min(g * (kUvThreads / 8) + rsub, Dout - 1);
    const u32x4* wrow = (const u32x4*)(w_uv + ((size_t)h * Dout + v) * 512);
#pragma unroll
    for (int j = 0; j < 8; ++j) wv[g][j] = wrow[j * 8 + lane8];
  }
  // So do the host partial's.
  const int c = t;  // float4 column (threads < 128)
  const bool merging = c < (p.Dv >> 2);
  float lb = neg_inf();
  float4 ob = make_float4(0.f, 0.f, 0.f, 0.f);
  if (FMT >= 0 && merging)
    load_b<(FMT >= 0 ? FMT : 0)>(p.b_out, p.b_aux0, p.b_aux1, qrow, p.Dv, c, lb, ob);
  const Plan plan =
      plan_build<kUvThreads>(p.gpu_len, p.add, p.cap, p.B, 1, p.grid, s_pref, s_scan, nullptr,
                             s_wpref, -1, p.ng);
  const int nbb = (plan_len(p.gpu_len, b, p.add, p.cap) + 31) >> 5;
  int n = 1;
  const float* src = p.out_g + (size_t)qrow * p.Dv;
  const uint16_t* pieces = nullptr;
  const float* lsrc = p.lse_g + qrow;
  size_t sstride = 0, lstride = 0;
  if (nbb > 0 && plan.n > 0) {
    const int row_start = s_pref[pv_seq];
    int w_first, nseg;
    plan_row_splits(plan, pv_seq, row_start, nbb, s_wpref, w_first, nseg);
    if (nseg > 1) {  // pieces hold hp heads each
      n = nseg;
      const size_t slot0 = (size_t)(w_first + pv_seq) * hp + h16;
      pieces = p.part_out + slot0 * p.Dv;
      lsrc = p.part_lse + slot0;
      sstride = (size_t)hp * p.Dv;
      lstride = hp;
    }
  }
  // The merging threads' piece columns are requested with the lse values.
  uint2 pv[8];
  float4 v1 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (merging) {
    if (!pieces)
      v1 = ((const float4*)src)[c];
    else if (n <= 8)
      preload_pieces(pieces + 4 * c, sstride, n, pv);
  }
  if (t < 64) {  // wave 0: the pieces' weights
    float mx = lb;
    for (int s = t; s < n; s += 64) {
      const float v = lsrc[(size_t)s * lstride];
      s_w[s] = v;
      mx = max_nan(mx, v);
    }
    for (int o = 1; o < 64; o <<= 1) mx = max_nan(mx, __shfl_xor(mx, o));
    float sum = 0.f;
    for (int s = t; s < n; s += 64) {
      const float w = mx == neg_inf() ? 0.f : __expf(s_w[s] - mx);
      s_w[s] = w;
      sum += w;
    }
    for (int o = 1; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
    const float wb = (FMT >= 0 && mx != neg_inf()) ? __expf(lb - mx) : 0.f;
    const float L = sum + wb;
    if (t == 0) {
      s_ml[0] = mx;
      s_ml[1] = L == 0.f ? 0.f : 1.f / L;
      if (p.lse_out) p.lse_out[qrow] = L == 0.f ? neg_inf() : mx + __logf(L);
    }
  }
  __syncthreads();
  if (merging) {
    const float mx = s_ml[0];
    const float inv = s_ml[1];
    const float wb = (FMT >= 0 && mx != neg_inf()) ? __expf(lb - mx) : 0.f;
    float4 a = wb > 0.f ? make_float4(wb * ob.x, wb * ob.y, wb * ob.z, wb * ob.w)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
    if (pieces) {
      if (n <= 8)
        accum_preloaded(pv, n, s_w, a);
      else
        accum_pieces(pieces + 4 * c, sstride, n, s_w, a);
    } else {
      const float w = s_w[0];
      a.x += w * v1.x; a.y += w * v1.y; a.z += w * v1.z; a.w += w * v1.w;
    }
    const float4 o = make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
    uint2 packed;
    packed.x = pack_bf16x2(o.x, o.y);
    packed.y = pack_bf16x2(o.z, o.w);
    if (p.out_bf16) ((uint2*)(p.out_bf16 + (size_t)qrow * p.Dv))[c] = packed;
    s_row[4 * c + 0] = bf16_to_f32(packed.x & 0xffffu);
    s_row[4 * c + 1] = bf16_to_f32(packed.x >> 16);
    s_row[4 * c + 2] = bf16_to_f32(packed.y & 0xffffu);
    s_row[4 * c + 3] = bf16_to_f32(packed.y >> 16);
  }
  __syncthreads();
  // out_v[b][h * Dout + v] = sum_k s_row[k] * W_UV[h][v][k]: eight lanes per
  // W_UV row, 32 rows per pass, kUvGroup passes per group of loads
  for (int v0 = 0; v0 < Dout; v0 += kUvGroup * (kUvThreads / 8)) {
    if (v0 > 0) {  // groups after the first load here
#pragma unroll
      for (int g = 0; g < kUvGroup; ++g) {
        const int v = min(v0 + g * (kUvThreads / 8) + rsub, Dout - 1);
        const u32x4* wrow = (const u32x4*)(w_uv + ((size_t)h * Dout + v) * 512);
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[g][j] = wrow[j * 8 + lane8];
      }
    }
#pragma unroll
    for (int g = 0; g < kUvGroup; ++g) {
      const int v = v0 + g * (kUvThreads / 8) + rsub;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4 w = wv[g][j];
        const float* r = s_row + 8 * (j * 8 + lane8);
        acc += bf16_to_f32(w.x & 0xffffu) * r[0] + bf16_to_f32(w.x >> 16) * r[1];
        acc += bf16_to_f32(w.y & 0xffffu) * r[2] + bf16_to_f32(w.y >> 16) * r[3];
        acc += bf16_to_f32(w.z & 0xffffu) * r[4] + bf16_to_f32(w.z >> 16) * r[5];
        acc += bf16_to_f32(w.w & 0xffffu) * r[6] + bf16_to_f32(w.w >> 16) * r[7];
      }
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      if (lane8 == 0 && v < Dout)
        out_v[(size_t)b * p.heads * Dout + (size_t)h * Dout + v] = f32_to_bf16(acc);
    }
  }
}


// Split combine without a host partial (the one-launch GQA entry points):
// one 64-lane workgroup per output row, Dv <= 256 so a row is one column
// chunk and out/lse may alias out_g/lse_g; out_bf16 (optional) receives the
// same output rounded to bf16.
int merge_split_pieces(const int32_t* len, int len_add, int B, int R, int heads, int Dv,
                       int cap, int n, const float* out_g, const float* lse_g,
                       const SplitWorkspace& w, float* out, float* lse, uint16_t* out_bf16,
                       hipStream_t stream) {
  if (Dv > 4 * kMergeChunk4)
    return set_error(WS_EINVAL, "merge_split_pieces: Dv %d > %d", Dv, 4 * kMergeChunk4);
  MergeSplitParams prm;
  prm.gpu_len = len;
  prm.B = B;
  prm.ng = 1;
  prm.R = R;
  prm.heads = heads;
  prm.Dv = Dv;
  prm.cap = cap;
  prm.grid = n;
  prm.add = len_add;
  prm.out_g = out_g;
  prm.lse_g = lse_g;
  prm.part_out = w.part_out;
  prm.part_lse = w.part_lse;
  prm.b_out = nullptr;
  prm.b_aux0 = nullptr;
  prm.b_aux1 = nullptr;
  prm.out_bf16 = out_bf16;
  prm.out_f32 = out;
  prm.lse_out = lse;
  hipLaunchKernelGGL(merge_split_kernel<-1>, dim3((unsigned)(B * R * heads)), dim3(64), 0,
                     stream, prm);
  return WS_OK;
}

// The host-partial formats: whether a format is known, and whether it needs
// b_aux1 (the triples' sum).
static bool fmt_known(int f) {
  return f == WS_PARTIAL_LSE_F32 || f == WS_TRIPLE_UNNORM_F32 || f == WS_TRIPLE_NORM_BF16 ||
         f == WS_TRIPLE_NORM_F32 || f == WS_PARTIAL_LSE_BF16;
}
static bool fmt_has_sum(int f) { return f != WS_PARTIAL_LSE_F32 && f != WS_PARTIAL_LSE_BF16; }

}  // namespace ws

using namespace ws;

extern "C" int ws_merge_split(const int32_t* gpu_len, int B, int rows_per_seq, int heads,
                              int Dv, int page_capacity, int n_workgroups,
                              const float* out_g, const float* lse_g,
                              const void* workspace, size_t workspace_bytes,
                              const void* b_out, const void* b_aux0, const void* b_aux1,
                              int fmt_b, uint16_t* out_bf16, float* out_f32,
                              float* lse_out, void* stream) {
  if (!gpu_len || !out_g || !lse_g || !workspace)
    return set_error(WS_EINVAL, "ws_merge_split: null input pointer");
  if (!out_bf16 && !out_f32)
    return set_error(WS_EINVAL, "ws_merge_split: no output");
  // an absorbed-MLA step with H = 16 ng heads planned (sequence, head group)
  // pairs, unless its layout is wide (ws_reduce.h mla_layout)
  const bool mla = Dv == 512 && rows_per_seq == 1 && heads > 16 && heads % 16 == 0;
  const int ng = mla ? mla_layout(B, heads).ng : 1;
  if (B < 0 || (long long)B * ng > kMaxSeqs || rows_per_seq <= 0 || heads <= 0 ||
      (heads > 16 && !mla) || Dv <= 0 || Dv % 4 || Dv > 512 || page_capacity <= 0 ||
      n_workgroups <= 0)
    return set_error(WS_EINVAL, "ws_merge_split: bad sizes");
  const int Bp = B * ng;      // plan sequences
  heads /= ng;                // heads per plan row
  if (b_out && (!b_aux0 || (fmt_has_sum(fmt_b) && !b_aux1)))
    return set_error(WS_EINVAL, "ws_merge_split: host partial without its lse / max / sum");
  if (b_out && !fmt_known(fmt_b))
    return set_error(WS_EINVAL, "ws_merge_split: unknown format %d", fmt_b);
  if (n_workgroups > kReduceMaxWeights)
    return set_error(WS_EINVAL, "ws_merge_split: %d workgroups exceed %d", n_workgroups,
                     kReduceMaxWeights);
  if (((uintptr_t)workspace & 255u) || ((uintptr_t)out_g | (uintptr_t)out_f32 |
                                         (uintptr_t)b_out) & 15u || ((uintptr_t)out_bf16 & 7u))
    return set_error(WS_EINVAL, "ws_merge_split: misaligned buffer");
  const long long rows_kv = (long long)Bp * rows_per_seq;
  if (rows_kv > (1 << 24))
    return set_error(WS_EINVAL, "ws_merge_split: %lld rows exceed %d", rows_kv, 1 << 24);
  const size_t need = ws::workspace_bytes((int)rows_kv, heads, Dv, n_workgroups);
  if (workspace_bytes < need)
    return set_error(WS_EWORKSPACE, "ws_merge_split: workspace %zu < %zu bytes",
                     workspace_bytes, need);
  if (B == 0) return WS_OK;
  const SplitWorkspace w = carve_workspace((void*)workspace, (int)rows_kv, heads, n_workgroups);
  MergeSplitParams prm;
  prm.gpu_len = gpu_len;
  prm.B = Bp;
  prm.ng = ng;
  prm.R = rows_per_seq;
  prm.heads = heads;
  prm.Dv = Dv;
  prm.cap = page_capacity;
  prm.grid = n_workgroups;
  prm.add = 0;
  prm.out_g = out_g;
  prm.lse_g = lse_g;
  prm.part_out = w.part_out;
  prm.part_lse = w.part_lse;
  prm.b_out = b_out;
  prm.b_aux0 = b_aux0;
  prm.b_aux1 = b_aux1;
  prm.out_bf16 = out_bf16;
  prm.out_f32 = out_f32;
  prm.lse_out = lse_out;
  const dim3 grid((unsigned)(rows_kv * heads), (unsigned)((Dv / 4 + kMergeChunk4 - 1) / kMergeChunk4));
  const dim3 block(64);
  hipStream_t s = (hipStream_t)stream;
  if (!b_out) {
    hipLaunchKernelGGL(merge_split_kernel<-1>, grid, block, 0, s, prm);
  } else {
    switch (fmt_b) {
      case WS_PARTIAL_LSE_F32:
        hipLaunchKernelGGL(merge_split_kernel<WS_PARTIAL_LSE_F32>, grid, block, 0, s, prm);
        break;
      case WS_TRIPLE_UNNORM_F32:
        hipLaunchKernelGGL(merge_split_kernel<WS_TRIPLE_UNNORM_F32>, grid, block, 0, s, prm);
        break;
      case WS_TRIPLE_NORM_BF16:
        hipLaunchKernelGGL(merge_split_kernel<WS_TRIPLE_NORM_BF16>, grid, block, 0, s, prm);
        break;
      case WS_PARTIAL_LSE_BF16:
        hipLaunchKernelGGL(merge_split_kernel<WS_PARTIAL_LSE_BF16>, grid, block, 0, s, prm);
        break;
      default:
        hipLaunchKernelGGL(merge_split_kernel<WS_TRIPLE_NORM_F32>, grid, block, 0, s, prm);
        break;
    }
  }
  return check_launch("ws_merge_split");
}

extern "C" int ws_lse_merge(const float* out_g, const float* lse_g,
                            const void* b_out, const void* b_aux0,
                            const void* b_aux1, int fmt_b, uint16_t* out_bf16,
                            float* out_f32, float* lse_out, int rows, int Dv,
                            void* stream) {
  if (!out_g || !lse_g || !b_out || !b_aux0)
    return set_error(WS_EINVAL, "ws_lse_merge: null input pointer");
  if (!fmt_known(fmt_b))
    return set_error(WS_EINVAL, "ws_lse_merge: unknown format %d", fmt_b);
  if (fmt_has_sum(fmt_b) && !b_aux1)
    return set_error(WS_EINVAL, "ws_lse_merge: triple format needs b_aux1 (sum)");
  if (rows < 0 || Dv <= 0 || Dv % 4 || Dv > 512)
    return set_error(WS_EINVAL, "ws_lse_merge: bad sizes rows=%d Dv=%d", rows, Dv);
  if (((uintptr_t)out_g | (uintptr_t)b_out | (uintptr_t)out_f32) & 15u ||
      ((uintptr_t)out_bf16 & 7u))
    return set_error(WS_EINVAL, "ws_lse_merge: misaligned buffer");
  if (rows == 0) return WS_OK;
  const int threads = ((Dv / 4 + 63) / 64) * 64;
  hipStream_t s = (hipStream_t)stream;
  switch (fmt_b) {
#define WS_MERGE_CASE(F)                                                         \
  case F:                                                                        \
    hipLaunchKernelGGL(lse_merge_kernel<F>, dim3(rows), dim3(threads), 0, s,     \
                       out_g, lse_g, b_out, b_aux0, b_aux1, out_bf16, out_f32,   \
                       lse_out, Dv);                                             \
    break;
    WS_MERGE_CASE(WS_PARTIAL_LSE_F32)
    WS_MERGE_CASE(WS_TRIPLE_UNNORM_F32)
    WS_MERGE_CASE(WS_TRIPLE_NORM_BF16)
    WS_MERGE_CASE(WS_TRIPLE_NORM_F32)
    WS_MERGE_CASE(WS_PARTIAL_LSE_BF16)
#undef WS_MERGE_CASE
    default:
      return set_error(WS_EINVAL, "ws_lse_merge: unknown format %d", fmt_b);
  }
  return check_launch("ws_lse_merge");
}

extern "C" int ws_mla_merge_split_uv(const int32_t* gpu_len, int B, int heads,
                                     int page_capacity, int n_workgroups, const float* out_g,
                                     const float* lse_g, const void* workspace,
                                     size_t workspace_bytes, const void* b_out,
                                     const void* b_aux0, const void* b_aux1, int fmt_b,
                                     const uint16_t* w_uv, int Dout, uint16_t* out_latent,
                                     uint16_t* out_v, float* lse_out, void* stream) {
  constexpr int Dv = 512;
  if (!gpu_len || !out_g || !lse_g || !workspace || !w_uv || !out_v)
    return set_error(WS_EINVAL, "ws_mla_merge_split_uv: null pointer");
  if (B < 0 || heads < 16 || heads % 16 || (long long)B * (heads / 16) > kMaxSeqs ||
      page_capacity <= 0 || n_workgroups <= 0 || Dout <= 0 || Dout % 32 || Dout > 512)
    return set_error(WS_EINVAL, "ws_mla_merge_split_uv: bad sizes B=%d heads=%d Dout=%d", B,
                     heads, Dout);
  const MlaLayout lay = mla_layout(B, heads);
  const int ng = lay.ng;
  const int Bp = lay.plan_seqs;  // plan sequences (sequence, head group)
  if (b_out && (!b_aux0 || (fmt_has_sum(fmt_b) && !b_aux1)))
    return set_error(WS_EINVAL, "ws_mla_merge_split_uv: host partial without its lse / max / sum");
  if (b_out && !fmt_known(fmt_b))
    return set_error(WS_EINVAL, "ws_mla_merge_split_uv: unknown format %d", fmt_b);
  if (n_workgroups > kReduceMaxWeights)
    return set_error(WS_EINVAL, "ws_mla_merge_split_uv: %d workgroups exceed %d", n_workgroups,
                     kReduceMaxWeights);
  if (((uintptr_t)workspace & 255u) || ((uintptr_t)out_g | (uintptr_t)b_out |
                                         (uintptr_t)w_uv) & 15u ||
      ((uintptr_t)out_latent & 7u) || ((uintptr_t)out_v & 1u))
    return set_error(WS_EINVAL, "ws_mla_merge_split_uv: misaligned buffer");
  const size_t need = ws::workspace_bytes(Bp, lay.piece_heads, Dv, n_workgroups);
  if (workspace_bytes < need)
    return set_error(WS_EWORKSPACE, "ws_mla_merge_split_uv: workspace %zu < %zu bytes",
                     workspace_bytes, need);
  if (B == 0) return WS_OK;
  const SplitWorkspace w =
      carve_workspace((void*)workspace, Bp, lay.piece_heads, n_workgroups);
  MergeSplitParams prm;
  prm.gpu_len = gpu_len;
  prm.B = Bp;
  prm.ng = ng;
  prm.R = 1;
  prm.heads = heads;
  prm.Dv = Dv;
  prm.cap = page_capacity;
  prm.grid = n_workgroups;
  prm.add = 0;
  prm.out_g = out_g;
  prm.lse_g = lse_g;
  prm.part_out = w.part_out;
  prm.part_lse = w.part_lse;
  prm.b_out = b_out;
  prm.b_aux0 = b_aux0;
  prm.b_aux1 = b_aux1;
  prm.out_bf16 = out_latent;
  prm.out_f32 = nullptr;
  prm.lse_out = lse_out;
  const dim3 grid((unsigned)(B * heads));
  const dim3 block(kUvThreads);
  hipStream_t s = (hipStream_t)stream;
  if (!b_out) {
    hipLaunchKernelGGL(merge_split_uv_kernel<-1>, grid, block, 0, s, prm, w_uv, Dout, out_v);
  } else {
    switch (fmt_b) {
      case WS_PARTIAL_LSE_F32:
        hipLaunchKernelGGL(merge_split_uv_kernel<WS_PARTIAL_LSE_F32>, grid, block, 0, s, prm,
                           w_uv, Dout, out_v);
        break;
      case WS_TRIPLE_UNNORM_F32:
        hipLaunchKernelGGL(merge_split_uv_kernel<WS_TRIPLE_UNNORM_F32>, grid, block, 0, s, prm,
                           w_uv, Dout, out_v);
        break;
      case WS_TRIPLE_NORM_BF16:
        hipLaunchKernelGGL(merge_split_uv_kernel<WS_TRIPLE_NORM_BF16>, grid, block, 0, s, prm,
                           w_uv, Dout, out_v);
        break;
      case WS_PARTIAL_LSE_BF16:
        hipLaunchKernelGGL(merge_split_uv_kernel<WS_PARTIAL_LSE_BF16>, grid, block, 0, s, prm,
                           w_uv, Dout, out_v);
        break;
      default:
        hipLaunchKernelGGL(merge_split_uv_kernel<WS_TRIPLE_NORM_F32>, grid, block, 0, s, prm,
                           w_uv, Dout, out_v);
        break;
    }
  }
  return check_launch("ws_mla_merge_split_uv");
}
