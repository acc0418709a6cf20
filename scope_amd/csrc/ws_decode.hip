// Split-KV decode attention over the HBM partition (gfx950).
//
// Both kernels treat one query-head group that shares a K/V stream as the
// N side of a 16x16x32 bf16 MFMA:
//   QK:  S^T[token, head] = sum_d K[token, d] * Q[head, d]
//        A = 16 tokens x 32 d straight from the page (16-byte loads),
//        B = Q^T (held in registers for the whole split).
//   PV:  O^T[d, head]   += sum_t V[t, d] * P[head, t]
//        A = V^T: each lane loads one 16-byte vector (8 consecutive d) of 8
//        tokens and v_perm_b32 pairs two tokens per dword, so no LDS transpose
//        is needed; B = P^T comes from the QK accumulator registers as they
//        are: the MFMA output layout (lane = head column, 4 token rows) equals
//        the B-operand layout (lane = head column, 8 k-slots) once two
//        16-token tiles are placed side by side in the k dimension.
// Softmax is online in the log2 domain (scores pre-multiplied by
// scale*log2(e), v_exp_f32); the running max is shared by the four lanes of a
// head column with two xor-shuffles per 32-token block.  P is rounded to bf16
// for the PV MFMA (as the reference's GPU partial does,
// roofline/bench_resident_kv.py:156) while the softmax sum stays fp32.
//
// Work decomposition: grid (split, row).  A split is tokens_per_split
// consecutive tokens of one row (GQA row = (b, kv head), MLA row = b); rows
// whose length fits one split write the final (out, lse) directly, others
// write partials that split_reduce_kernel combines.
#include <math.h>

#include "ws_common.h"

namespace ws {

constexpr int kGqaD = 128;

__device__ __forceinline__ int clamp_page(int pid, int num_pages) {
  return pid < 0 ? 0 : (pid >= num_pages ? num_pages - 1 : pid);
}

// Token rows feeding k-slot i of lane group j when two 16-token QK tiles form
// the 32-token k dimension of the PV MFMA.
__device__ __forceinline__ int pv_token(int i, int j) {
  return 16 * (i >> 2) + 4 * j + (i & 3);
}

// Online-softmax update of one 32-token block.  s0/s1 are the QK accumulators
// of tokens [0,16) and [16,32) (lane holds tokens 4j+i of head n16); nt is the
// number of valid tokens.  Returns P^T packed as the PV B operand and alpha,
// the rescale factor of the previous accumulators.
__device__ __forceinline__ u32x4 softmax_block(const f32x4& s0, const f32x4& s1,
                                               int j, int nt, float scale_log2,
                                               float& m_run, float& l_run,
                                               float& alpha) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = (4 * j + i < nt) ? s0[i] * scale_log2 : neg_inf();
    x[4 + i] = (16 + 4 * j + i < nt) ? s1[i] * scale_log2 : neg_inf();
  }
  float bm = x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) bm = fmaxf(bm, x[i]);
  bm = wave_max_xor16_32(bm);
  const float m_new = fmaxf(m_run, bm);
  alpha = __builtin_amdgcn_exp2f(m_run - m_new);
  float p[8];
  float ps = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
    ps += p[i];
  }
  l_run = l_run * alpha + ps;
  m_run = m_new;
  u32x4 pb;
  pb[0] = pack_bf16x2(p[0], p[1]);
  pb[1] = pack_bf16x2(p[2], p[3]);
  pb[2] = pack_bf16x2(p[4], p[5]);
  pb[3] = pack_bf16x2(p[6], p[7]);
  return pb;
}

// PV update of 8 output tiles from the 8 V vectors vr[i] (token pv_token(i,j),
// columns col0 + 8*n16 .. +8).  Tile e covers columns col0 + 8*m + e.
__device__ __forceinline__ void pv_block(f32x4 (&acc)[8], const u32x4 (&vr)[8],
                                         const u32x4& pb, float alpha) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int w = e >> 1;
    u32x4 va;
    if (e & 1) {
      va[0] = pair_hi(vr[0][w], vr[1][w]);
      va[1] = pair_hi(vr[2][w], vr[3][w]);
      va[2] = pair_hi(vr[4][w], vr[5][w]);
      va[3] = pair_hi(vr[6][w], vr[7][w]);
    } else {
      va[0] = pair_lo(vr[0][w], vr[1][w]);
      va[1] = pair_lo(vr[2][w], vr[3][w]);
      va[2] = pair_lo(vr[4][w], vr[5][w]);
      va[3] = pair_lo(vr[6][w], vr[7][w]);
    }
    acc[e] = acc[e] * alpha;
    acc[e] = mfma16x16x32(va, pb, acc[e]);
  }
}

// Writes the 32 outputs a lane owns: head row `orow`, columns
// col0 + 32*j + 8*i + e (acc[e][i]), divided by l.
__device__ __forceinline__ void store_out(float* __restrict__ dst,
                                          const f32x4 (&acc)[8], int j,
                                          float inv_l) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float4 lo = make_float4(acc[0][i] * inv_l, acc[1][i] * inv_l,
                            acc[2][i] * inv_l, acc[3][i] * inv_l);
    float4 hi = make_float4(acc[4][i] * inv_l, acc[5][i] * inv_l,
                            acc[6][i] * inv_l, acc[7][i] * inv_l);
    float4* p = (float4*)(dst + 32 * j + 8 * i);
    p[0] = lo;
    p[1] = hi;
  }
}

__device__ __forceinline__ void store_empty(float* __restrict__ dst, int j) {
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 8; ++i) ((float4*)(dst + 32 * j))[i] = z;
}

// ---------------------------------------------------------------------------
// GQA: one wave per (split, b * Hkv + kvh).  G query heads share the K/V
// stream; heads are the MFMA N dimension (columns >= G are padding).
template <int G>
__global__ __launch_bounds__(64) void gqa_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pages,
    const uint16_t* __restrict__ v_pages, const int32_t* __restrict__ page_table,
    const int32_t* __restrict__ gpu_len, int Hkv, int page_size, int max_pages,
    int num_pages, int tokens_per_split, float scale_log2,
    float* __restrict__ part_out, float* __restrict__ part_lse,
    float* __restrict__ out, float* __restrict__ lse, int rows_q) {
  constexpr int D = kGqaD;
  const int split = blockIdx.x;
  const int row = blockIdx.y;
  const int b = row / Hkv;
  const int kvh = row - b * Hkv;
  const int lane = threadIdx.x;
  const int n16 = lane & 15;
  const int j = lane >> 4;
  const int qrow = b * (Hkv * G) + kvh * G + n16;
  const bool head_ok = n16 < G;

  // Never address past the grid's splits or the page table row, whatever
  // gpu_len holds.
  const int len = min(gpu_len[b], min((int)gridDim.x * tokens_per_split,
                                      page_size * max_pages));
  const int t_begin = split * tokens_per_split;
  if (len <= 0) {
    if (split == 0 && head_ok) {
      store_empty(out + (size_t)qrow * D, j);
      if (j == 0) lse[qrow] = neg_inf();
    }
    return;
  }
  if (t_begin >= len) return;
  const int t_end = min(len, t_begin + tokens_per_split);
  const int n_valid = (len + tokens_per_split - 1) / tokens_per_split;

  u32x4 qb[4];
  if (head_ok) {
    const u32x4* qp = (const u32x4*)(q + (size_t)qrow * D);
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = qp[4 * s + j];
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = u32x4{0u, 0u, 0u, 0u};
  }

  f32x4 acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = neg_inf();
  float l_run = 0.f;

  const int32_t* pt = page_table + (size_t)b * max_pages;
  for (int t0 = t_begin; t0 < t_end; t0 += 32) {
    const int page = t0 / page_size;
    const int off0 = t0 - page * page_size;
    const int pid = clamp_page(pt[page], num_pages);
    const size_t tok0 = ((size_t)pid * Hkv + kvh) * page_size + off0;
    const uint16_t* kb = k_pages + tok0 * D;
    const uint16_t* vb = v_pages + tok0 * D;
    const int nt = min(32, t_end - t0);

    u32x4 ka[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int r = min(16 * tt + n16, nt - 1);
      const u32x4* kr = (const u32x4*)(kb + (size_t)r * D);
#pragma unroll
      for (int s = 0; s < 4; ++s) ka[tt][s] = kr[4 * s + j];
    }
    u32x4 vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(pv_token(i, j), nt - 1);
      vr[i] = ((const u32x4*)(vb + (size_t)r * D))[n16];
    }

    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s0 = mfma16x16x32(ka[0][s], qb[s], s0);
      s1 = mfma16x16x32(ka[1][s], qb[s], s1);
    }
    float alpha;
    const u32x4 pb = softmax_block(s0, s1, j, nt, scale_log2, m_run, l_run, alpha);
    pv_block(acc, vr, pb, alpha);
  }

  const float l_tot = wave_sum_xor16_32(l_run);
  if (!head_ok) return;
  const float inv_l = 1.f / l_tot;
  const float lse_v = (m_run + __log2f(l_tot)) * kLn2;
  if (n_valid == 1) {
    store_out(out + (size_t)qrow * D, acc, j, inv_l);
    if (j == 0) lse[qrow] = lse_v;
  } else {
    const size_t prow = (size_t)split * rows_q + qrow;
    store_out(part_out + prow * D, acc, j, inv_l);
    if (j == 0) part_lse[prow] = lse_v;
  }
}

// ---------------------------------------------------------------------------
// MLA (absorbed): one 256-thread workgroup per (split, b).  16 heads share the
// 576-wide latent of each token.  Per 32-token block, wave w computes the QK
// partial of token tile (w & 1) over latent half (w >> 1) (9 MFMA k-steps);
// the four partial tiles meet in LDS, every wave runs the same softmax, and
// wave w accumulates output columns [128w, 128w + 128).
constexpr int kMlaH = 16;
constexpr int kMlaL = 576;
constexpr int kMlaC = 512;

__global__ __launch_bounds__(256) void mla_partial_kernel(
    const uint16_t* __restrict__ q_nope, const uint16_t* __restrict__ q_pe,
    const uint16_t* __restrict__ latent, const int32_t* __restrict__ page_table,
    const int32_t* __restrict__ gpu_len, int page_size, int max_pages,
    int num_pages, int tokens_per_split, float scale_log2,
    float* __restrict__ part_out, float* __restrict__ part_lse,
    float* __restrict__ out, float* __restrict__ lse, int rows) {
  __shared__ f32x4 sbuf[2][2][2][64];  // [buffer][latent half][token tile][lane]
  const int split = blockIdx.x;
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15;
  const int j = lane >> 4;
  const int tt = wave & 1;
  const int kh = wave >> 1;
  const int orow = b * kMlaH + n16;
  const int col0 = 128 * wave;

  // Never address past the grid's splits or the page table row, whatever
  // gpu_len holds.
  const int len = min(gpu_len[b], min((int)gridDim.x * tokens_per_split,
                                      page_size * max_pages));
  const int t_begin = split * tokens_per_split;
  if (len <= 0) {
    if (split == 0) {
      store_empty(out + (size_t)orow * kMlaC + col0, j);
      if (wave == 0 && j == 0) lse[orow] = neg_inf();
    }
    return;
  }
  if (t_begin >= len) return;
  const int t_end = min(len, t_begin + tokens_per_split);
  const int n_valid = (len + tokens_per_split - 1) / tokens_per_split;

  // Q^T for this wave's 9 k-steps: k = 32*(9*kh + u) + 8*j .. +8.
  u32x4 qb[9];
#pragma unroll
  for (int u = 0; u < 9; ++u) {
    const int k0 = 32 * (9 * kh + u) + 8 * j;
    if (k0 < kMlaC)
      qb[u] = ((const u32x4*)(q_nope + (size_t)orow * kMlaC))[k0 >> 3];
    else
      qb[u] = ((const u32x4*)(q_pe + (size_t)orow * 64))[(k0 - kMlaC) >> 3];
  }

  f32x4 acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = neg_inf();
  float l_run = 0.f;

  const int32_t* pt = page_table + (size_t)b * max_pages;
  int buf = 0;
  for (int t0 = t_begin; t0 < t_end; t0 += 32, buf ^= 1) {
    const int page = t0 / page_size;
    const int off0 = t0 - page * page_size;
    const int pid = clamp_page(pt[page], num_pages);
    const uint16_t* lb =
        latent + ((size_t)pid * page_size + off0) * (size_t)kMlaL;
    const int nt = min(32, t_end - t0);

    u32x4 ka[9];
    {
      const int r = min(16 * tt + n16, nt - 1);
      const u32x4* kr = (const u32x4*)(lb + (size_t)r * kMlaL);
#pragma unroll
      for (int u = 0; u < 9; ++u) ka[u] = kr[4 * (9 * kh + u) + j];
    }
    u32x4 vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(pv_token(i, j), nt - 1);
      vr[i] = ((const u32x4*)(lb + (size_t)r * kMlaL))[(col0 >> 3) + n16];
    }

    f32x4 sp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 9; ++u) sp = mfma16x16x32(ka[u], qb[u], sp);
    sbuf[buf][kh][tt][lane] = sp;
    __syncthreads();
    const f32x4 s0 = sbuf[buf][0][0][lane] + sbuf[buf][1][0][lane];
    const f32x4 s1 = sbuf[buf][0][1][lane] + sbuf[buf][1][1][lane];

    float alpha;
    const u32x4 pb = softmax_block(s0, s1, j, nt, scale_log2, m_run, l_run, alpha);
    pv_block(acc, vr, pb, alpha);
  }

  const float l_tot = wave_sum_xor16_32(l_run);
  const float inv_l = 1.f / l_tot;
  const float lse_v = (m_run + __log2f(l_tot)) * kLn2;
  if (n_valid == 1) {
    store_out(out + (size_t)orow * kMlaC + col0, acc, j, inv_l);
    if (wave == 0 && j == 0) lse[orow] = lse_v;
  } else {
    const size_t prow = (size_t)split * rows + orow;
    store_out(part_out + prow * kMlaC + col0, acc, j, inv_l);
    if (wave == 0 && j == 0) part_lse[prow] = lse_v;
  }
}

// ---------------------------------------------------------------------------
// LSE combine of the valid splits of each row; Dv / 4 threads, float4 each.
__global__ __launch_bounds__(128) void split_reduce_kernel(
    const float* __restrict__ part_out, const float* __restrict__ part_lse,
    const int32_t* __restrict__ gpu_len, int rows, int heads_per_len, int Dv,
    int n_splits, int tokens_per_split, float* __restrict__ out,
    float* __restrict__ lse) {
  const int row = blockIdx.x;
  const int len = gpu_len[row / heads_per_len];
  int n_valid = len > 0 ? (len + tokens_per_split - 1) / tokens_per_split : 0;
  if (n_valid == 1) return;
  const int c = threadIdx.x;  // float4 column
  float4* o = (float4*)(out + (size_t)row * Dv) + c;
  if (n_valid == 0) {
    if (c < Dv / 4) *o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c == 0) lse[row] = neg_inf();
    return;
  }
  if (n_valid > n_splits) n_valid = n_splits;
  float M = neg_inf();
  for (int s = 0; s < n_valid; ++s) M = fmaxf(M, part_lse[(size_t)s * rows + row]);
  float wsum = 0.f;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s = 0; s < n_valid; ++s) {
    const size_t pr = (size_t)s * rows + row;
    const float w = __expf(part_lse[pr] - M);
    wsum += w;
    if (c < Dv / 4) {
      const float4 v = ((const float4*)(part_out + pr * Dv))[c];
      a.x += w * v.x;
      a.y += w * v.y;
      a.z += w * v.z;
      a.w += w * v.w;
    }
  }
  const float inv = 1.f / wsum;
  if (c < Dv / 4) *o = make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
  if (c == 0) lse[row] = M + __logf(wsum);
}

static int launch_split_reduce(const float* part_out, const float* part_lse,
                               const int32_t* gpu_len, int rows,
                               int heads_per_len, int Dv, int n_splits,
                               int tps, float* out, float* lse,
                               hipStream_t stream) {
  const int threads = ((Dv / 4 + 63) / 64) * 64;
  hipLaunchKernelGGL(split_reduce_kernel, dim3(rows), dim3(threads), 0, stream,
                     part_out, part_lse, gpu_len, rows, heads_per_len, Dv,
                     n_splits, tps, out, lse);
  return check_launch("split_reduce");
}

// Tokens per split: enough splits to put `target` waves in flight, in
// multiples of 32 tokens, between 64 and 8192.
static int choose_split(int max_len, int rows, int target) {
  long long want = ((long long)max_len * rows + target - 1) / target;
  if (want < 64) want = 64;
  if (want > 8192) want = 8192;
  return (int)((want + 31) / 32 * 32);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Waves (GQA) or 4-wave workgroups (MLA) the automatic split aims to launch.
constexpr int kGqaTargetWaves = 4096;
constexpr int kMlaTargetGroups = 1024;

}  // namespace ws

using namespace ws;

extern "C" int ws_decode_plan(int kind, int rows_kv, int max_len,
                              int tokens_per_split, int* tps_out,
                              int* n_splits_out) {
  if ((kind != 0 && kind != 1) || rows_kv < 0 || max_len < 0 ||
      tokens_per_split < 0 || tokens_per_split % 32)
    return set_error(WS_EINVAL, "ws_decode_plan: bad arguments");
  const int tps = tokens_per_split
                      ? tokens_per_split
                      : choose_split(max_len, rows_kv > 0 ? rows_kv : 1,
                                     kind == 0 ? kGqaTargetWaves : kMlaTargetGroups);
  if (tps_out) *tps_out = tps;
  if (n_splits_out) *n_splits_out = max_len > 0 ? (max_len + tps - 1) / tps : 1;
  return WS_OK;
}

extern "C" int ws_split_reduce(const float* part_out, const float* part_lse,
                               const int32_t* gpu_len, int rows,
                               int heads_per_len, int Dv, int n_splits,
                               int tokens_per_split, float* out, float* lse,
                               void* stream) {
  if (!part_out || !part_lse || !gpu_len || !out || !lse)
    return set_error(WS_EINVAL, "ws_split_reduce: null pointer");
  if (rows < 0 || heads_per_len <= 0 || Dv <= 0 || Dv % 4 || Dv > 512 ||
      n_splits <= 0 || tokens_per_split <= 0)
    return set_error(WS_EINVAL, "ws_split_reduce: bad sizes");
  if (rows == 0) return WS_OK;
  return launch_split_reduce(part_out, part_lse, gpu_len, rows, heads_per_len,
                             Dv, n_splits, tokens_per_split, out, lse,
                             (hipStream_t)stream);
}

extern "C" int ws_gqa_decode_partial(
    const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
    const int32_t* page_table, const int32_t* gpu_len, int B, int Hq, int Hkv,
    int D, int page_size, int max_pages, int num_pages, int max_len,
    int tokens_per_split, float scale, float* out, float* lse,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k_pages || !v_pages || !page_table || !gpu_len || !out || !lse)
    return set_error(WS_EINVAL, "ws_gqa_decode_partial: null pointer");
  if (B < 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv)
    return set_error(WS_EINVAL, "ws_gqa_decode_partial: bad heads Hq=%d Hkv=%d", Hq, Hkv);
  const int G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16)
    return set_error(WS_EINVAL,
                     "ws_gqa_decode_partial: group size %d unsupported (1,2,4,8,16)", G);
  if (D != kGqaD)
    return set_error(WS_EINVAL, "ws_gqa_decode_partial: head_dim %d unsupported (128)", D);
  if (page_size <= 0 || max_pages <= 0 || num_pages <= 0 || max_len < 0 ||
      (page_size % 32 && max_pages != 1) ||
      (long long)max_len > (long long)page_size * max_pages)
    return set_error(WS_EINVAL,
                     "ws_gqa_decode_partial: bad paging page_size=%d max_pages=%d "
                     "num_pages=%d max_len=%d (page_size must be a multiple of 32 "
                     "unless max_pages == 1)",
                     page_size, max_pages, num_pages, max_len);
  if (tokens_per_split < 0 || tokens_per_split % 32)
    return set_error(WS_EINVAL,
                     "ws_gqa_decode_partial: tokens_per_split %d not a multiple of 32",
                     tokens_per_split);
  if (!aligned16(q) || !aligned16(k_pages) || !aligned16(v_pages) ||
      !aligned16(out))
    return set_error(WS_EINVAL, "ws_gqa_decode_partial: buffers must be 16-byte aligned");
  if (B == 0) return WS_OK;
  const int rows_kv = B * Hkv;
  const int rows_q = B * Hq;
  int tps = 0, n_splits = 0;
  ws_decode_plan(0, rows_kv, max_len, tokens_per_split, &tps, &n_splits);
  float* part_out = nullptr;
  float* part_lse = nullptr;
  if (n_splits > 1) {
    const size_t need = ws_decode_workspace_bytes(rows_q, D, n_splits);
    if (!workspace || workspace_bytes < need)
      return set_error(WS_EWORKSPACE,
                       "ws_gqa_decode_partial: workspace %zu < %zu bytes",
                       workspace_bytes, need);
    part_out = (float*)workspace;
    part_lse = part_out + (size_t)n_splits * rows_q * D;
  }
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(n_splits, rows_kv);
#define WS_GQA_LAUNCH(GG)                                                        \
  hipLaunchKernelGGL(gqa_partial_kernel<GG>, grid, dim3(64), 0, s, q, k_pages,   \
                     v_pages, page_table, gpu_len, Hkv, page_size, max_pages,    \
                     num_pages, tps, scale_log2, part_out, part_lse, out, lse,   \
                     rows_q)
  switch (G) {
    case 1: WS_GQA_LAUNCH(1); break;
    case 2: WS_GQA_LAUNCH(2); break;
    case 4: WS_GQA_LAUNCH(4); break;
    case 8: WS_GQA_LAUNCH(8); break;
    case 16: WS_GQA_LAUNCH(16); break;
    default:
      return set_error(WS_EINVAL,
                       "ws_gqa_decode_partial: group size %d unsupported (1,2,4,8,16)", G);
  }
#undef WS_GQA_LAUNCH
  int rc = check_launch("ws_gqa_decode_partial");
  if (rc) return rc;
  if (n_splits > 1)
    return launch_split_reduce(part_out, part_lse, gpu_len, rows_q, Hq, D,
                               n_splits, tps, out, lse, s);
  return WS_OK;
}

extern "C" int ws_mla_decode_partial(
    const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* latent_pages,
    const int32_t* page_table, const int32_t* gpu_len, int B, int H,
    int page_size, int max_pages, int num_pages, int max_len,
    int tokens_per_split, float scale, float* out, float* lse,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (!q_nope || !q_pe || !latent_pages || !page_table || !gpu_len || !out || !lse)
    return set_error(WS_EINVAL, "ws_mla_decode_partial: null pointer");
  if (B < 0 || H != kMlaH)
    return set_error(WS_EINVAL, "ws_mla_decode_partial: H=%d unsupported (16)", H);
  if (page_size <= 0 || max_pages <= 0 || num_pages <= 0 || max_len < 0 ||
      (page_size % 32 && max_pages != 1) ||
      (long long)max_len > (long long)page_size * max_pages)
    return set_error(WS_EINVAL,
                     "ws_mla_decode_partial: bad paging page_size=%d max_pages=%d "
                     "num_pages=%d max_len=%d",
                     page_size, max_pages, num_pages, max_len);
  if (tokens_per_split < 0 || tokens_per_split % 32)
    return set_error(WS_EINVAL,
                     "ws_mla_decode_partial: tokens_per_split %d not a multiple of 32",
                     tokens_per_split);
  if (!aligned16(q_nope) || !aligned16(q_pe) || !aligned16(latent_pages) ||
      !aligned16(out))
    return set_error(WS_EINVAL, "ws_mla_decode_partial: buffers must be 16-byte aligned");
  if (B == 0) return WS_OK;
  const int rows = B * H;
  int tps = 0, n_splits = 0;
  ws_decode_plan(1, B, max_len, tokens_per_split, &tps, &n_splits);
  float* part_out = nullptr;
  float* part_lse = nullptr;
  if (n_splits > 1) {
    const size_t need = ws_decode_workspace_bytes(rows, kMlaC, n_splits);
    if (!workspace || workspace_bytes < need)
      return set_error(WS_EWORKSPACE,
                       "ws_mla_decode_partial: workspace %zu < %zu bytes",
                       workspace_bytes, need);
    part_out = (float*)workspace;
    part_lse = part_out + (size_t)n_splits * rows * kMlaC;
  }
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(mla_partial_kernel, dim3(n_splits, B), dim3(256), 0, s,
                     q_nope, q_pe, latent_pages, page_table, gpu_len, page_size,
                     max_pages, num_pages, tps, scale * kLog2e, part_out,
                     part_lse, out, lse, rows);
  int rc = check_launch("ws_mla_decode_partial");
  if (rc) return rc;
  if (n_splits > 1)
    return launch_split_reduce(part_out, part_lse, gpu_len, rows, H, kMlaC,
                               n_splits, tps, out, lse, s);
  return WS_OK;
}
