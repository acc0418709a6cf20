// MFMA building blocks of the split-KV decode kernels (gfx950).
//
// A query-head group that shares one K/V stream is the N side of a
// 16x16x32 bf16 MFMA (heads beyond the group are zero padding):
//   QK:  S^T[token, head] = sum_d K[token, d] * Q[head, d]
//        A = 16 tokens x 32 d loaded straight from the page (16-byte loads),
//        B = Q^T, held in registers for the whole call.
//   PV:  O^T[d, head] += sum_t V[t, d] * P[head, t]
//        A = V^T: each lane loads one 16-byte vector (8 consecutive d) of 8
//        tokens and v_perm_b32 pairs two tokens per dword, so no LDS transpose
//        is needed; B = P^T comes from the QK accumulators as they are: the
//        MFMA output layout (lane = head column, 4 token rows) equals the B
//        operand layout (lane = head column, 8 k-slots) once two 16-token
//        tiles are placed side by side in k.
// Softmax is online in the log2 domain (scores pre-multiplied by
// scale * log2(e)); the block max is shared by the four lanes of a head
// column with two lane exchanges per 32-token block, and the accumulators are
// rescaled lazily (kLazyRescaleLog2).  P is rounded to bf16 for
// the PV MFMA (as the reference's GPU partial rounds its probabilities,
// roofline/bench_resident_kv.py:156) while the softmax sum stays fp32.
#pragma once

#include "ws_common.h"

namespace ws {

__device__ __forceinline__ int clamp_page(int pid, int num_pages) {
  return pid < 0 ? 0 : (pid >= num_pages ? num_pages - 1 : pid);
}

// Token of the 32-token block feeding k-slot i of lane group j when two
// 16-token QK tiles form the k dimension of the PV MFMA.
__device__ __forceinline__ int pv_token(int i, int j) {
  return 16 * (i >> 2) + 4 * j + (i & 3);
}

// Lazy rescaling: the accumulators stay relative to a reference max m_run
// that moves only when some head's block max exceeds it by more than this
// (log2 domain), so most blocks skip the rescale of the accumulators.  The
// probabilities then stay below 2^8: exact enough in bf16 (a relative
// format) and far from any fp32 limit.
constexpr float kLazyRescaleLog2 = 8.f;

// Online-softmax update of one 32-token block.  s0/s1 are the QK accumulators
// of tokens [0,16) and [16,32) (lane holds tokens 4j+i of head n16); nt is the
// number of valid tokens.  Returns P^T packed as the PV B operand; `rescale`
// (the same in every lane) says whether the reference max moved, in which
// case alpha is the factor for the previous accumulators.  Every lane of the
// wave must be active.
__device__ __forceinline__ u32x4 softmax_block(const f32x4& s0, const f32x4& s1,
                                               int j, int nt, float scale_log2,
                                               float& m_run, float& l_run,
                                               float& alpha, bool& rescale) {
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
  rescale = __builtin_amdgcn_ballot_w64(bm > m_run + kLazyRescaleLog2) != 0;
  alpha = 1.f;
  if (rescale) {
    const float m_new = fmaxf(m_run, bm);
    alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    m_run = m_new;
  }
  float p[8];
  float ps = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p[i] = __builtin_amdgcn_exp2f(x[i] - m_run);
    ps += p[i];
  }
  l_run += ps;
  u32x4 pb;
  pb[0] = pack_bf16x2(p[0], p[1]);
  pb[1] = pack_bf16x2(p[2], p[3]);
  pb[2] = pack_bf16x2(p[4], p[5]);
  pb[3] = pack_bf16x2(p[6], p[7]);
  return pb;
}

// PV update of C output tiles from the 8 V vectors vr[i] (token pv_token(i,j),
// C columns starting at C*n16 of the lane's 16*C-column slice, as C / 2
// dwords of bf16 pairs).  Tile e covers columns C*m + e of the slice.  The
// accumulators are scaled by alpha first when the softmax moved its
// reference max.
template <int C, class VT>
__device__ __forceinline__ void pv_block(f32x4 (&acc)[C], const VT (&vr)[8], const u32x4& pb,
                                         float alpha, bool rescale) {
  static_assert(C % 2 == 0, "columns per lane come in bf16 pairs");
  if (rescale) {
#pragma unroll
    for (int e = 0; e < C; ++e) acc[e] = acc[e] * alpha;
  }
#pragma unroll
  for (int e = 0; e < C; ++e) {
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
    acc[e] = mfma16x16x32(va, pb, acc[e]);
  }
}

}  // namespace ws
