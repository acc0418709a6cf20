// AVX-512 BF16 kernels of the host partial.  Compiled with
// -mavx512f -mavx512bw -mavx512vl -mavx512bf16; called only after the
// library has checked the CPU supports them.
//
// GQA (per KV row, G query heads, head_dim D):
//   QK   for 16 tokens at a time, acc[j] += vdpbf16ps(q chunk, k_j chunk)
//        over the D/32 chunks, then one transpose-add tree turns the 16
//        accumulators into one vector of 16 token scores;
//   PV   the value rows of two tokens are interleaved as bf16 pairs
//        (vpunpck{l,h}wd) once per block, and every head accumulates
//        o += vdpbf16ps(broadcast (p_t, p_t+1), pair row) in fp32.
// MLA (per sequence, 16 heads sharing a 576-wide latent):
//   lanes are heads throughout, so no horizontal reductions: the query is
//   pair-transposed once per range (qt[p][h] = (q_h[2p], q_h[2p+1])), scores
//   are acc_t += vdpbf16ps(qt[p], broadcast latent pair p of token t), the
//   softmax is vertical over tokens, and PV is o[d] += vdpbf16ps(
//   (p_t, p_t+1) per head, broadcast (c_t[d], c_t+1[d])).
// Probabilities enter PV rounded to bf16 (as on the GPU path); the running
// sum l adds the fp32 probabilities.
// GQA over fp32 inputs: the same blocks with fp32 FMAs (scores through the
// same transpose-add tree), value rows read as they are, probabilities fp32.
#include "wh_kernels.h"

#include <immintrin.h>

#include <cmath>
#include <cstring>

namespace wh {

alignas(64) const uint16_t kZeroRow[1024] = {};

namespace {

// 2^x.  x = n + f with n = round(x), |f| <= 1/2; 2^f = e^(f ln 2) from the
// Taylor series to degree 6 (relative error below 2e-7 on |f| <= 1/2); 2^n is
// applied with vscalefps.  x is clamped at -250, where the result flushes to 0.
inline __m512 exp2v(__m512 x) {
  x = _mm512_max_ps(x, _mm512_set1_ps(-250.f));
  const __m512 n = _mm512_roundscale_ps(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m512 y = _mm512_mul_ps(_mm512_sub_ps(x, n), _mm512_set1_ps(0.6931471805599453f));
  __m512 p = _mm512_set1_ps(1.f / 720.f);
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f / 120.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f / 24.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f / 6.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(0.5f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f));
  p = _mm512_fmadd_ps(p, y, _mm512_set1_ps(1.f));
  return _mm512_scalef_ps(p, n);
}

// Lane j of the result is the sum of the 16 lanes of a[j].  Four levels of
// 128-bit / 32-bit shuffles and adds; the tree leaves lane 4Q+e holding
// a[{0,2,1,3}[e] + {0,8,4,12}[Q]], which the final permute puts in order.
inline __m512 reduce16(const __m512* a) {
  __m512 b[8], c[4], d[2];
#pragma GCC unroll 8
  for (int j = 0; j < 8; ++j)
    b[j] = _mm512_add_ps(_mm512_shuffle_f32x4(a[j], a[j + 8], _MM_SHUFFLE(1, 0, 1, 0)),
                         _mm512_shuffle_f32x4(a[j], a[j + 8], _MM_SHUFFLE(3, 2, 3, 2)));
#pragma GCC unroll 4
  for (int j = 0; j < 4; ++j)
    c[j] = _mm512_add_ps(_mm512_shuffle_f32x4(b[j], b[j + 4], _MM_SHUFFLE(2, 0, 2, 0)),
                         _mm512_shuffle_f32x4(b[j], b[j + 4], _MM_SHUFFLE(3, 1, 3, 1)));
#pragma GCC unroll 2
  for (int j = 0; j < 2; ++j)
    d[j] = _mm512_add_ps(_mm512_shuffle_ps(c[j], c[j + 2], _MM_SHUFFLE(1, 0, 1, 0)),
                         _mm512_shuffle_ps(c[j], c[j + 2], _MM_SHUFFLE(3, 2, 3, 2)));
  const __m512 e = _mm512_add_ps(_mm512_shuffle_ps(d[0], d[1], _MM_SHUFFLE(2, 0, 2, 0)),
                                 _mm512_shuffle_ps(d[0], d[1], _MM_SHUFFLE(3, 1, 3, 1)));
  const __m512i idx = _mm512_setr_epi32(0, 2, 1, 3, 8, 10, 9, 11, 4, 6, 5, 7, 12, 14, 13, 15);
  return _mm512_permutexvar_ps(idx, e);
}

inline __m512bh ld_bh(const void* p) { return (__m512bh)_mm512_loadu_si512(p); }

// acc + vdpbf16ps(a, the bf16 pair at p in every lane), with the pair as the
// instruction's {1to16} memory operand: one instruction, where the intrinsic
// over a broadcast compiles to a separate vpbroadcastd load per product.
inline __m512 dp_pair(__m512 acc, __m512bh a, const void* p) {
  asm("vdpbf16ps %2%{1to16%}, %1, %0" : "+v"(acc) : "v"(a), "m"(*(const int32_t*)p));
  return acc;
}

// The 16 bf16 values at p in the low half of a zmm, zeros above (no read
// past them).
inline __m512i ld16(const void* p) { return _mm512_maskz_loadu_epi16(0xFFFFu, p); }

// Interleaves the value rows of tokens (a, b) as bf16 pairs into dst (D words,
// staging order; a last 16-column chunk in column order).
template <int D>
inline void stage_pair(const uint16_t* a, const uint16_t* b, uint32_t* dst) {
#pragma GCC unroll 8
  for (int c = 0; c < D / 32; ++c) {
    const __m512i x = _mm512_loadu_si512(a + 32 * c), y = _mm512_loadu_si512(b + 32 * c);
    _mm512_store_si512(dst + 32 * c, _mm512_unpacklo_epi16(x, y));
    _mm512_store_si512(dst + 32 * c + 16, _mm512_unpackhi_epi16(x, y));
  }
  if constexpr (D % 32 != 0) {
    constexpr int c = D / 32;
    const __m512i x = ld16(a + 32 * c), y = ld16(b + 32 * c);
    // 128-bit lanes 0, 1 of unpacklo hold the pairs of columns 0-3, 8-11; of
    // unpackhi 4-7, 12-15
    const __m512i idx = _mm512_setr_epi64(0, 1, 8, 9, 2, 3, 10, 11);
    _mm512_store_si512(dst + 32 * c, _mm512_permutex2var_epi64(_mm512_unpacklo_epi16(x, y),
                                                               idx,
                                                               _mm512_unpackhi_epi16(x, y)));
  }
}

// ---------------------------------------------------------------------------
// GQA

// Scores of the 16 tokens at k (token j at k + j*D) against one head.
template <int D>
inline __m512 gqa_scores16(const uint16_t* qg, const uint16_t* k) {
  __m512 acc[16];
#pragma GCC unroll 16
  for (int j = 0; j < 16; ++j) acc[j] = _mm512_setzero_ps();
#pragma GCC unroll 8
  for (int c = 0; c < D / 32; ++c) {
    const __m512bh qv = ld_bh(qg + 32 * c);
#pragma GCC unroll 16
    for (int j = 0; j < 16; ++j) acc[j] = _mm512_dpbf16_ps(acc[j], qv, ld_bh(k + j * D + 32 * c));
  }
  if constexpr (D % 32 != 0) {  // a last 16-column chunk, zeros in the upper half
    constexpr int c = D / 32;
    const __m512bh qv = (__m512bh)ld16(qg + 32 * c);
#pragma GCC unroll 16
    for (int j = 0; j < 16; ++j)
      acc[j] = _mm512_dpbf16_ps(acc[j], qv, (__m512bh)ld16(k + j * D + 32 * c));
  }
  return reduce16(acc);
}

// o[0 .. 16W) = o * corr + sum over the np staged pairs.
template <int W, int D>
inline void gqa_pv(float* og, const uint32_t* vst, const uint32_t* pw, int np, __m512 corr) {
  __m512 acc[W];
#pragma GCC unroll 8
  for (int r = 0; r < W; ++r) acc[r] = _mm512_mul_ps(_mm512_loadu_ps(og + 16 * r), corr);
  for (int kq = 0; kq < np; ++kq) {
    const __m512bh bp = (__m512bh)_mm512_set1_epi32((int)pw[kq]);
    const uint32_t* src = vst + (size_t)kq * D;
#pragma GCC unroll 8
    for (int r = 0; r < W; ++r)
      acc[r] = _mm512_dpbf16_ps(acc[r], bp, (__m512bh)_mm512_load_si512(src + 16 * r));
  }
#pragma GCC unroll 8
  for (int r = 0; r < W; ++r) _mm512_storeu_ps(og + 16 * r, acc[r]);
}

// DK: key width (q rows and k tokens), D: value width (v tokens and o).
template <int DK, int D>
void gqa_attend_d(const uint16_t* q, const uint16_t* k, const uint16_t* v, int G, int t0,
                  int t1, float sl2, float* m, float* l, float* o) {
  constexpr int NZ = D / 16;  // zmm per value row
  alignas(64) float sc[16][32];
  alignas(64) uint32_t vst[16 * D];
  alignas(64) uint32_t pw[16];
  alignas(64) uint16_t tile[16 * DK];
  const __m512 ninf = _mm512_set1_ps(-INFINITY);
  const __m512 vsl2 = _mm512_set1_ps(sl2);
  for (int tb = t0; tb < t1; tb += 32) {
    const int n = t1 - tb < 32 ? t1 - tb : 32;
    // scores
    for (int half = 0; half < 2; ++half) {
      const int valid = n - 16 * half;
      if (valid <= 0) {
        for (int g = 0; g < G; ++g) _mm512_store_ps(sc[g] + 16 * half, ninf);
        continue;
      }
      const uint16_t* kb = k + (size_t)(tb + 16 * half) * DK;
      if (valid < 16) {  // copy the tail into a zeroed tile: no read past the range
        std::memset(tile, 0, sizeof(tile));
        std::memcpy(tile, kb, sizeof(uint16_t) * valid * DK);
        kb = tile;
      }
      const __mmask16 vm = valid < 16 ? (__mmask16)((1u << valid) - 1) : (__mmask16)0xFFFF;
      for (int g = 0; g < G; ++g) {
        const __m512 s = _mm512_mul_ps(gqa_scores16<DK>(q + (size_t)g * DK, kb), vsl2);
        _mm512_store_ps(sc[g] + 16 * half, _mm512_mask_blend_ps(vm, ninf, s));
      }
    }
    // value pairs
    const int np = (n + 1) >> 1;
    for (int kq = 0; kq < np; ++kq) {
      const uint16_t* va = v + (size_t)(tb + 2 * kq) * D;
      stage_pair<D>(va, 2 * kq + 1 < n ? va + D : kZeroRow, vst + (size_t)kq * D);
    }
    // online softmax and PV per head
    for (int g = 0; g < G; ++g) {
      const __m512 s0 = _mm512_load_ps(sc[g]), s1 = _mm512_load_ps(sc[g] + 16);
      const float mx = _mm512_reduce_max_ps(_mm512_max_ps(s0, s1));
      const float mo = m[g];
      const float mn = mo > mx ? mo : mx;
      const float corr = std::exp2(mo - mn);  // 0 when the state is empty
      const __m512 mnv = _mm512_set1_ps(mn);
      const __m512 p0 = exp2v(_mm512_sub_ps(s0, mnv)), p1 = exp2v(_mm512_sub_ps(s1, mnv));
      l[g] = l[g] * corr + _mm512_reduce_add_ps(_mm512_add_ps(p0, p1));
      m[g] = mn;
      _mm512_store_si512(pw, (__m512i)_mm512_cvtne2ps_pbh(p1, p0));  // word t = p_t
      float* og = o + (size_t)g * D;
      const __m512 cv = _mm512_set1_ps(corr);
      int z = 0;
      for (; z + 8 <= NZ; z += 8) gqa_pv<8, D>(og + 16 * z, vst + 16 * z, pw, np, cv);
      if constexpr (NZ % 8 != 0) gqa_pv<NZ % 8, D>(og + 16 * z, vst + 16 * z, pw, np, cv);
    }
  }
}

}  // namespace

bool gqa_dims_supported(int Dk, int Dv) {
  return (Dk == Dv && Dk >= 16 && Dk <= 256 && Dk % 16 == 0) || (Dk == 192 && Dv == 128);
}

void gqa_attend(const uint16_t* q, const uint16_t* k, const uint16_t* v, int G, int Dk,
                int Dv, int t0, int t1, float sl2, float* m, float* l, float* o) {
  if (Dk == 192 && Dv == 128) return gqa_attend_d<192, 128>(q, k, v, G, t0, t1, sl2, m, l, o);
  if (Dk != Dv) return;  // rejected by the caller
  switch (Dk) {
#define WH_BF16_CASE(DD) \
  case DD:               \
    return gqa_attend_d<DD, DD>(q, k, v, G, t0, t1, sl2, m, l, o);
    WH_BF16_CASE(16) WH_BF16_CASE(32) WH_BF16_CASE(48) WH_BF16_CASE(64)
    WH_BF16_CASE(80) WH_BF16_CASE(96) WH_BF16_CASE(112) WH_BF16_CASE(128)
    WH_BF16_CASE(144) WH_BF16_CASE(160) WH_BF16_CASE(176) WH_BF16_CASE(192)
    WH_BF16_CASE(208) WH_BF16_CASE(224) WH_BF16_CASE(240) WH_BF16_CASE(256)
#undef WH_BF16_CASE
    default: return;  // rejected by the caller
  }
}

// ---------------------------------------------------------------------------
// GQA, fp32 inputs

namespace {

// Scores of the 16 fp32 tokens at k (token j at k + j*DK) against one head.
template <int DK>
inline __m512 gqa_scores16_f32(const float* qg, const float* k) {
  __m512 acc[16];
#pragma GCC unroll 16
  for (int j = 0; j < 16; ++j) acc[j] = _mm512_setzero_ps();
#pragma GCC unroll 16
  for (int c = 0; c < DK / 16; ++c) {
    const __m512 qv = _mm512_loadu_ps(qg + 16 * c);
#pragma GCC unroll 16
    for (int j = 0; j < 16; ++j)
      acc[j] = _mm512_fmadd_ps(qv, _mm512_loadu_ps(k + j * DK + 16 * c), acc[j]);
  }
  return reduce16(acc);
}

// DK: key width, D: value width (both multiples of 16).  Per 32-token
// block: the scores of all heads, then per head the online-softmax update
// and o = o * corr + sum_t p_t v_t with fp32 FMAs.
template <int DK, int D>
void gqa_attend_f32_d(const float* q, const float* k, const float* v, int G, int t0, int t1,
                      float sl2, float* m, float* l, float* o) {
  constexpr int NZ = D / 16;  // zmm per value row
  alignas(64) float sc[16][32];
  alignas(64) float pt[32];
  alignas(64) float tile[16 * DK];
  const __m512 ninf = _mm512_set1_ps(-INFINITY);
  const __m512 vsl2 = _mm512_set1_ps(sl2);
  for (int tb = t0; tb < t1; tb += 32) {
    const int n = t1 - tb < 32 ? t1 - tb : 32;
    for (int half = 0; half < 2; ++half) {
      const int valid = n - 16 * half;
      if (valid <= 0) {
        for (int g = 0; g < G; ++g) _mm512_store_ps(sc[g] + 16 * half, ninf);
        continue;
      }
      const float* kb = k + (size_t)(tb + 16 * half) * DK;
      if (valid < 16) {  // copy the tail into a zeroed tile: no read past the range
        std::memset(tile, 0, sizeof(tile));
        std::memcpy(tile, kb, sizeof(float) * valid * DK);
        kb = tile;
      }
      const __mmask16 vm = valid < 16 ? (__mmask16)((1u << valid) - 1) : (__mmask16)0xFFFF;
      for (int g = 0; g < G; ++g) {
        const __m512 s = _mm512_mul_ps(gqa_scores16_f32<DK>(q + (size_t)g * DK, kb), vsl2);
        _mm512_store_ps(sc[g] + 16 * half, _mm512_mask_blend_ps(vm, ninf, s));
      }
    }
    const float* vb = v + (size_t)tb * D;
    for (int g = 0; g < G; ++g) {
      const __m512 s0 = _mm512_load_ps(sc[g]), s1 = _mm512_load_ps(sc[g] + 16);
      const float mx = _mm512_reduce_max_ps(_mm512_max_ps(s0, s1));
      const float mo = m[g];
      const float mn = mo > mx ? mo : mx;
      const float corr = std::exp2(mo - mn);  // 0 when the state is empty
      const __m512 mnv = _mm512_set1_ps(mn);
      const __m512 p0 = exp2v(_mm512_sub_ps(s0, mnv)), p1 = exp2v(_mm512_sub_ps(s1, mnv));
      l[g] = l[g] * corr + _mm512_reduce_add_ps(_mm512_add_ps(p0, p1));
      m[g] = mn;
      _mm512_store_ps(pt, p0);
      _mm512_store_ps(pt + 16, p1);
      float* og = o + (size_t)g * D;
      const __m512 cv = _mm512_set1_ps(corr);
      __m512 acc[NZ];
#pragma GCC unroll 16
      for (int r = 0; r < NZ; ++r) acc[r] = _mm512_mul_ps(_mm512_loadu_ps(og + 16 * r), cv);
      for (int t = 0; t < n; ++t) {
        const __m512 pv = _mm512_set1_ps(pt[t]);
        const float* vr = vb + (size_t)t * D;
#pragma GCC unroll 16
        for (int r = 0; r < NZ; ++r)
          acc[r] = _mm512_fmadd_ps(pv, _mm512_loadu_ps(vr + 16 * r), acc[r]);
      }
#pragma GCC unroll 16
      for (int r = 0; r < NZ; ++r) _mm512_storeu_ps(og + 16 * r, acc[r]);
    }
  }
}

}  // namespace

bool gqa_f32_dims_supported(int Dk, int Dv) {
  return (Dk == Dv && Dk >= 16 && Dk <= 256 && Dk % 16 == 0) || (Dk == 192 && Dv == 128);
}

void gqa_attend_f32(const float* q, const float* k, const float* v, int G, int Dk, int Dv,
                    int t0, int t1, float sl2, float* m, float* l, float* o) {
  if (Dk == 192 && Dv == 128)
    return gqa_attend_f32_d<192, 128>(q, k, v, G, t0, t1, sl2, m, l, o);
  if (Dk != Dv) return;  // rejected by the caller
#define WH_F32_CASE(DD) \
  case DD: return gqa_attend_f32_d<DD, DD>(q, k, v, G, t0, t1, sl2, m, l, o);
  switch (Dk) {
    WH_F32_CASE(16) WH_F32_CASE(32) WH_F32_CASE(48) WH_F32_CASE(64)
    WH_F32_CASE(80) WH_F32_CASE(96) WH_F32_CASE(112) WH_F32_CASE(128)
    WH_F32_CASE(144) WH_F32_CASE(160) WH_F32_CASE(176) WH_F32_CASE(192)
    WH_F32_CASE(208) WH_F32_CASE(224) WH_F32_CASE(240) WH_F32_CASE(256)
    default: return;  // rejected by the caller
  }
#undef WH_F32_CASE
}

// ---------------------------------------------------------------------------
// MLA

void mla_prepare_q(const uint16_t* q_nope, const uint16_t* q_pe, uint32_t* qt) {
  for (int h = 0; h < kMlaHeads; ++h) {
    for (int p = 0; p < kMlaC / 2; ++p)
      std::memcpy(qt + (size_t)p * kMlaHeads + h, q_nope + (size_t)h * kMlaC + 2 * p, 4);
    for (int p = 0; p < kMlaPe / 2; ++p)
      std::memcpy(qt + (size_t)(kMlaC / 2 + p) * kMlaHeads + h, q_pe + (size_t)h * kMlaPe + 2 * p,
                  4);
  }
}

namespace {

// Scores (lanes = heads) of 16 tokens: latent row j at c + j*CT, rope row at
// pe + j*PT (token strides known at compile time, so each row is an
// immediate displacement off one base register).
// pf_c / pf_pe: the next 16 tokens' rows, prefetched one cache line per
// pair step (256 lines from pf_c, 32 from pf_pe: the 16 rows of either
// compiled layout), so the next group streams in while this one computes;
// nullptr for none.
template <int CT, int PT>
inline void mla_scores16(const uint32_t* qt, const uint16_t* c, const uint16_t* pe,
                         __m512* acc, const char* pf_c = nullptr, const char* pf_pe = nullptr) {
#pragma GCC unroll 16
  for (int j = 0; j < 16; ++j) acc[j] = _mm512_setzero_ps();
  for (int p = 0; p < kMlaC / 2; ++p) {
    if (pf_c) _mm_prefetch(pf_c + 64 * p, _MM_HINT_T0);
    const __m512bh qv = (__m512bh)_mm512_loadu_si512(qt + 16 * p);
#pragma GCC unroll 16
    for (int j = 0; j < 16; ++j)
      acc[j] = dp_pair(acc[j], qv, c + j * CT + 2 * p);
  }
  for (int p = 0; p < kMlaPe / 2; ++p) {
    if (pf_pe) _mm_prefetch(pf_pe + 64 * p, _MM_HINT_T0);
    const __m512bh qv = (__m512bh)_mm512_loadu_si512(qt + 16 * (kMlaC / 2 + p));
#pragma GCC unroll 16
    for (int j = 0; j < 16; ++j)
      acc[j] = dp_pair(acc[j], qv, pe + j * PT + 2 * p);
  }
}

// CT, PT: the caller's token strides when they are one of the compiled
// layouts (separate 512 / 64 rows, or shared 576-wide rows); 0 for any other
// stride, which gathers every 16 tokens into a dense tile first.
template <int CT, int PT>
void mla_attend_t(const uint32_t* qt, const uint16_t* c, size_t c_tok, const uint16_t* pe,
                  size_t pe_tok, int t0, int t1, float sl2, float* m, float* l, float* o,
                  uint32_t* vst) {
  alignas(64) float sc[32][16];
  alignas(64) uint32_t p2[16][16];
  alignas(64) uint16_t tc[16 * kMlaC];
  alignas(64) uint16_t tpe[16 * kMlaPe];
  constexpr bool dense = CT != 0;
  // word 2h <- p_a[h], word 2h + 1 <- p_b[h] of the packed [p_a | p_b]
  const __m512i ilv = _mm512_set_epi16(31, 15, 30, 14, 29, 13, 28, 12, 27, 11, 26, 10, 25, 9,
                                       24, 8, 23, 7, 22, 6, 21, 5, 20, 4, 19, 3, 18, 2, 17, 1,
                                       16, 0);
  const __m512 vsl2 = _mm512_set1_ps(sl2);
  __m512 mv = _mm512_loadu_ps(m), lv = _mm512_loadu_ps(l);
  for (int tb = t0; tb < t1; tb += 32) {
    const int n = t1 - tb < 32 ? t1 - tb : 32;
    for (int grp = 0; grp < 2; ++grp) {
      const int valid = n - 16 * grp;
      if (valid <= 0) break;
      const size_t t = (size_t)(tb + 16 * grp);
      const uint16_t* cb = c + t * c_tok;
      const uint16_t* pb = pe + t * pe_tok;
      if (valid < 16 || !dense) {  // gather into a dense zero-padded tile
        const int cnt = valid < 16 ? valid : 16;
        if (cnt < 16) {
          std::memset(tc, 0, sizeof(tc));
          std::memset(tpe, 0, sizeof(tpe));
        }
        for (int j = 0; j < cnt; ++j) {
          std::memcpy(tc + j * kMlaC, cb + j * c_tok, 2 * kMlaC);
          std::memcpy(tpe + j * kMlaPe, pb + j * pe_tok, 2 * kMlaPe);
        }
        cb = tc;
        pb = tpe;
      }
      __m512 acc[16];
      if (cb == tc) {
        mla_scores16<kMlaC, kMlaPe>(qt, cb, pb, acc);
      } else {
        // the 16 tokens after these (in this range: the caller's range is one
        // page, so nothing past its end is touched)
        const bool more = t + 32 <= (size_t)t1;
        const char* pf_c = more ? (const char*)(cb + 16 * c_tok) : nullptr;
        const char* pf_pe = !more ? nullptr
                            : (CT == PT ? pf_c + 256 * 64 : (const char*)(pb + 16 * pe_tok));
        mla_scores16<(dense ? CT : kMlaC), (dense ? PT : kMlaPe)>(qt, cb, pb, acc, pf_c, pf_pe);
      }
#pragma GCC unroll 16
      for (int j = 0; j < 16; ++j) _mm512_store_ps(sc[16 * grp + j], _mm512_mul_ps(acc[j], vsl2));
    }
    __m512 mx = _mm512_set1_ps(-INFINITY);
    for (int j = 0; j < n; ++j) mx = _mm512_max_ps(mx, _mm512_load_ps(sc[j]));
    const __m512 mn = _mm512_max_ps(mv, mx);
    const __m512 corr = exp2v(_mm512_sub_ps(mv, mn));  // 0 where the state is empty
    lv = _mm512_mul_ps(lv, corr);
    const int np = (n + 1) >> 1;
    for (int kq = 0; kq < np; ++kq) {
      const __m512 pa = exp2v(_mm512_sub_ps(_mm512_load_ps(sc[2 * kq]), mn));
      const __m512 pb = 2 * kq + 1 < n ? exp2v(_mm512_sub_ps(_mm512_load_ps(sc[2 * kq + 1]), mn))
                                       : _mm512_setzero_ps();
      lv = _mm512_add_ps(lv, _mm512_add_ps(pa, pb));
      const __m512i packed = (__m512i)_mm512_cvtne2ps_pbh(pb, pa);
      _mm512_store_si512(p2[kq], _mm512_permutexvar_epi16(ilv, packed));
    }
    if (_mm512_cmp_ps_mask(corr, _mm512_set1_ps(1.f), _CMP_NEQ_UQ)) {
      for (int s = 0; s < kMlaC; ++s)
        _mm512_storeu_ps(o + 16 * s, _mm512_mul_ps(_mm512_loadu_ps(o + 16 * s), corr));
    }
    mv = mn;
    for (int kq = 0; kq < np; ++kq) {
      const uint16_t* ca = c + (size_t)(tb + 2 * kq) * c_tok;
      stage_pair<kMlaC>(ca, 2 * kq + 1 < n ? ca + c_tok : kZeroRow, vst + (size_t)kq * kMlaC);
    }
    for (int s0 = 0; s0 < kMlaC; s0 += 16) {
      __m512 acc[16];
#pragma GCC unroll 16
      for (int i = 0; i < 16; ++i) acc[i] = _mm512_loadu_ps(o + 16 * (s0 + i));
      for (int kq = 0; kq < np; ++kq) {
        const __m512bh pv = (__m512bh)_mm512_load_si512(p2[kq]);
        const uint32_t* src = vst + (size_t)kq * kMlaC + s0;
#pragma GCC unroll 16
        for (int i = 0; i < 16; ++i) acc[i] = dp_pair(acc[i], pv, src + i);
      }
#pragma GCC unroll 16
      for (int i = 0; i < 16; ++i) _mm512_storeu_ps(o + 16 * (s0 + i), acc[i]);
    }
  }
  _mm512_storeu_ps(m, mv);
  _mm512_storeu_ps(l, lv);
}

}  // namespace

double sum_lines(const double* p, size_t words) {
  __m512d a0 = _mm512_setzero_pd(), a1 = _mm512_setzero_pd();
  size_t i = 0;
  for (; i + 16 <= words; i += 16) {
    a0 = _mm512_add_pd(a0, _mm512_loadu_pd(p + i));
    a1 = _mm512_add_pd(a1, _mm512_loadu_pd(p + i + 8));
  }
  if (i < words) a0 = _mm512_add_pd(a0, _mm512_loadu_pd(p + i));
  return _mm512_reduce_add_pd(_mm512_add_pd(a0, a1));
}

namespace {

// In-register transpose of a 16 x 16 float tile: r[i] element j becomes r[j]
// element i (unpack pairs, then 128-bit lane shuffles).
inline void transpose16(__m512 (&r)[16]) {
  __m512 t[16];
  for (int i = 0; i < 16; i += 2) {
    t[i] = _mm512_unpacklo_ps(r[i], r[i + 1]);
    t[i + 1] = _mm512_unpackhi_ps(r[i], r[i + 1]);
  }
  for (int i = 0; i < 16; i += 4) {
    const __m512d a0 = _mm512_castps_pd(t[i]), a1 = _mm512_castps_pd(t[i + 1]);
    const __m512d b0 = _mm512_castps_pd(t[i + 2]), b1 = _mm512_castps_pd(t[i + 3]);
    r[i] = _mm512_castpd_ps(_mm512_unpacklo_pd(a0, b0));
    r[i + 1] = _mm512_castpd_ps(_mm512_unpackhi_pd(a0, b0));
    r[i + 2] = _mm512_castpd_ps(_mm512_unpacklo_pd(a1, b1));
    r[i + 3] = _mm512_castpd_ps(_mm512_unpackhi_pd(a1, b1));
  }
  // r[4g + k] now holds, in 128-bit lane L, row 4L + (k's pair) elements of
  // column block g; gather the lanes
  for (int i = 0; i < 4; ++i) {
    const __m512 a = r[i], b = r[4 + i], c = r[8 + i], d = r[12 + i];
    const __m512 ab0 = _mm512_shuffle_f32x4(a, b, 0x44), ab1 = _mm512_shuffle_f32x4(a, b, 0xee);
    const __m512 cd0 = _mm512_shuffle_f32x4(c, d, 0x44), cd1 = _mm512_shuffle_f32x4(c, d, 0xee);
    r[i] = _mm512_shuffle_f32x4(ab0, cd0, 0x88);
    r[4 + i] = _mm512_shuffle_f32x4(ab0, cd0, 0xdd);
    r[8 + i] = _mm512_shuffle_f32x4(ab1, cd1, 0x88);
    r[12 + i] = _mm512_shuffle_f32x4(ab1, cd1, 0xdd);
  }
}

// bf16 of 16 floats, nearest even, a NaN made quiet (the scalar to_out).
inline __m256i to_bf16(__m512 v) {
  const __m512i u = _mm512_castps_si512(v);
  const __m512i abs = _mm512_and_si512(u, _mm512_set1_epi32(0x7fffffff));
  const __mmask16 nan = _mm512_cmpgt_epu32_mask(abs, _mm512_set1_epi32(0x7f800000));
  const __m512i lsb = _mm512_and_si512(_mm512_srli_epi32(u, 16), _mm512_set1_epi32(1));
  const __m512i rnd = _mm512_add_epi32(_mm512_add_epi32(u, _mm512_set1_epi32(0x7fff)), lsb);
  __m512i r = _mm512_srli_epi32(rnd, 16);
  r = _mm512_mask_or_epi32(r, nan, _mm512_srli_epi32(u, 16), _mm512_set1_epi32(0x40));
  return _mm512_cvtepi32_epi16(r);
}

// The 32 staged slots of chunk c of every head, scaled: h0[h] holds slots
// 32c .. 32c+15 of head h, h1[h] slots 32c+16 .. 32c+31.
inline void mla_chunk(const float* o, __m512 vinv, int c, __m512 (&h0)[16], __m512 (&h1)[16]) {
  for (int k = 0; k < 16; ++k) {
    h0[k] = _mm512_mul_ps(_mm512_loadu_ps(o + (size_t)(32 * c + k) * 16), vinv);
    h1[k] = _mm512_mul_ps(_mm512_loadu_ps(o + (size_t)(32 * c + 16 + k) * 16), vinv);
  }
  transpose16(h0);
  transpose16(h1);
}

}  // namespace

// Slot 16*half + 4a + b of a chunk is column 8a + 4*half + b: the column
// order interleaves 4-column pieces of the two halves.
void mla_final_f32(const float* o, const float* inv, float* out, size_t out_stride) {
  const __m512 vinv = _mm512_loadu_ps(inv);
  const __m512i lo = _mm512_setr_epi32(0, 1, 2, 3, 16, 17, 18, 19, 4, 5, 6, 7, 20, 21, 22, 23);
  const __m512i hi = _mm512_setr_epi32(8, 9, 10, 11, 24, 25, 26, 27, 12, 13, 14, 15, 28, 29, 30,
                                       31);
  for (int c = 0; c < kMlaC / 32; ++c) {
    __m512 h0[16], h1[16];
    mla_chunk(o, vinv, c, h0, h1);
    for (int h = 0; h < 16; ++h) {
      float* dst = out + (size_t)h * out_stride + 32 * c;
      _mm512_storeu_ps(dst, _mm512_permutex2var_ps(h0[h], lo, h1[h]));
      _mm512_storeu_ps(dst + 16, _mm512_permutex2var_ps(h0[h], hi, h1[h]));
    }
  }
}

void mla_final_bf16(const float* o, const float* inv, uint16_t* out, size_t out_stride) {
  const __m512 vinv = _mm512_loadu_ps(inv);
  const __m512i idx = _mm512_setr_epi64(0, 8, 1, 9, 2, 10, 3, 11);
  for (int c = 0; c < kMlaC / 32; ++c) {
    __m512 h0[16], h1[16];
    mla_chunk(o, vinv, c, h0, h1);
    for (int h = 0; h < 16; ++h) {
      const __m512i a = _mm512_castsi256_si512(to_bf16(h0[h]));
      const __m512i b = _mm512_castsi256_si512(to_bf16(h1[h]));
      _mm512_storeu_si512(out + (size_t)h * out_stride + 32 * c,
                          _mm512_permutex2var_epi64(a, idx, b));
    }
  }
}

// Separate multiplies and adds (no contraction into FMAs), as the scalar
// combine computes them.
#pragma GCC push_options
#pragma GCC optimize("fp-contract=off")
void mla_combine_o(const float* const* src, const float* w, int cnt, float* dst) {
  constexpr int kH = kMlaHeads;
  for (int i = 0; i < kMlaC * kH; i += kH) {
    __m512 acc = _mm512_setzero_ps();
    for (int s = 0; s < cnt; ++s)
      acc = _mm512_add_ps(acc, _mm512_mul_ps(_mm512_loadu_ps(w + s * kH),
                                             _mm512_loadu_ps(src[s] + i)));
    _mm512_storeu_ps(dst + i, acc);
  }
}
#pragma GCC pop_options

void mla_attend(const uint32_t* qt, const uint16_t* c, size_t c_tok, const uint16_t* pe,
                size_t pe_tok, int t0, int t1, float sl2, float* m, float* l, float* o,
                uint32_t* vst) {
  if (c_tok == (size_t)kMlaC && pe_tok == (size_t)kMlaPe)
    mla_attend_t<kMlaC, kMlaPe>(qt, c, c_tok, pe, pe_tok, t0, t1, sl2, m, l, o, vst);
  else if (c_tok == (size_t)(kMlaC + kMlaPe) && pe_tok == (size_t)(kMlaC + kMlaPe))
    mla_attend_t<kMlaC + kMlaPe, kMlaC + kMlaPe>(qt, c, c_tok, pe, pe_tok, t0, t1, sl2, m, l,
                                                  o, vst);
  else
    mla_attend_t<0, 0>(qt, c, c_tok, pe, pe_tok, t0, t1, sl2, m, l, o, vst);
}

}  // namespace wh
