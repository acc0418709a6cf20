// AVX-512 BF16 kernels of the host partial (libwshost.so).
//
// Each kernel attends the query heads of one row over a token range
// [t0, t1) of that row and folds the result into an online-softmax state:
//   m[h]  running max of the scaled scores, log2 domain (-inf when empty),
//   l[h]  running sum of 2^(score - m),
//   o     running sum of 2^(score - m) * v, fp32, in *staging order*.
// Staging order: the value columns come out of the bf16 pair interleave
// (vpunpck{l,h}wd of two tokens' rows) permuted inside each 32-column chunk;
// column d of chunk c sits at slot stage_slot(d) below.  Callers keep o in
// staging order until the final write, which un-permutes it.  A width that
// is not a multiple of 32 ends with a 16-column chunk, staged in column
// order.
#pragma once

#include <cstddef>
#include <cstdint>

namespace wh {

// Column held by slot s of a D-column row in staging order: inside a
// 32-column chunk, slot 16*half + i holds column 8*(i/4) + 4*half + i%4; the
// slots of a last 16-column chunk hold their own columns.
inline int stage_col(int s, int D) {
  if (s >= (D & ~31)) return s;
  const int c = s >> 5, half = (s >> 4) & 1, i = s & 15;
  return 32 * c + 8 * (i >> 2) + 4 * half + (i & 3);
}

// Zero row used in place of tokens past the end of a range (no read past
// the caller's buffers).  Wide enough for the 576-column MLA latent.
extern const uint16_t kZeroRow[1024];

// GQA: q holds G rows of Dk bf16 (the query heads sharing one KV head); token
// t of the row is k + t*Dk / v + t*Dv.  (Dk, Dv): Dk == Dv a multiple of 16
// up to 256, or (192, 128) (gqa_dims_supported); G at most 16.  m, l: G
// floats; o: G*Dv floats (staging order).  scale_log2 = softmax scale *
// log2(e).
bool gqa_dims_supported(int Dk, int Dv);
void gqa_attend(const uint16_t* q, const uint16_t* k, const uint16_t* v, int G, int Dk,
                int Dv, int t0, int t1, float scale_log2, float* m, float* l, float* o);

// GQA over fp32 q / K / V (the float32 inputs the reference CPU kernel also
// takes): the same layout as gqa_attend with floats; (Dk, Dv): Dk == Dv a
// multiple of 16 up to 256, or (192, 128) (gqa_f32_dims_supported); G at
// most 16.  o: G*Dv floats in natural column order (no staging); the
// probabilities enter PV in fp32.
bool gqa_f32_dims_supported(int Dk, int Dv);
void gqa_attend_f32(const float* q, const float* k, const float* v, int G, int Dk, int Dv,
                    int t0, int t1, float scale_log2, float* m, float* l, float* o);

// MLA (absorbed, 16 heads): qt is the query in pair-transposed form
// (mla_prepare_q); token t's latent is c + t*c_tok (512 bf16, also the value)
// and pe + t*pe_tok (64 bf16).  m, l: 16 floats; o: 512*16 floats, slot-major
// (o[s*16 + h]).  vst is scratch of kMlaScratchWords 32-bit words.
constexpr int kMlaHeads = 16;
constexpr int kMlaC = 512;
constexpr int kMlaPe = 64;
constexpr int kMlaPairs = (kMlaC + kMlaPe) / 2;          // 288
constexpr size_t kMlaScratchWords = 16 * kMlaC;          // 16 token pairs x 512 columns
constexpr size_t kMlaQtWords = (size_t)kMlaPairs * kMlaHeads;
void mla_prepare_q(const uint16_t* q_nope, const uint16_t* q_pe, uint32_t* qt);
void mla_attend(const uint32_t* qt, const uint16_t* c, size_t c_tok, const uint16_t* pe,
                size_t pe_tok, int t0, int t1, float scale_log2, float* m, float* l, float* o,
                uint32_t* vst);

// Final rows of an MLA state (16 heads): row h of out (row stride
// out_stride elements) gets o[s*16 + h] * inv[h] in column order, as fp32 or
// as bf16 rounded to nearest even (a NaN stays a quiet NaN) -- the values
// and rounding of the scalar write, 16 heads at a time.
void mla_final_f32(const float* o, const float* inv, float* out, size_t out_stride);
void mla_final_bf16(const float* o, const float* inv, uint16_t* out, size_t out_stride);

// o part of an MLA state combine: dst[i] = sum over s < cnt of
// w[s*16 + i%16] * src[s][i] for the 512*16 slot-major values (multiplies
// and adds, in source order, as the scalar combine).
void mla_combine_o(const float* const* src, const float* w, int cnt, float* dst);

// Sum of `words` doubles (a multiple of 8) streamed with 512-bit loads: the
// reading side of the host bandwidth probe.
double sum_lines(const double* p, size_t words);

}  // namespace wh
