// libwshost.so: the host partial of the partitioned decode KV cache.
//
// Work plan (the same one the GPU kernels build on the device): the rows of
// a call (GQA row = (sequence, kv head), MLA row = sequence) are cut into
// 32-token blocks, T blocks in all; thread i of n takes the blocks
// [i*T/n, (i+1)*T/n) and walks them as row segments.  A segment that covers
// its whole row writes the final (out, lse); one that does not leaves its
// online-softmax state in slot i + row (distinct for every (thread, row)
// pair, because both coordinates only grow along the block order).  After a
// barrier, each split row is combined from the slots of its owner threads.
//
// This file is built for the baseline ISA; the kernels (wh_kernels.cpp) are
// built for AVX-512 BF16 and only reached after wh_isa_supported().
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <type_traits>
#include <vector>

#include "../../include/wshost.h"
#include "wh_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

constexpr int kBlock = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct Plan {
  std::vector<int64_t> pref;  // R + 1 exclusive prefix of blocks per row
  int64_t T = 0;
  int64_t start(int i, int n) const { return (int64_t)i * T / n; }
  int owner(int64_t blk, int n) const { return (int)(((blk + 1) * n + T - 1) / T) - 1; }
};

// State layout of one (row, heads) segment: m[H], l[H], o[H * Dv].
struct StateView {
  float* m;
  float* l;
  float* o;
};
inline StateView view(float* base, int H) { return {base, base + H, base + 2 * H}; }

void state_init(float* base, int H, int Dv) {
  for (int h = 0; h < H; ++h) base[h] = -INFINITY;
  std::memset(base + H, 0, sizeof(float) * (size_t)H * (Dv + 1));
}

// Per-head weights 2^(m_s - M) of `cnt` slot states (w[s*H + h]) and the
// combined m, l into dst.
void state_weights(const float* const* src, int cnt, int H, float* dst, float* w) {
  StateView d = view(dst, H);
  for (int h = 0; h < H; ++h) {
    float M = -INFINITY;
    for (int s = 0; s < cnt; ++s) M = std::max(M, src[s][h]);
    float L = 0.f;
    for (int s = 0; s < cnt; ++s) {
      const float ms = src[s][h];
      const float ws = (M == -INFINITY || ms == -INFINITY) ? 0.f : std::exp2(ms - M);
      w[(size_t)s * H + h] = ws;
      L += ws * src[s][H + h];
    }
    d.m[h] = M;
    d.l[h] = L;
  }
}

// Folds the states of `cnt` slots into dst (same layout); `oh(i)` is the head
// of o element i.
template <class HeadOf>
void state_combine(const float* const* src, int cnt, int H, int Dv, float* dst, HeadOf oh) {
  StateView d = view(dst, H);
  std::vector<float> w((size_t)cnt * H);
  state_weights(src, cnt, H, dst, w.data());
  const size_t no = (size_t)H * Dv;
  for (size_t i = 0; i < no; ++i) {
    const int h = oh(i);
    float acc = 0.f;
    for (int s = 0; s < cnt; ++s) acc += w[(size_t)s * H + h] * src[s][2 * H + i];
    d.o[i] = acc;
  }
}

bool isa_ok() {
  static const bool ok = __builtin_cpu_supports("avx512f") &&
                         __builtin_cpu_supports("avx512bw") &&
                         __builtin_cpu_supports("avx512bf16");
  return ok;
}

int resolve_threads(int n_threads, int64_t T) {
  int n = n_threads > 0 ? n_threads : omp_get_max_threads();
  n = std::min<int64_t>(n, 1024);
  return (int)std::max<int64_t>(1, std::min<int64_t>(n, T));
}

// Runs the plan.  seg(row, tok0, tok1, state) fills a state; fin(row, state)
// writes a row's output; empty(row) writes the empty result.  Slots hold
// states of rows split across threads.
template <class Seg, class Fin, class Empty, class Comb>
void run_plan(const Plan& P, int R, int H, int Dv, int n_req, const int32_t* row_len, Seg seg,
              Fin fin, Empty empty, Comb comb) {
  const size_t ssz = (size_t)H * (Dv + 2);
  if (P.T == 0) {
    for (int r = 0; r < R; ++r) empty(r);
    return;
  }
  const int n_want = resolve_threads(n_req, P.T);
  std::unique_ptr<float[]> slots(new float[(size_t)(n_want + R) * ssz]);
#pragma omp parallel num_threads(n_want)
  {
    const int n = omp_get_num_threads();  // the runtime may give fewer
    const int i = omp_get_thread_num();
    std::unique_ptr<float[]> st(new float[ssz]);
    int64_t b0 = P.start(i, n);
    const int64_t b1 = P.start(i + 1, n);
    int r = (int)(std::upper_bound(P.pref.begin(), P.pref.end(), b0) - P.pref.begin()) - 1;
    while (b0 < b1) {
      while (P.pref[r + 1] <= b0) ++r;  // rows without blocks
      const int64_t e = std::min(b1, P.pref[r + 1]);
      const int tk0 = (int)((b0 - P.pref[r]) * kBlock);
      const int tk1 = (int)std::min<int64_t>(row_len[r], (e - P.pref[r]) * kBlock);
      state_init(st.get(), H, Dv);
      seg(r, tk0, tk1, st.get());
      if (b0 == P.pref[r] && e == P.pref[r + 1])
        fin(r, st.get());
      else
        std::memcpy(slots.get() + (size_t)(i + r) * ssz, st.get(), sizeof(float) * ssz);
      b0 = e;
    }
#pragma omp barrier
    std::vector<const float*> src;
#pragma omp for schedule(static)
    for (int row = 0; row < R; ++row) {
      if (P.pref[row + 1] == P.pref[row]) {
        empty(row);
        continue;
      }
      const int o0 = P.owner(P.pref[row], n), o1 = P.owner(P.pref[row + 1] - 1, n);
      if (o0 == o1) continue;  // written by its only thread
      src.clear();
      for (int o = o0; o <= o1; ++o) src.push_back(slots.get() + (size_t)(o + row) * ssz);
      comb(src.data(), (int)src.size(), st.get());
      fin(row, st.get());
    }
  }
}

Plan make_plan(const int32_t* row_len, int R) {
  Plan P;
  P.pref.resize((size_t)R + 1);
  P.pref[0] = 0;
  for (int r = 0; r < R; ++r) P.pref[r + 1] = P.pref[r] + (row_len[r] + kBlock - 1) / kBlock;
  P.T = P.pref[R];
  return P;
}

// An output value as stored: fp32 as is, or bf16 rounded to nearest even
// (a NaN stays a quiet NaN).
inline float to_out(float v, float*) { return v; }
inline uint16_t to_out(float v, uint16_t*) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Where a call's rows go: the (out, lse) form, or the reference CPU kernel's
// triple (out, max, sum) (kernel/cpu_attn.cpp:540-567): max the row's largest
// scaled score in natural-log units, sum the sum of exp(score - max), out
// divided by sum when `normalize` (fused_cpu_attn) or not (fused_cpu_attn_mla,
// _mla_compressed).  Output row i of a call is out + i * Dv, lse[i] / mx[i] /
// sm[i].
template <class OutT>
struct Sink {
  OutT* out;
  float* lse;      // (out, lse) form; nullptr selects the triple form
  float* mx;       // triple form
  float* sm;
  bool normalize;  // triple form: out / sum
  bool ok() const { return out && (lse || (mx && sm)); }
};

template <class OutT>
void write_empty(const Sink<OutT>& k, size_t row0, int H, int Dv) {
  std::memset(k.out + row0 * Dv, 0, sizeof(OutT) * H * Dv);
  for (int h = 0; h < H; ++h) {
    if (k.lse) {
      k.lse[row0 + h] = -INFINITY;
    } else {
      k.mx[row0 + h] = -INFINITY;
      k.sm[row0 + h] = 0.f;
    }
  }
}

// Final rows row0 .. row0 + H - 1 of H heads from a state; o_at(h, s) reads o
// in staging order (kStaged) or in column order.  The state's m is the row
// max in log2 units (scores scaled by scale * log2(e)) and l the sum of
// 2^(score - m), which is the sum of exp(natural score - natural max).
template <class OutT, bool kStaged = true, class OAt>
void write_final(const float* base, int H, int Dv, const Sink<OutT>& k, size_t row0, OAt o_at) {
  for (int h = 0; h < H; ++h) {
    const size_t r = row0 + h;
    const float l = base[H + h];
    OutT* dst = k.out + r * Dv;
    if (!(l > 0.f)) {
      write_empty(k, r, 1, Dv);
      continue;
    }
    const float inv = (k.lse || k.normalize) ? 1.f / l : 1.f;
    for (int s = 0; s < Dv; ++s)
      dst[kStaged ? wh::stage_col(s, Dv) : s] = to_out(o_at(h, s) * inv, dst);
    if (k.lse) {
      k.lse[r] = (base[h] + std::log2(l)) * kLn2;
    } else {
      k.mx[r] = base[h] * kLn2;
      k.sm[r] = l;
    }
  }
}

// Validates the paging of a call: page size, lengths within the table, and
// every page id a length reaches inside the pool.
int check_pages(const char* fn, const int32_t* page_table, const int32_t* lens, int B,
                int page_size, int max_pages, int num_pages) {
  if (page_size < 1 || max_pages < 1 || num_pages < 1)
    return fail(WH_EINVAL, "%s: bad paging page_size=%d max_pages=%d num_pages=%d", fn,
                page_size, max_pages, num_pages);
  if (page_size % kBlock != 0 && max_pages != 1)
    return fail(WH_EINVAL, "%s: page_size %d is not a multiple of %d", fn, page_size, kBlock);
  const int64_t cap = (int64_t)page_size * max_pages;
  if (cap > (int64_t)1 << 30) return fail(WH_EINVAL, "%s: %lld tokens per sequence", fn,
                                          (long long)cap);
  for (int b = 0; b < B; ++b) {
    if (lens[b] < 0 || lens[b] > cap)
      return fail(WH_EINVAL, "%s: lens[%d] = %d outside [0, %lld]", fn, b, lens[b],
                  (long long)cap);
    const int np = (int)((lens[b] + (int64_t)page_size - 1) / page_size);
    for (int p = 0; p < np; ++p) {
      const int32_t pid = page_table[(size_t)b * max_pages + p];
      if (pid < 0 || pid >= num_pages)
        return fail(WH_EINVAL, "%s: page_table[%d][%d] = %d outside [0, %d)", fn, b, p, pid,
                    num_pages);
    }
  }
  return WH_OK;
}

// Calls f(page_id, a, e) for each page overlapping tokens [t0, t1) of a
// sequence, with [a, e) the overlap in page-local token indices.
template <class F>
void for_pages(const int32_t* table_row, int page_size, int t0, int t1, F f) {
  for (int t = t0; t < t1;) {
    const int p = t / page_size;
    const int e = std::min(t1, (p + 1) * page_size);
    f(table_row[p], t - p * page_size, e - p * page_size);
    t = e;
  }
}

}  // namespace

namespace {

// InT: uint16_t (bf16 inputs, the AVX-512 BF16 kernels) or float (fp32
// inputs, fp32 FMAs).
template <class InT, class OutT>
int attn_partial(const char* fn, const InT* q, const InT* k_pages, const InT* v_pages,
                 const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv, int Dk,
                 int D, int page_size, int max_pages, int num_pages, float scale,
                 const Sink<OutT>& sink, int n_threads) {
  constexpr bool kF32 = std::is_same_v<InT, float>;
  g_err[0] = '\0';
  if (!isa_ok()) return fail(WH_ENOTSUP, "%s: this CPU lacks AVX-512 F/BW/BF16", fn);
  if (B < 0 || Hkv < 1 || Hq < 1 || Hq % Hkv != 0)
    return fail(WH_EINVAL, "%s: bad shape B=%d Hq=%d Hkv=%d", fn, B, Hq, Hkv);
  const int G = Hq / Hkv;
  if (G > 16) return fail(WH_EINVAL, "%s: group size %d > 16", fn, G);
  if (kF32 ? !wh::gqa_f32_dims_supported(Dk, D) : !wh::gqa_dims_supported(Dk, D))
    return fail(WH_EINVAL,
                "%s: head_dim Dk=%d Dv=%d unsupported (equal multiples of 16 in [16, 256], "
                "or 192 / 128)",
                fn, Dk, D);
  if (B == 0) return WH_OK;
  if (!q || !k_pages || !v_pages || !page_table || !lens || !sink.ok())
    return fail(WH_EINVAL, "%s: null pointer", fn);
  if (int rc = check_pages(fn, page_table, lens, B, page_size, max_pages, num_pages)) return rc;
  const int R = B * Hkv;
  std::vector<int32_t> row_len((size_t)R);
  for (int r = 0; r < R; ++r) row_len[r] = lens[r / Hkv];
  const Plan P = make_plan(row_len.data(), R);
  const float sl2 = scale * kLog2e;
  auto seg = [&](int r, int t0, int t1, float* st) {
    const int b = r / Hkv, kvh = r % Hkv;
    StateView s = view(st, G);
    for_pages(page_table + (size_t)b * max_pages, page_size, t0, t1,
              [&](int pid, int a, int e) {
                const size_t head = ((size_t)pid * Hkv + kvh) * page_size;  // first token
                if constexpr (kF32)
                  wh::gqa_attend_f32(q + (size_t)r * G * Dk, k_pages + head * Dk,
                                     v_pages + head * D, G, Dk, D, a, e, sl2, s.m, s.l, s.o);
                else
                  wh::gqa_attend(q + (size_t)r * G * Dk, k_pages + head * Dk,
                                 v_pages + head * D, G, Dk, D, a, e, sl2, s.m, s.l, s.o);
              });
  };
  auto fin = [&](int r, const float* st) {
    write_final<OutT, !kF32>(st, G, D, sink, (size_t)r * G,
                             [&](int h, int s) { return st[2 * G + h * D + s]; });
  };
  auto empty = [&](int r) { write_empty(sink, (size_t)r * G, G, D); };
  run_plan(P, R, G, D, n_threads, row_len.data(), seg, fin, empty,
           [G, D](const float* const* src, int cnt, float* dst) {
             state_combine(src, cnt, G, D, dst, [D](size_t i) { return (int)(i / D); });
           });
  return WH_OK;
}

template <class OutT>
int mla_partial(const char* fn, const uint16_t* q_nope, const uint16_t* q_pe,
                const uint16_t* c_pages, int c_stride, const uint16_t* pe_pages, int pe_stride,
                const int32_t* page_table, const int32_t* lens, int B, int H, int page_size,
                int max_pages, int num_pages, float scale, const Sink<OutT>& sink,
                int n_threads) {
  using namespace wh;
  g_err[0] = '\0';
  if (!isa_ok()) return fail(WH_ENOTSUP, "%s: this CPU lacks AVX-512 F/BW/BF16", fn);
  if (B < 0) return fail(WH_EINVAL, "%s: bad batch %d", fn, B);
  if (H < kMlaHeads || H % kMlaHeads)
    return fail(WH_EINVAL, "%s: %d heads is not a multiple of %d", fn, H, kMlaHeads);
  if (c_stride < kMlaC || pe_stride < kMlaPe)
    return fail(WH_EINVAL, "%s: token strides %d / %d below 512 / 64", fn,
                c_stride, pe_stride);
  if (B == 0) return WH_OK;
  if (!q_nope || !q_pe || !c_pages || !pe_pages || !page_table || !lens || !sink.ok())
    return fail(WH_EINVAL, "%s: null pointer", fn);
  if (int rc = check_pages(fn, page_table, lens, B, page_size, max_pages,
                           num_pages))
    return rc;
  // Rows of the plan: (sequence b, 16-head group g), v = b * ng + g, whose
  // query / output rows are v * 16 + h = b * H + 16 g + h.
  const int ng = H / kMlaHeads;
  const int R = B * ng;
  const int Hg = kMlaHeads, Dv = kMlaC;
  std::vector<int32_t> row_len((size_t)R);
  for (int v = 0; v < R; ++v) row_len[v] = lens[v / ng];
  const Plan P = make_plan(row_len.data(), R);
  const float sl2 = scale * kLog2e;
  auto seg = [&](int v, int t0, int t1, float* st) {
    // per-thread scratch: the pair-transposed query, then the staged value
    // pairs (64-byte aligned: the kernel stores them with aligned stores)
    thread_local std::vector<uint32_t> scratch;
    scratch.resize(kMlaQtWords + kMlaScratchWords + 16);
    uint32_t* qt = scratch.data();
    qt += (64 - ((uintptr_t)qt & 63)) / 4 % 16;
    uint32_t* vs = qt + kMlaQtWords;
    mla_prepare_q(q_nope + (size_t)v * Hg * kMlaC, q_pe + (size_t)v * Hg * kMlaPe, qt);
    StateView s = view(st, Hg);
    for_pages(page_table + (size_t)(v / ng) * max_pages, page_size, t0, t1,
              [&](int pid, int a, int e) {
                const size_t tok0 = (size_t)pid * page_size;
                mla_attend(qt, c_pages + tok0 * c_stride, (size_t)c_stride,
                           pe_pages + tok0 * pe_stride, (size_t)pe_stride, a, e, sl2, s.m, s.l,
                           s.o, vs);
              });
  };
  // the 16 rows of a group, 16 heads at a time (AVX-512; the values and
  // rounding of write_final)
  auto fin = [&](int v, const float* st) {
    const size_t row0 = (size_t)v * Hg;
    float inv[kMlaHeads];
    for (int h = 0; h < Hg; ++h) {
      const float l = st[Hg + h];
      inv[h] = (sink.lse || sink.normalize) ? 1.f / l : 1.f;
    }
    if constexpr (std::is_same_v<OutT, uint16_t>)
      mla_final_bf16(st + 2 * Hg, inv, sink.out + row0 * Dv, (size_t)Dv);
    else
      mla_final_f32(st + 2 * Hg, inv, sink.out + row0 * Dv, (size_t)Dv);
    for (int h = 0; h < Hg; ++h) {
      const size_t r = row0 + h;
      const float l = st[Hg + h];
      if (!(l > 0.f)) {
        write_empty(sink, r, 1, Dv);
      } else if (sink.lse) {
        sink.lse[r] = (st[h] + std::log2(l)) * kLn2;
      } else {
        sink.mx[r] = st[h] * kLn2;
        sink.sm[r] = l;
      }
    }
  };
  auto empty = [&](int v) { write_empty(sink, (size_t)v * Hg, Hg, Dv); };
  run_plan(P, R, Hg, Dv, n_threads, row_len.data(), seg, fin, empty,
           [](const float* const* src, int cnt, float* dst) {
             std::vector<float> w((size_t)cnt * kMlaHeads);
             std::vector<const float*> so((size_t)cnt);
             for (int s = 0; s < cnt; ++s) so[s] = src[s] + 2 * kMlaHeads;  // the o parts
             state_weights(src, cnt, kMlaHeads, dst, w.data());
             mla_combine_o(so.data(), w.data(), cnt, dst + 2 * kMlaHeads);
           });
  return WH_OK;
}

}  // namespace

extern "C" {

const char* wh_last_error(void) { return g_err; }

const char* wh_version(void) { return "wshost 0.2 avx512bf16"; }

int wh_isa_supported(void) { return isa_ok() ? 1 : 0; }

int wh_gqa_partial(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                   const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                   int D, int page_size, int max_pages, int num_pages, float scale,
                   float* out, float* lse, int n_threads) {
  return attn_partial("wh_gqa_partial", q, k_pages, v_pages, page_table, lens, B, Hq, Hkv, D,
                      D, page_size, max_pages, num_pages, scale,
                      Sink<float>{out, lse, nullptr, nullptr, true}, n_threads);
}

int wh_gqa_partial_bf16(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                        const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                        int D, int page_size, int max_pages, int num_pages, float scale,
                        uint16_t* out, float* lse, int n_threads) {
  return attn_partial("wh_gqa_partial_bf16", q, k_pages, v_pages, page_table, lens, B, Hq, Hkv,
                      D, D, page_size, max_pages, num_pages, scale,
                      Sink<uint16_t>{out, lse, nullptr, nullptr, true}, n_threads);
}

int wh_attn_partial(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                    const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                    int Dk, int Dv, int page_size, int max_pages, int num_pages, float scale,
                    float* out, float* lse, int n_threads) {
  return attn_partial("wh_attn_partial", q, k_pages, v_pages, page_table, lens, B, Hq, Hkv, Dk,
                      Dv, page_size, max_pages, num_pages, scale,
                      Sink<float>{out, lse, nullptr, nullptr, true}, n_threads);
}

int wh_attn_partial_f32(const float* q, const float* k_pages, const float* v_pages,
                        const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                        int Dk, int Dv, int page_size, int max_pages, int num_pages,
                        float scale, float* out, float* lse, int n_threads) {
  return attn_partial("wh_attn_partial_f32", q, k_pages, v_pages, page_table, lens, B, Hq, Hkv,
                      Dk, Dv, page_size, max_pages, num_pages, scale,
                      Sink<float>{out, lse, nullptr, nullptr, true}, n_threads);
}

int wh_attn_triple(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                   const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                   int Dk, int Dv, int page_size, int max_pages, int num_pages, float scale,
                   int normalize, float* out, float* row_max, float* row_sum, int n_threads) {
  return attn_partial("wh_attn_triple", q, k_pages, v_pages, page_table, lens, B, Hq, Hkv, Dk,
                      Dv, page_size, max_pages, num_pages, scale,
                      Sink<float>{out, nullptr, row_max, row_sum, normalize != 0}, n_threads);
}

int wh_attn_triple_f32(const float* q, const float* k_pages, const float* v_pages,
                       const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                       int Dk, int Dv, int page_size, int max_pages, int num_pages, float scale,
                       int normalize, float* out, float* row_max, float* row_sum,
                       int n_threads) {
  return attn_partial("wh_attn_triple_f32", q, k_pages, v_pages, page_table, lens, B, Hq, Hkv,
                      Dk, Dv, page_size, max_pages, num_pages, scale,
                      Sink<float>{out, nullptr, row_max, row_sum, normalize != 0}, n_threads);
}

int wh_mla_partial(const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_pages,
                   int c_stride, const uint16_t* pe_pages, int pe_stride,
                   const int32_t* page_table, const int32_t* lens, int B, int H, int page_size,
                   int max_pages, int num_pages, float scale, float* out, float* lse,
                   int n_threads) {
  return mla_partial("wh_mla_partial", q_nope, q_pe, c_pages, c_stride, pe_pages, pe_stride,
                     page_table, lens, B, H, page_size, max_pages, num_pages, scale,
                     Sink<float>{out, lse, nullptr, nullptr, true}, n_threads);
}

int wh_mla_partial_bf16(const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_pages,
                        int c_stride, const uint16_t* pe_pages, int pe_stride,
                        const int32_t* page_table, const int32_t* lens, int B, int H,
                        int page_size, int max_pages, int num_pages, float scale,
                        uint16_t* out, float* lse, int n_threads) {
  return mla_partial("wh_mla_partial_bf16", q_nope, q_pe, c_pages, c_stride, pe_pages,
                     pe_stride, page_table, lens, B, H, page_size, max_pages, num_pages, scale,
                     Sink<uint16_t>{out, lse, nullptr, nullptr, true}, n_threads);
}

int wh_mla_triple(const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_pages,
                  int c_stride, const uint16_t* pe_pages, int pe_stride,
                  const int32_t* page_table, const int32_t* lens, int B, int H, int page_size,
                  int max_pages, int num_pages, float scale, int normalize, float* out,
                  float* row_max, float* row_sum, int n_threads) {
  return mla_partial("wh_mla_triple", q_nope, q_pe, c_pages, c_stride, pe_pages, pe_stride,
                     page_table, lens, B, H, page_size, max_pages, num_pages, scale,
                     Sink<float>{out, nullptr, row_max, row_sum, normalize != 0}, n_threads);
}

double wh_host_read_gbs(size_t bytes, int n_threads, int reps) {
  if (bytes < ((size_t)1 << 20) || reps < 1) return 0.0;
  if (!isa_ok()) return 0.0;
  const int n = n_threads > 0 ? n_threads : omp_get_max_threads();
  const size_t words = bytes / 64 * 8;  // 64-byte lines of 8 doubles
  std::unique_ptr<double[]> buf(new double[words]);
  double best = 0.0;
#pragma omp parallel num_threads(n)
  {
    // first touch by the reading threads (their pages on their memory)
#pragma omp for schedule(static)
    for (size_t i = 0; i < words; ++i) buf[i] = 1.0;
    for (int r = 0; r <= reps; ++r) {
#pragma omp barrier
      double t0 = 0.0;
#pragma omp master
      t0 = omp_get_wtime();
      const int nt = omp_get_num_threads(), it = omp_get_thread_num();
      const size_t lines = words / 8;
      const size_t l0 = lines * it / nt, l1 = lines * (it + 1) / nt;
      const double sum = wh::sum_lines(buf.get() + 8 * l0, 8 * (l1 - l0));
#pragma omp barrier
#pragma omp master
      {
        const double dt = omp_get_wtime() - t0;
        if (r > 0 && sum >= 0.0 && dt > 0.0) best = std::max(best, (double)(words * 8) / dt / 1e9);
      }
    }
  }
  return best;
}

}  // extern "C"
