// Split-KV GQA decode attention over the HBM partition (gfx950), optionally
// fused with the append of the decode step's new token.
//
// Work decomposition (ws_plan.h): the work list is every 32-token block of
// every kv row (kv row = b * Hkv + kvh), rows in order, and every *wave* of
// the grid is one split of the plan: split w streams the blocks
// [floor(w T / n), floor((w + 1) T / n)), so each wave reads the same number
// of bytes whatever the lengths.  A wave streams its range through a
// two-stage register ring that runs straight across row boundaries: while
// block i is consumed, block i + 1 (its K, V and the q rows of its kv row)
// is in flight, so a wave whose range spans two rows never drains and
// restarts its loads.  When the consumed block opens a new row, the finished
// row's piece (normalised out, lse) is written: to out/lse (fp32) when the
// wave held the whole row, else to workspace slot w + row (out in bf16),
// where ws_merge_split (or the one-launch entry points' own merge) finds it.
// Waves never wait for each other.
//
// The block metadata (kv row, pool token index, valid tokens, the new
// token's row) is computed 64 blocks at a time, one block per lane, page
// table reads included, and read in the loop with readlane: the loop issues
// no load whose address depends on another load in flight.
//
// With k_new != nullptr the call also appends one token per sequence: token
// len_in[b] of sequence b is read from k_new/v_new instead of the page, the
// wave that consumes that block writes it into its page slot from the
// registers it already holds, and len_out[b] = len_in[b] + 1.  No wave reads
// the slot being written and len_out is not read, so the fused step has no
// intra-launch race.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "ws_attn.h"
#include "ws_plan.h"
#include "ws_reduce.h"

namespace ws {

constexpr int kGqaD = 128;   // value width (and key width of the Dk == Dv calls)
constexpr int kGqaDk192 = 192;  // key width of the decompressed DeepSeek-V2 layout
constexpr int kGqaMaxD = 256;   // widest key / value rows
constexpr int kGqaWaves = 2;        // waves per workgroup, each its own split
constexpr int kGqaStages = 2;       // register stages of a wave's load ring
constexpr int kGqaSplitsPerCu = 2;  // default splits (waves) per CU

// Register stages of the ring: two 256-wide K and V stages (256 VGPRs) do
// not fit beside the accumulators and q even in the 512 registers of one wave
// per SIMD (the compiler spilled 730 bytes per lane), so 256-wide values
// stream one block per wave at a time.
__host__ __device__ constexpr int gqa_stages(int DV) { return DV > kGqaD ? 1 : kGqaStages; }
// Waves per SIMD the kernel is compiled for (its register budget): rings
// wider than 128 need the 512 registers of one wave per SIMD, and so does the
// 128-wide ring with the group size read at run time (G = 0: it spilled in
// 256).  The grid never places more than one wave per SIMD, so this costs no
// occupancy the launch uses.
__host__ __device__ constexpr int gqa_waves_per_simd(int G, int DK, int DV) {
  return G > 0 && DK <= kGqaD && DV <= kGqaD ? 2 : 1;
}

// Value columns per lane of a DV-wide row: the smallest even count >= DV / 16
// that divides DV (64: 4, 128: 8, 256: 16; 80: 8).  Lanes n16 < DV / C hold
// columns; the other lanes read the row's first columns, and the MFMA rows
// they feed give output columns that are never stored.
__host__ __device__ constexpr int gqa_lane_cols(int DV) {
  int c = (DV / 16 + 1) & ~1;
  while (DV % c) c += 2;
  return c;
}

// N dwords of a lane's V columns: 8, 16 or 32 bytes as vector loads, other
// sizes as dword arrays (4, 12, 20, 24 or 28 bytes: 4-byte aligned only).
template <int N> struct DwVec {
  uint32_t w[N];
  __device__ __forceinline__ uint32_t operator[](int i) const { return w[i]; }
};
template <int N> struct VVec { typedef DwVec<N> type; };
template <> struct VVec<2> { typedef uint32_t type __attribute__((ext_vector_type(2))); };
template <> struct VVec<4> { typedef u32x4 type; };
template <> struct VVec<8> { typedef uint32_t type __attribute__((ext_vector_type(8))); };

template <class VT> __device__ __forceinline__ VT ld_v(const uint16_t* p) {
  return __builtin_nontemporal_load((const VT*)p);
}
template <class VT, int N = sizeof(VT) / 4>
__device__ __forceinline__ VT ld_dw(const uint16_t* p) {
  VT v;
#pragma unroll
  for (int d = 0; d < N; ++d) v.w[d] = __builtin_nontemporal_load((const uint32_t*)p + d);
  return v;
}
template <class VT> __device__ __forceinline__ VT ld_lane(const uint16_t* p) {
  if constexpr (sizeof(VT) == 8 || sizeof(VT) == 16 || sizeof(VT) == 32) return ld_v<VT>(p);
  else return ld_dw<VT>(p);
}

// Calls f(integral_constant<int, I>) ... f(integral_constant<int, N - 1>).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

struct GqaParams {
  const uint16_t* q;
  const uint16_t* k_pages;
  const uint16_t* v_pages;
  uint16_t* k_pages_w;  // same pools, written by the fused append
  uint16_t* v_pages_w;
  const int32_t* page_table;
  const int32_t* len_in;
  int32_t* len_out;
  const uint16_t* k_new;  // [B][Hkv][1][DK] or nullptr (v_new [B][Hkv][1][DV])
  const uint16_t* v_new;
  float* out;
  float* lse;
  SplitWorkspace ws;
  int B, Hkv, G, page_size, max_pages, num_pages, cap, n_splits;
  float scale_log2;
};

// Block metadata, uniform across the wave.
struct GqaBlock {
  int row;       // kv row
  uint32_t tok;  // pool index of the block's first token: (pid * Hkv + kvh) * page_size + off
  int nt;        // valid tokens (1..32) | kFirst (row's first block) | kLast (row's last
                 // block) | kBadPage (the page table entry was out of range, clamped)
  int nr;        // row of the appended token in this block when in [0, 32)
};
constexpr int kNtMask = 63;
constexpr int kFirst = 64;
constexpr int kLast = 128;
constexpr int kBadPage = 256;

// Key width DK and value width DV, multiples of 16 up to 256.  Lane (n16, j)
// holds C = gqa_lane_cols(DV) value columns of 8 tokens per block, and C
// accumulator tiles.  A key width that is not a multiple of 32 ends with a
// half k-step: its upper 16 columns are zero in both MFMA operands.  G: the
// group size, or 0 to take it from p.G.  (A key or value ring wider than 128
// needs more than the 256 registers of two waves per SIMD; the grid holds one
// workgroup per CU, so one wave per SIMD costs no occupancy the launch would
// use.)
template <int G, int DK, int DV, bool APPEND>
__global__ __launch_bounds__(64 * kGqaWaves, gqa_waves_per_simd(G, DK, DV)) void
gqa_decode_kernel(
    const GqaParams p) {
  static_assert(DK % 16 == 0 && DK <= kGqaMaxD, "key width: a multiple of 16 up to 256");
  static_assert(DV % 16 == 0 && DV <= kGqaMaxD, "value width: a multiple of 16 up to 256");
  constexpr int D = DV;
  constexpr int C = gqa_lane_cols(DV);  // value columns (and accumulator tiles) per lane
  constexpr int LV = DV / C;            // lanes n16 that hold value columns
  using VT = typename VVec<C / 2>::type;
  constexpr int KS = (DK + 31) / 32;    // QK k-steps (32 key columns each)
  constexpr bool KPAD = DK % 32 != 0;   // the last k-step has 16 columns
  // Key column of (k-step s, lane group j); the padding of a half step reads
  // column 0 (its values are zeroed before the MFMA).
  auto kcol = [](int s, int jj) { return (KPAD && s == KS - 1 && jj >= 2) ? 0 : 8 * (4 * s + jj); };
  constexpr int W = kGqaWaves;
  constexpr int NT = 64 * W;
  constexpr int add = APPEND ? 1 : 0;
  __shared__ int s_pref[kMaxSeqs + 1];
  __shared__ int s_len[kMaxSeqs];
  __shared__ int s_wpref[kSeqPlanMax + 1];
  __shared__ int s_scan[W + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int n16 = lane & 15;
  const int j = lane >> 4;
  const int GG = G > 0 ? G : p.G;
  const bool head_ok = n16 < GG;

  // Lengths (len_in clamped to what the page table row holds) and the plan.
  if (APPEND && p.len_out && blockIdx.x == 0)
    for (int b = tid; b < p.B; b += NT) p.len_out[b] = step_len_out(p.len_in, b, add, p.cap);
  const Plan plan =
      plan_build<NT>(p.len_in, add, p.cap, p.B, p.Hkv, p.n_splits, s_pref, s_scan, s_len,
                     s_wpref, uniform(blockIdx.x * W + (tid >> 6)));
  if (blockIdx.x == 0) {  // sequences without tokens: the empty partial (0, -inf),
    for (int b = 0; b < p.B; ++b) {  // or NaN for an invalid length
      if (s_pref[b + 1] != s_pref[b]) continue;
      const bool ok = len_ok(p.len_in[b], add, p.cap);
      const size_t q0 = (size_t)b * p.Hkv * GG;
      for (int idx = tid; idx < p.Hkv * GG * D; idx += NT) p.out[q0 * D + idx] = ok ? 0.f : qnan();
      for (int idx = tid; idx < p.Hkv * GG; idx += NT) p.lse[q0 + idx] = ok ? neg_inf() : qnan();
    }
  }
  const int split = uniform(blockIdx.x * W + (tid >> 6));
  if (!plan.has_work) return;  // no barrier below: waves run independently
  const int x_begin = uniform(plan.begin);  // (the compiler cannot tell on its own)
  const int x_end = uniform(plan.end);
  const int nblk = x_end - x_begin;  // >= 1

  // Metadata window: lane l describes block xb + l (the range's last block
  // past its end).
  int m_row, m_nt, m_nr;
  uint32_t m_tok;
  auto fetch_meta = [&](int xb) __attribute__((always_inline)) {
    const int x = min(xb + lane, x_end - 1);
    int lo = 0, hi = p.B - 1;  // the sequence holding x: last b with s_pref[b] <= x
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_pref[mid] <= x) lo = mid;
      else hi = mid - 1;
    }
    const int len = s_len[lo];
    const int nbb = (len + 31) >> 5;
    const int rel = x - s_pref[lo];
    const int kvh = rel / nbb;
    const int t0 = (rel - kvh * nbb) * 32;
    const int page = t0 / p.page_size;
    const int raw = p.page_table[(size_t)lo * p.max_pages + page];
    const int pid = clamp_page(raw, p.num_pages);
    m_row = lo * p.Hkv + kvh;
    m_tok = ((uint32_t)pid * (uint32_t)p.Hkv + (uint32_t)kvh) * (uint32_t)p.page_size +
            (uint32_t)(t0 - page * p.page_size);
    m_nt = min(32, len - t0) | (t0 == 0 ? kFirst : 0) | (t0 + 32 >= len ? kLast : 0) |
           (raw == pid ? 0 : kBadPage);
    m_nr = APPEND ? len - 1 - t0 : -1;
  };
  auto read_meta = [&](int l) __attribute__((always_inline)) {
    GqaBlock m;
    m.row = __builtin_amdgcn_readlane(m_row, l);
    m.tok = (uint32_t)__builtin_amdgcn_readlane((int)m_tok, l);
    m.nt = __builtin_amdgcn_readlane(m_nt, l);
    m.nr = __builtin_amdgcn_readlane(m_nr, l);
    return m;
  };

  // K/V of one block.  Rows past the valid tokens repeat the last valid one
  // and are masked in the softmax; the appended token's row reads
  // k_new/v_new.  With valid == false (the request past the range's last
  // block) every lane reads the first row of q instead: same instructions
  // and registers, a cache hit, no HBM traffic.
  auto load_block = [&](const GqaBlock& m, bool valid, u32x4 (&ka)[2][KS],
                        VT (&vr)[8]) __attribute__((always_inline)) {
    const uint16_t* kb = valid ? p.k_pages + (size_t)m.tok * DK : p.q;
    const uint16_t* vb = valid ? p.v_pages + (size_t)m.tok * D : p.q;
    const int last = valid ? (m.nt & kNtMask) - 1 : 0;
    const int new_r = (APPEND && valid) ? m.nr : -1;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int r = min(16 * tt + n16, last);
      const uint16_t* kr =
          (APPEND && r == new_r) ? p.k_new + (size_t)m.row * DK : kb + (size_t)r * DK;
#pragma unroll
      for (int s = 0; s < KS; ++s) ka[tt][s] = ld_stream(kr + kcol(s, j));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(pv_token(i, j), last);
      const uint16_t* vrow =
          (APPEND && r == new_r) ? p.v_new + (size_t)m.row * D : vb + (size_t)r * D;
      vr[i] = ld_lane<VT>(vrow + ((LV == 16 || n16 < LV) ? C * n16 : 0));
    }
  };
  // The q rows of kv row `row` as the QK B operand.  Lanes of padding head
  // columns (n16 >= G) load head G - 1: MFMA columns are independent and
  // those columns are never written.
  u32x4 qb[KS];
  auto load_q = [&](int row) __attribute__((always_inline)) {
    const u32x4* qp = (const u32x4*)(p.q + (size_t)(row * GG + min(n16, GG - 1)) * DK);
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = qp[(KPAD && s == KS - 1 && j >= 2) ? 0 : 4 * s + j];
  };

  f32x4 acc[C];
#pragma unroll
  for (int e = 0; e < C; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = neg_inf();
  float l_run = 0.f;

  auto compute_block = [&](const GqaBlock& m, const u32x4 (&ka)[2][KS],
                           const VT (&vr)[8]) __attribute__((always_inline)) {
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (KPAD && s == KS - 1) {  // the half step's upper 16 columns are zero
        const u32x4 z = {0u, 0u, 0u, 0u};
        const bool lo = j < 2;
        const u32x4 qs = lo ? qb[s] : z;
        s0 = mfma16x16x32(lo ? ka[0][s] : z, qs, s0);
        s1 = mfma16x16x32(lo ? ka[1][s] : z, qs, s1);
      } else {
        s0 = mfma16x16x32(ka[0][s], qb[s], s0);
        s1 = mfma16x16x32(ka[1][s], qb[s], s1);
      }
    }
    float alpha;
    bool rescale;
    const u32x4 pb = softmax_block(s0, s1, j, m.nt & kNtMask, p.scale_log2, m_run, l_run,
                                   alpha, rescale);
    pv_block(acc, vr, pb, alpha, rescale);
    // Fused append: the new token's K row sits in lanes n16 == nr % 16 of
    // ka[nr / 16] (16 bytes per (lane, s)), its V row in vr[4 (nr / 16) +
    // nr % 4] of the lanes j == (nr % 16) / 4 (C columns each).
    if (APPEND && m.nr >= 0 && m.nr < 32 && !(m.nt & kBadPage)) {
      const size_t dst = ((size_t)m.tok + m.nr) * D;
      const size_t dst_k = ((size_t)m.tok + m.nr) * DK;
      const int tt = m.nr >> 4;
      if (n16 == (m.nr & 15)) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
          if (t2 == tt) {
#pragma unroll
            for (int s = 0; s < KS; ++s)
              if (!(KPAD && s == KS - 1 && j >= 2))
                *(u32x4*)(p.k_pages_w + dst_k + 8 * (4 * s + j)) = ka[t2][s];
          }
      }
      if (j == ((m.nr & 15) >> 2) && (LV == 16 || n16 < LV)) {
        const int isel = 4 * tt + (m.nr & 3);
        if constexpr (sizeof(VT) == 8 || sizeof(VT) == 16 || sizeof(VT) == 32) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i == isel) ((VT*)(p.v_pages_w + dst))[n16] = vr[i];
        } else {  // dword rows: a select chain per dword (indexing the row array by
                  // isel put it in scratch)
          uint32_t* vd = (uint32_t*)(p.v_pages_w + dst + C * n16);
#pragma unroll
          for (int d = 0; d < C / 2; ++d) {
            uint32_t x = vr[0][d];
#pragma unroll
            for (int i = 1; i < 8; ++i) x = i == isel ? vr[i][d] : x;
            vd[d] = x;
          }
        }
      }
    }
  };

  // Writes the piece of kv row `row` held in (m_run, l_run, acc); `whole`:
  // this wave consumed the row's first and last blocks, so the piece is the
  // row's final partial; `bad`: one of its blocks had a page id outside the
  // pool (read clamped), so the piece is NaN.
  // (The final partial goes to out / lse in fp32, a piece to its workspace
  // slot in bf16.)
  auto flush = [&](int row, bool whole, bool bad) __attribute__((always_inline)) {
    const float l_tot = wave_sum_xor16_32(l_run);
    if (head_ok) {
      const float inv = bad ? qnan() : 1.f / l_tot;
      const float lse_v = bad ? qnan() : (m_run + __log2f(l_tot)) * kLn2;
      // acc[e][i] of lane group j is output column C * (4 j + i) + e; rows
      // 4 j + i >= LV are padding (nothing stored).
      if (whole) {
        float* o = p.out + ((size_t)row * GG + n16) * D + 4 * C * j;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (LV < 16 && 4 * j + i >= LV) continue;
          if constexpr (C % 4 == 0) {
#pragma unroll
            for (int e = 0; e < C; e += 4)
              ((float4*)(o + C * i + e))[0] = make_float4(acc[e][i] * inv, acc[e + 1][i] * inv,
                                                          acc[e + 2][i] * inv, acc[e + 3][i] * inv);
          } else {
#pragma unroll
            for (int e = 0; e < C; e += 2)
              ((float2*)(o + C * i + e))[0] = make_float2(acc[e][i] * inv, acc[e + 1][i] * inv);
          }
        }
        if (j == 0) p.lse[(size_t)row * GG + n16] = lse_v;
      } else {
        const size_t slot = (size_t)(split + row) * GG + n16;
        uint16_t* o = p.ws.part_out + slot * D + 4 * C * j;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (LV < 16 && 4 * j + i >= LV) continue;
          if constexpr (C % 8 == 0) {
#pragma unroll
            for (int e = 0; e < C; e += 8)
              store_piece8(o + C * i + e, acc[e][i] * inv, acc[e + 1][i] * inv,
                           acc[e + 2][i] * inv, acc[e + 3][i] * inv, acc[e + 4][i] * inv,
                           acc[e + 5][i] * inv, acc[e + 6][i] * inv, acc[e + 7][i] * inv);
          } else if constexpr (C == 4) {
            uint2 v;
            v.x = pack_bf16x2(acc[0][i] * inv, acc[1][i] * inv);
            v.y = pack_bf16x2(acc[2][i] * inv, acc[3][i] * inv);
            *(uint2*)(o + C * i) = v;
          } else {
#pragma unroll
            for (int e = 0; e < C; e += 2)
              *(uint32_t*)(o + C * i + e) = pack_bf16x2(acc[e][i] * inv, acc[e + 1][i] * inv);
          }
        }
        if (j == 0) p.ws.part_lse[slot] = lse_v;
      }
    }
  };

  // Ring of S register stages: stage st holds the block k with k % S == st
  // and its metadata mq[st].  Step k requests block k + S - 1 into stage
  // (k + S - 1) % S, then runs block k's math; past the range's end the
  // request is the q-row dummy of load_block.  After block k's math, qb
  // takes the q rows of block k + 1's kv row (an L2 hit, issued every block
  // so that no load in the loop is conditional), ahead of the next block
  // requests, so waiting for it costs nothing extra.  sched_barrier keeps
  // the compiler from sinking the loads below the math (which would
  // serialise them again).  The loop body is a whole turn of the ring with no
  // early exit (the last nblk % S blocks run after it): a path around one
  // step would make the compiler assume that step's loads are still in
  // flight when the ring comes back to it, and wait.
  constexpr int S = gqa_stages(DV);
  int xb = x_begin;
  fetch_meta(xb);
  GqaBlock mq[S];
  u32x4 ka[S][2][KS];
  VT vr[S][8];
  mq[0] = read_meta(0);
  int run_row = mq[0].row;
  bool run_first = (mq[0].nt & kFirst) != 0;  // the running row's first block was ours
  bool run_last = false;                      // ... and its last block (so far)
  bool run_bad = false;                       // a block of the running row had a bad page
  load_q(mq[0].row);
  static_for<0, S - 1>([&](auto i) __attribute__((always_inline)) {
    constexpr int st = decltype(i)::value;
    const bool valid = st < nblk;
    if (st > 0) mq[st] = valid ? read_meta(st) : mq[0];
    load_block(mq[st], valid, ka[st], vr[st]);
  });
  auto step = [&](auto stage, int k) __attribute__((always_inline)) {
    constexpr int st = decltype(stage)::value;
    constexpr int ld = (st + S - 1) % S;  // stage of the block requested now
    constexpr int nx = (st + 1) % S;      // stage of block k + 1
    const bool valid = k + S - 1 < nblk;
    if (valid && x_begin + k + S - 1 - xb == 64) {
      xb += 64;
      fetch_meta(xb);
    }
    if (S > 1) mq[ld] = valid ? read_meta(x_begin + k + S - 1 - xb) : mq[st];
    else mq[0] = read_meta(x_begin + k - xb);  // (one stage: block k itself, always valid)
    load_block(mq[ld], valid, ka[ld], vr[ld]);
    if (S == 1) load_q(mq[0].row);
    __builtin_amdgcn_sched_barrier(0);
    const GqaBlock& cur = mq[st];
    if (cur.row != run_row) {
      flush(run_row, run_first && run_last, run_bad);
      run_row = cur.row;
      run_first = (cur.nt & kFirst) != 0;
      run_bad = false;
      m_run = neg_inf();
      l_run = 0.f;
#pragma unroll
      for (int e = 0; e < C; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    run_last = (cur.nt & kLast) != 0;
    run_bad |= (cur.nt & kBadPage) != 0;
    compute_block(cur, ka[st], vr[st]);
    __builtin_amdgcn_sched_barrier(0);
    // (One stage: block k + 1's row is not known yet; its step requests q
    // right after its block.)
    if (S > 1) load_q(mq[nx].row);
  };
  int base = 0;
  for (; base + S <= nblk; base += S)
    static_for<0, S>([&](auto i) __attribute__((always_inline)) {
      step(i, base + decltype(i)::value);
    });
  static_for<0, S - 1>([&](auto i) __attribute__((always_inline)) {
    if (base + decltype(i)::value < nblk) step(i, base + decltype(i)::value);
  });
  flush(run_row, run_first && run_last, run_bad);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Key / value widths with a kernel: equal multiples of 16 up to 256, and 192
// keys with 128 values (group size 1).
static bool gqa_widths_ok(int Dk, int Dv) {
  if (Dk == kGqaDk192 && Dv == kGqaD) return true;
  return Dk == Dv && Dv >= 16 && Dv <= kGqaMaxD && Dv % 16 == 0;
}

}  // namespace ws

using namespace ws;

// Splits (waves) of a GQA call: n_splits when given, else two per CU (one
// two-wave workgroup), at most what the blocks of the longest possible batch
// can feed with 2 blocks each.  Measured on MI355X at 537 MB per launch: two
// long streams per CU beat four or eight shorter ones (79.7 us against 80.5
// and 84.0), and a third register stage gains nothing.  Small calls (split
// step + merge, r = 1, us per layer): B1 Hkv4 L4096 (516 blocks) 14.4 at 8
// blocks per split (71 splits), 12.5-12.8 at 2 (258); B1 Hkv8 L4096 16.2 ->
// 11.9; B4 Hkv4 L4096 16.3 -> 13.3; one block per split makes the merge's
// rows longer (128 pieces) and was slower again (14.0).  Other widths (B16
// Hkv8 G4 L16384): 64-wide blocks (8 KB per wave) need four waves per CU in
// flight (88 us against 104 at two, 92 at six); the one-stage 256-wide ring
// is fastest at two as well (363 us against 382 at four, 476 at three).
static int gqa_splits(int n_splits, int rows_kv, int max_len, int Dv) {
  if (n_splits > 0) return n_splits;
  const long long max_blocks = (long long)rows_kv * ((max_len + 31) / 32);
  return choose_workgroups(0, Dv <= 64 ? 4 : kGqaSplitsPerCu, max_blocks, 2);
}

static int gqa_launch(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                      uint16_t* k_pages, uint16_t* v_pages, const int32_t* page_table,
                      const int32_t* len_in, int32_t* len_out, int B, int Hq, int Hkv,
                      int Dk, int D, int page_size, int max_pages, int num_pages, int max_len,
                      int n_splits, float scale, float* out, float* lse,
                      void* workspace, size_t workspace_bytes, void* stream,
                      bool combine, const char* name, uint16_t* out_bf16 = nullptr) {
  if (!q || !k_pages || !v_pages || !page_table || !len_in || !out || !lse)
    return set_error(WS_EINVAL, "%s: null pointer", name);
  if (B < 0 || B > kMaxSeqs || Hkv <= 0 || Hq <= 0 || Hq % Hkv)
    return set_error(WS_EINVAL, "%s: bad batch/heads B=%d Hq=%d Hkv=%d (B <= %d)", name,
                     B, Hq, Hkv, kMaxSeqs);
  const int G = Hq / Hkv;
  if (G < 1 || G > 16)
    return set_error(WS_EINVAL, "%s: group size %d unsupported (1 to 16)", name, G);
  if (!gqa_widths_ok(Dk, D))
    return set_error(WS_EINVAL,
                     "%s: head_dim Dk=%d Dv=%d unsupported (equal multiples of 16 up to 256, "
                     "192/128)",
                     name, Dk, D);
  if (Dk == kGqaDk192 && D == kGqaD && G != 1)
    return set_error(WS_EINVAL, "%s: Dk=192 takes group size 1 (got %d)", name, G);
  if (page_size <= 0 || max_pages <= 0 || num_pages <= 0 || max_len < 0 ||
      (page_size % 32 && max_pages != 1) ||
      (long long)max_len > (long long)page_size * max_pages)
    return set_error(WS_EINVAL,
                     "%s: bad paging page_size=%d max_pages=%d num_pages=%d max_len=%d "
                     "(page_size must be a multiple of 32 unless max_pages == 1)",
                     name, page_size, max_pages, num_pages, max_len);
  if ((long long)num_pages * Hkv * page_size > 0xffffffffLL)
    return set_error(WS_EINVAL, "%s: pools of %lld tokens exceed the 32-bit token index", name,
                     (long long)num_pages * Hkv * page_size);
  if (n_splits < 0) return set_error(WS_EINVAL, "%s: n_splits %d < 0", name, n_splits);
  if (!aligned16(q) || !aligned16(k_pages) || !aligned16(v_pages) || !aligned16(out) ||
      (k_new && (!aligned16(k_new) || !aligned16(v_new))))
    return set_error(WS_EINVAL, "%s: buffers must be 16-byte aligned", name);
  if (k_new && !v_new) return set_error(WS_EINVAL, "%s: v_new is null", name);
  if (len_out && len_out == len_in)
    return set_error(WS_EINVAL, "%s: len_out must not alias len_in", name);
  if (B == 0) return WS_OK;
  if ((long long)B * Hkv * ((max_len + 32) / 32) * 4096 >= (1LL << 31))
    return set_error(WS_EINVAL, "%s: %lld kv rows of %d tokens exceed the block index range",
                     name, (long long)B * Hkv, max_len);
  const int rows_kv = B * Hkv;
  const int n = gqa_splits(n_splits, rows_kv, max_len, D);
  if (n > kReduceMaxWeights)
    return set_error(WS_EINVAL, "%s: %d splits exceed the merge's %d", name, n,
                     kReduceMaxWeights);
  const size_t need = ws::workspace_bytes(rows_kv, G, D, n);
  if (!workspace || workspace_bytes < need)
    return set_error(WS_EWORKSPACE, "%s: workspace %zu < %zu bytes", name, workspace_bytes,
                     need);
  if (((uintptr_t)workspace & 255u) != 0)
    return set_error(WS_EINVAL, "%s: workspace must be 256-byte aligned", name);
  GqaParams prm;
  prm.q = q;
  prm.k_pages = k_pages;
  prm.v_pages = v_pages;
  prm.k_pages_w = k_pages;
  prm.v_pages_w = v_pages;
  prm.page_table = page_table;
  prm.len_in = len_in;
  prm.len_out = len_out;
  prm.k_new = k_new;
  prm.v_new = v_new;
  prm.out = out;
  prm.lse = lse;
  prm.ws = carve_workspace(workspace, rows_kv, G, n);
  prm.B = B;
  prm.Hkv = Hkv;
  prm.G = G;
  prm.page_size = page_size;
  prm.max_pages = max_pages;
  prm.num_pages = num_pages;
  prm.cap = (int)std::min<long long>((long long)page_size * max_pages, 1LL << 30);
  prm.scale_log2 = scale * kLog2e;
  prm.n_splits = n;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((n + kGqaWaves - 1) / kGqaWaves), block(64 * kGqaWaves);
#define WS_GQA_LAUNCH(GG, DKK, DVV)                                                         \
  if (k_new)                                                                                \
    hipLaunchKernelGGL((gqa_decode_kernel<GG, DKK, DVV, true>), grid, block, 0, s, prm);    \
  else                                                                                      \
    hipLaunchKernelGGL((gqa_decode_kernel<GG, DKK, DVV, false>), grid, block, 0, s, prm);
#define WS_GQA_CASE(GG, DKK, DVV) \
  case GG:                        \
    WS_GQA_LAUNCH(GG, DKK, DVV)   \
    break;
#define WS_GQA_GROUPS(DD)        \
  switch (G) {                   \
    WS_GQA_CASE(1, DD, DD)       \
    WS_GQA_CASE(2, DD, DD)       \
    WS_GQA_CASE(4, DD, DD)       \
    WS_GQA_CASE(8, DD, DD)       \
    WS_GQA_CASE(16, DD, DD)      \
    default:                     \
      WS_GQA_LAUNCH(0, DD, DD)   \
      break;                     \
  }
  // 64, 128 and 256 (and the ds2 pair) are instantiated per power-of-two
  // group size; other group sizes and the other widths take it at run time
  // (prm.G).
#define WS_GQA_ANY(DD)        \
  case DD:                    \
    WS_GQA_LAUNCH(0, DD, DD)  \
    break;
  if (Dk == kGqaDk192 && D == kGqaD) {
    switch (G) { WS_GQA_CASE(1, kGqaDk192, kGqaD) }
  } else if (D == 64) {
    WS_GQA_GROUPS(64)
  } else if (D == kGqaMaxD) {
    WS_GQA_GROUPS(kGqaMaxD)
  } else if (D == kGqaD) {
    WS_GQA_GROUPS(kGqaD)
  } else {
    switch (D) {
      WS_GQA_ANY(16) WS_GQA_ANY(32) WS_GQA_ANY(48) WS_GQA_ANY(80) WS_GQA_ANY(96)
      WS_GQA_ANY(112) WS_GQA_ANY(144) WS_GQA_ANY(160) WS_GQA_ANY(176) WS_GQA_ANY(192)
      WS_GQA_ANY(208) WS_GQA_ANY(224) WS_GQA_ANY(240)
    }
  }
#undef WS_GQA_ANY
#undef WS_GQA_GROUPS
#undef WS_GQA_CASE
#undef WS_GQA_LAUNCH
  int rc = check_launch(name);
  if (rc != WS_OK || !combine) return rc;
  // One-launch entry points: the rows held by several waves are combined by
  // the split merge on the same stream, in place (each element is read and
  // written by the same thread; the merge workgroups of a row's column chunks
  // all write its unchanged lse when one wave held it).
  rc = merge_split_pieces(len_in, k_new ? 1 : 0, B, Hkv, G, D, prm.cap, n, out, lse, prm.ws,
                          out, lse, out_bf16, s);
  return rc != WS_OK ? rc : check_launch(name);
}

extern "C" int ws_decode_plan(int kind, int rows_kv, int heads, int max_len,
                              int n_workgroups, int* n_workgroups_out,
                              size_t* workspace_bytes_out) {
  if ((kind != 0 && kind != 1) || rows_kv < 0 || max_len < 0 || n_workgroups < 0 ||
      heads <= 0 || (kind == 0 && heads > 16) || (kind == 1 && heads % 16))
    return set_error(WS_EINVAL, "ws_decode_plan: bad arguments");
  int n;
  size_t bytes;
  if (kind == 0) {
    n = gqa_splits(n_workgroups, rows_kv, max_len, kGqaD);
    bytes = ws::workspace_bytes(rows_kv, heads, kGqaD, n);
  } else {  // one plan sequence per (sequence, 16-head group), or per sequence (wide)
    const MlaLayout lay = mla_layout(rows_kv, heads);
    n = mla_workgroups(n_workgroups, lay.plan_seqs, max_len);
    bytes = ws::workspace_bytes(lay.plan_seqs, lay.piece_heads, 512, n);
  }
  if (n_workgroups_out) *n_workgroups_out = n;
  if (workspace_bytes_out) *workspace_bytes_out = bytes;
  return WS_OK;
}

extern "C" int ws_attn_decode_plan(int rows_kv, int heads, int Dk, int Dv, int max_len,
                                   int n_splits, int* n_splits_out,
                                   size_t* workspace_bytes_out) {
  if (!gqa_widths_ok(Dk, Dv))
    return set_error(WS_EINVAL,
                     "ws_attn_decode_plan: head_dim Dk=%d Dv=%d unsupported (equal multiples "
                     "of 16 up to 256, 192/128)", Dk, Dv);
  if (rows_kv < 0 || max_len < 0 || n_splits < 0 || heads <= 0 || heads > 16)
    return set_error(WS_EINVAL, "ws_attn_decode_plan: bad arguments");
  if (Dk == kGqaDk192 && Dv == kGqaD && heads != 1)
    return set_error(WS_EINVAL, "ws_attn_decode_plan: Dk=192 takes group size 1 (got %d)",
                     heads);
  const int n = gqa_splits(n_splits, rows_kv, max_len, Dv);
  if (n_splits_out) *n_splits_out = n;
  if (workspace_bytes_out) *workspace_bytes_out = ws::workspace_bytes(rows_kv, heads, Dv, n);
  return WS_OK;
}

extern "C" int ws_gqa_decode_partial(
    const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
    const int32_t* page_table, const int32_t* gpu_len, int B, int Hq, int Hkv, int D,
    int page_size, int max_pages, int num_pages, int max_len, int n_workgroups,
    float scale, float* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  return gqa_launch(q, nullptr, nullptr, (uint16_t*)k_pages, (uint16_t*)v_pages,
                    page_table, gpu_len, nullptr, B, Hq, Hkv, D, D, page_size, max_pages,
                    num_pages, max_len, n_workgroups, scale, out, lse, workspace,
                    workspace_bytes, stream, true, "ws_gqa_decode_partial");
}

extern "C" int ws_gqa_append_decode_partial(
    const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_pages,
    uint16_t* v_pages, const int32_t* page_table, const int32_t* len_in,
    int32_t* len_out, int B, int Hq, int Hkv, int D, int page_size, int max_pages,
    int num_pages, int max_len, int n_workgroups, float scale, float* out,
    float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  if (!k_new)
    return set_error(WS_EINVAL, "ws_gqa_append_decode_partial: k_new is null");
  return gqa_launch(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out, B,
                    Hq, Hkv, D, D, page_size, max_pages, num_pages, max_len, n_workgroups,
                    scale, out, lse, workspace, workspace_bytes, stream, true,
                    "ws_gqa_append_decode_partial");
}

extern "C" int ws_gqa_append_decode_split(
    const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_pages,
    uint16_t* v_pages, const int32_t* page_table, const int32_t* len_in,
    int32_t* len_out, int B, int Hq, int Hkv, int D, int page_size, int max_pages,
    int num_pages, int max_len, int n_workgroups, float scale, float* out,
    float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  if (!k_new)
    return set_error(WS_EINVAL, "ws_gqa_append_decode_split: k_new is null");
  return gqa_launch(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out, B,
                    Hq, Hkv, D, D, page_size, max_pages, num_pages, max_len, n_workgroups,
                    scale, out, lse, workspace, workspace_bytes, stream, false,
                    "ws_gqa_append_decode_split");
}

extern "C" int ws_attn_decode_partial(
    const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
    const int32_t* page_table, const int32_t* gpu_len, int B, int Hq, int Hkv, int Dk, int Dv,
    int page_size, int max_pages, int num_pages, int max_len, int n_splits, float scale,
    float* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return gqa_launch(q, nullptr, nullptr, (uint16_t*)k_pages, (uint16_t*)v_pages,
                    page_table, gpu_len, nullptr, B, Hq, Hkv, Dk, Dv, page_size, max_pages,
                    num_pages, max_len, n_splits, scale, out, lse, workspace,
                    workspace_bytes, stream, true, "ws_attn_decode_partial");
}

extern "C" int ws_attn_append_decode_partial(
    const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_pages,
    uint16_t* v_pages, const int32_t* page_table, const int32_t* len_in, int32_t* len_out,
    int B, int Hq, int Hkv, int Dk, int Dv, int page_size, int max_pages, int num_pages,
    int max_len, int n_splits, float scale, float* out, float* lse, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (!k_new)
    return set_error(WS_EINVAL, "ws_attn_append_decode_partial: k_new is null");
  return gqa_launch(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out, B,
                    Hq, Hkv, Dk, Dv, page_size, max_pages, num_pages, max_len, n_splits,
                    scale, out, lse, workspace, workspace_bytes, stream, true,
                    "ws_attn_append_decode_partial");
}

extern "C" int ws_gqa_append_decode_full(
    const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_pages,
    uint16_t* v_pages, const int32_t* page_table, const int32_t* len_in, int32_t* len_out,
    int B, int Hq, int Hkv, int D, int page_size, int max_pages, int num_pages, int max_len,
    int n_splits, float scale, uint16_t* out_bf16, float* out, float* lse, void* workspace,
    size_t workspace_bytes, void* stream) {
  static const char* name = "ws_gqa_append_decode_full";
  if (!k_new) return set_error(WS_EINVAL, "%s: k_new is null", name);
  if (!out_bf16) return set_error(WS_EINVAL, "%s: out_bf16 is null", name);
  if (((uintptr_t)out_bf16 & 15u) != 0)
    return set_error(WS_EINVAL, "%s: buffers must be 16-byte aligned", name);
  return gqa_launch(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out, B, Hq,
                    Hkv, D, D, page_size, max_pages, num_pages, max_len, n_splits, scale, out,
                    lse, workspace, workspace_bytes, stream, true, name, out_bf16);
}
