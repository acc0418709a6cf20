// Load-balanced work plan of the decode kernels, computed on the device.
//
// The work of a call is the list of 32-token blocks of every row (GQA row =
// (sequence, kv head), MLA row = sequence), rows in order.  With
// nb(b) = ceil(len_b / 32) blocks per row of sequence b and R rows per
// sequence, T = sum_b R * nb(b).  A grid of n workgroups gives workgroup g
// the blocks [floor(g T / n), floor((g + 1) T / n)), so every workgroup
// streams the same amount of KV whatever the lengths (n is capped at T, so
// no range is empty).  A workgroup walks its range as row segments; a row
// covered by several workgroups gets one partial per workgroup, stored in
// slot g + row: along the block order both g and row are non-decreasing, so
// g + row is distinct for every (workgroup, row) pair and slots stay below
// n + rows.
#pragma once

#include "ws_common.h"

namespace ws {

// Most sequences a call takes (the per-sequence prefix lives in LDS).
constexpr int kMaxSeqs = 2048;

struct Plan {
  int T;  // total blocks (the host keeps it below 2^31 / grid)
  int n;  // workgroups with work (min(grid, T)), at most 4096
  int q, r;  // T = q n + r
  bool seq;  // sequence-aligned ranges (plan_build with s_wpref)
  // The calling split's range [begin, end) (when it passed its index g),
  // and the sequence of block `begin` (-1: not known, use plan_seq).
  bool has_work;
  int begin, end, b0;
};

// Wave-wide inclusive prefix sum from the ROCm device library (ockl), a
// DPP sequence: every lane of the wave must be active.
extern "C" __device__ int __ockl_wfscan_add_i32(int, bool);

// Most sequences the sequence-aligned plan takes (one per lane).
constexpr int kSeqPlanMax = 64;
// Blocks per split the sequence-aligned plan may add over ceil(T / n) and
// still be chosen: a split whose range enters a second sequence restarts
// its load stream there, which costs the MLA step about four blocks' time.
constexpr int kAlignSlack = 3;

// Workgroup-uniform value moved to a scalar register.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// A length the call can serve: 0 <= l <= cap - add (room for the appended
// token when add == 1).  A length outside that range (a caller's mistake, or
// the -1 a fused step leaves after one) is not clamped: the sequence gets no
// blocks, its outputs are NaN and a fused step writes len_out = -1.
__device__ __forceinline__ bool len_ok(int l, int add, int cap) {
  return l >= 0 && l <= cap - add;
}

// Sequence length used by the kernels: len_in[b] + add (1 when the call
// appends the step's new token), or 0 for a length outside the valid range.
__device__ __forceinline__ int plan_len(const int32_t* len_in, int b, int add, int cap) {
  const int l = len_in[b];
  return len_ok(l, add, cap) ? l + add : 0;
}

// Length slot of plan sequence v.  A call whose sequences carry ng groups
// of 16 query heads over one shared latent (absorbed MLA with H = 16 ng)
// plans over v = b ng + group: each group is its own plan sequence with
// sequence b's length.
__device__ __forceinline__ int seq_of(int v, int ng) { return ng == 1 ? v : v / ng; }

// len_out of a fused step: the new length, or -1 for an invalid len_in.
__device__ __forceinline__ int step_len_out(const int32_t* len_in, int b, int add, int cap) {
  const int l = len_in[b];
  return len_ok(l, add, cap) ? l + add : -1;
}

__device__ __forceinline__ Plan plan_of(int T, int grid) {
  Plan p;
  p.T = T;
  p.n = min(grid, T);
  p.q = p.n > 0 ? (int)((unsigned)T / (unsigned)p.n) : 0;
  p.r = T - p.q * p.n;
  p.seq = false;
  p.has_work = false;
  p.begin = p.end = 0;
  p.b0 = -1;
  return p;
}

// floor(g T / n) as g q + floor(g r / n): 32-bit products (g r < n^2 <= 2^24)
// and one 32-bit division, for 0 <= g <= n.
__device__ __forceinline__ int plan_start(const Plan& p, int g) {
  return g * p.q + (int)((unsigned)(g * p.r) / (unsigned)p.n);
}

// Builds s_pref[0..B] (exclusive prefix of blocks per sequence, R rows each)
// with the NT threads of the workgroup and returns the plan; with s_len, also
// the lengths s_len[0..B) (plan_len), so callers need not read len_in again.
// s_scan holds NT / 64 + 1 ints.  Every thread must call it.  With at most
// 64 sequences every wave builds the whole plan by itself (lane b: sequence
// b) and writes the same values, reading back only what it wrote: no barrier
// between the kernel start and its first loads.  Otherwise the workgroup
// builds it together, behind barriers.
//
// With s_wpref (kSeqPlanMax + 1 ints), one row per sequence (R == 1) and 2
// to 64 sequences, the plan may instead be sequence-aligned: sequence b gets
// n_b = ceil(nb(b) / M) splits, M the smallest block count per split with
// sum_b n_b <= n, which take equal shares of its blocks, so no split spans
// two sequences.  It is chosen when M <= ceil(T / n) + kAlignSlack (seq set,
// s_wpref[b] = first split of sequence b, s_wpref[B] = splits used).  Every
// kernel of a call (step and merge) passes the same arguments and so makes
// the same choice.
//
// A split that passes its index g >= 0 gets its range in has_work / begin /
// end (and, with at most 64 sequences, the sequence of its first block in
// b0), computed from registers.
//
// ng > 1: B counts plan sequences v = b ng + group, whose lengths are
// len_in[v / ng] (seq_of).
template <int NT>
__device__ Plan plan_build(const int32_t* len_in, int add, int cap, int B, int R,
                           int grid, int* s_pref, int* s_scan, int* s_len = nullptr,
                           int* s_wpref = nullptr, int g = -1, int ng = 1) {
  constexpr int NW = NT / 64;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  if (B >= 1 && B <= 64) {
    const int l = lane < B ? plan_len(len_in, seq_of(lane, ng), add, cap) : 0;
    const int nb = R * ((l + 31) >> 5);
    const int incl = __ockl_wfscan_add_i32(nb, true);
    if (lane < B) {
      s_pref[lane] = incl - nb;
      if (s_len) s_len[lane] = l;
    }
    const int T = __builtin_amdgcn_readlane(incl, B - 1);
    if (lane == 0) s_pref[B] = T;
    Plan p = plan_of(T, grid);
    if (s_wpref && R == 1 && B >= 2 && p.n > 0) {
      // splits needed with M = base + c blocks per split, c = 0..3, summed
      // over the wave as four 16-bit counts (each at most n + 64)
      const int base = (T + p.n - 1) / p.n;
      uint32_t c01 = 0, c23 = 0;
      if (nb > 0) {
        const uint32_t u = (uint32_t)nb;
        c01 = (u + base - 1) / base | ((u + base) / (base + 1)) << 16;
        c23 = (u + base + 1) / (base + 2) | ((u + base + 2) / (base + 3)) << 16;
      }
      c01 = __ockl_wfred_add_u32(c01);
      c23 = __ockl_wfred_add_u32(c23);
      const int cnt[4] = {(int)(c01 & 0xffffu), (int)(c01 >> 16), (int)(c23 & 0xffffu),
                          (int)(c23 >> 16)};
      int M = 0;
#pragma unroll
      for (int c = kAlignSlack; c >= 0; --c)
        if (uniform(cnt[c]) <= p.n) M = base + c;
      if (M > 0) {
        const int ns = nb > 0 ? (nb + M - 1) / M : 0;
        const int w = __ockl_wfscan_add_i32(ns, true);
        const int used = __builtin_amdgcn_readlane(w, B - 1);
        if (lane < B) s_wpref[lane] = w - ns;
        if (lane == 0) s_wpref[B] = used;
        p.seq = true;
        if (g >= 0 && g < used) {
          // split g: sequence b (the first with w > g), its j-th of ns splits
          const int b = __builtin_ctzll(__builtin_amdgcn_ballot_w64(lane < B && w > g));
          const int j = g - (__builtin_amdgcn_readlane(w, b) - __builtin_amdgcn_readlane(ns, b));
          const int nsb = __builtin_amdgcn_readlane(ns, b);
          const int first = __builtin_amdgcn_readlane(incl, b) - __builtin_amdgcn_readlane(nb, b);
          const int nbb = __builtin_amdgcn_readlane(nb, b);
          p.has_work = true;
          p.begin = first + j * nbb / nsb;
          p.end = first + (j + 1) * nbb / nsb;
          p.b0 = b;
        }
        return p;
      }
    }
    if (g >= 0 && g < p.n) {
      p.has_work = true;
      p.begin = plan_start(p, g);
      p.end = plan_start(p, g + 1);
      p.b0 = __builtin_ctzll(__builtin_amdgcn_ballot_w64(lane < B && incl > p.begin));
    }
    return p;
  }
  const int chunk = (B + NT - 1) / NT;
  const int b0 = min(B, t * chunk);
  const int b1 = min(B, b0 + chunk);
  int local = 0;
  for (int b = b0; b < b1; ++b) {
    const int l = plan_len(len_in, seq_of(b, ng), add, cap);
    if (s_len) s_len[b] = l;
    local += R * ((l + 31) >> 5);
  }
  // inclusive scan of `local` across the wave
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_scan[wave] = incl;
  __syncthreads();
  if (t == 0) {
    int run = 0;
    for (int w = 0; w < NW; ++w) {
      const int v = s_scan[w];
      s_scan[w] = run;
      run += v;
    }
    s_scan[NW] = run;
  }
  __syncthreads();
  int run = s_scan[wave] + incl - local;
  for (int b = b0; b < b1; ++b) {
    s_pref[b] = run;
    run += R * (((s_len ? s_len[b] : plan_len(len_in, seq_of(b, ng), add, cap)) + 31) >> 5);
  }
  if (t == 0) s_pref[B] = s_scan[NW];
  __syncthreads();
  Plan p = plan_of(uniform(s_scan[NW]), grid);
  if (g >= 0 && g < p.n) {
    p.has_work = true;
    p.begin = plan_start(p, g);
    p.end = plan_start(p, g + 1);
  }
  return p;
}


// Workgroup whose range holds block blk: ceil((blk + 1) n / T) - 1.  The
// double quotient is exact enough: the operands are integers below 2^53, and
// a quotient that is not an integer lies at least 1 / T > 2^-31 below the
// next one, far above the rounding error of a quotient of at most 4096.
__device__ __forceinline__ int plan_owner(const Plan& p, int blk) {
  return (int)ceil((double)(blk + 1) * (double)p.n / (double)p.T) - 1;
}

// Splits holding row `row` (sequence b under a sequence-aligned plan, whose
// rows are sequences), blocks [row_start, row_start + nbb), nbb >= 1: the
// first split and how many.
__device__ __forceinline__ void plan_row_splits(const Plan& p, int b, int row_start, int nbb,
                                                const int* s_wpref, int& w_first, int& nseg) {
  if (p.seq) {
    w_first = s_wpref[b];
    nseg = s_wpref[b + 1] - s_wpref[b];
  } else {
    w_first = plan_owner(p, row_start);
    nseg = plan_owner(p, row_start + nbb - 1) - w_first + 1;
  }
}

// Sequence holding block blk: the last b with s_pref[b] <= blk (B >= 1).
__device__ __forceinline__ int plan_seq(const int* s_pref, int B, int blk) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (uniform(s_pref[mid]) <= blk) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

}  // namespace ws
