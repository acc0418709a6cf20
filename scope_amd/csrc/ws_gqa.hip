// Split-KV GQA decode attention over the HBM partition (gfx950), optionally
// fused with the append of the decode step's new token.
//
// Work decomposition (ws_plan.h): the grid's workgroups (4 waves each) take
// equal shares of all 32-token blocks of all kv rows (kv row = b * Hkv + kvh),
// so a batch of ragged lengths keeps every workgroup streaming for the same
// time.  A workgroup walks its share as row segments; inside a segment its
// waves take blocks round robin, each wave requesting its next block's K/V
// before the MFMAs of the current one run, and the waves combine their
// (max, sum, out) in LDS at the segment's end.  A row held by one workgroup
// is written final; otherwise each workgroup stores a partial and the last to
// arrive combines them (ws_reduce.h), so one launch produces the partition's
// final partial.
//
// With k_new != nullptr the call also appends one token per sequence: token
// len_in[b] of sequence b is read from k_new/v_new instead of the page, the
// workgroup whose segment holds that position writes it into its page slot,
// and len_out[b] = len_in[b] + 1.  No workgroup reads the slot being written
// and len_out is not read, so the fused step has no intra-launch race.
#include <math.h>

#include <algorithm>

#include "ws_attn.h"
#include "ws_plan.h"
#include "ws_reduce.h"

namespace ws {

constexpr int kGqaD = 128;
constexpr int kGqaWaves = 4;
// Register stages per wave.  Two keep two waves per SIMD (about 230 VGPRs);
// measured on MI355X, deeper rings at one wave per SIMD stream no faster.
constexpr int kGqaStages = 2;

struct GqaParams {
  const uint16_t* q;
  const uint16_t* k_pages;
  const uint16_t* v_pages;
  uint16_t* k_pages_w;  // same pools, written by the fused append
  uint16_t* v_pages_w;
  const int32_t* page_table;
  const int32_t* len_in;
  int32_t* len_out;
  const uint16_t* k_new;  // [B][Hkv][1][D] or nullptr
  const uint16_t* v_new;
  float* out;
  float* lse;
  SplitWorkspace ws;
  int B, Hkv, page_size, max_pages, num_pages, cap;
  float scale_log2;
};

// COMBINE: rows held by several workgroups are combined in this launch by the
// last one to arrive; without it their partials stay in the workspace for
// ws_merge_split (the combine then rides on the merge launch of the step).
template <int G, bool APPEND, bool COMBINE>
__global__ __launch_bounds__(64 * kGqaWaves, kGqaStages <= 2 ? 2 : 1) void gqa_decode_kernel(
    const GqaParams p) {
  constexpr int D = kGqaD;
  constexpr int W = kGqaWaves;
  constexpr int S = kGqaStages;
  constexpr int NT = 64 * W;
  constexpr int add = APPEND ? 1 : 0;
  __shared__ float s_m[W][16];
  __shared__ float s_l[W][16];
  __shared__ float s_acc[W][G][D];
  __shared__ float s_w[kReduceMaxWeights];
  __shared__ float s_red[32 * W + 32];
  __shared__ int s_pref[kMaxSeqs + 1];
  __shared__ int s_scan[W + 1];
  __shared__ int s_flag;

  const int g = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n16 = lane & 15;
  const int j = lane >> 4;
  const bool head_ok = n16 < G;

  // Lengths (len_in clamped to what the page table row holds) and the plan.
  if (APPEND && p.len_out && g == 0)
    for (int b = tid; b < p.B; b += NT) p.len_out[b] = plan_len(p.len_in, b, add, p.cap);
  const Plan plan = plan_build<NT>(p.len_in, add, p.cap, p.B, p.Hkv, gridDim.x, s_pref, s_scan);
  if (g == 0) {  // sequences without tokens: the empty partial (0, -inf)
    for (int b = 0; b < p.B; ++b) {
      if (s_pref[b + 1] != s_pref[b]) continue;
      const size_t q0 = (size_t)b * p.Hkv * G;
      for (int idx = tid; idx < p.Hkv * G * D; idx += NT) p.out[q0 * D + idx] = 0.f;
      for (int idx = tid; idx < p.Hkv * G; idx += NT) p.lse[q0 + idx] = neg_inf();
    }
  }
  if (g >= plan.n) return;
  const int blk_end = plan_start(plan, g + 1);
  int blk = plan_start(plan, g);

  while (blk < blk_end) {
    // the row segment holding blk (all workgroup-uniform)
    const int b = plan_seq(s_pref, p.B, blk);
    const int len = uniform(plan_len(p.len_in, b, add, p.cap));
    const int len_old = len - add;
    const int nbb = (len + 31) >> 5;
    const int seq_start = uniform(s_pref[b]);
    const int kvh = (blk - seq_start) / nbb;
    const int row = b * p.Hkv + kvh;
    const int row_start = seq_start + kvh * nbb;
    const int row_end = row_start + nbb;
    const int seg_end = min(blk_end, row_end);
    const int t_begin = (blk - row_start) * 32;
    const int t_end = min(len, (seg_end - row_start) * 32);
    const int q0 = row * G;
    const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
    const size_t new_row = (size_t)row * D;

    // Fused append: write the new token into its page slot.
    if (APPEND && wave == 0 && lane < 32 && len_old >= t_begin && len_old < t_end) {
      const int page = len_old / p.page_size;
      const int pid = pt[page];
      if (pid >= 0 && pid < p.num_pages) {
        const size_t dst =
            (((size_t)pid * p.Hkv + kvh) * p.page_size + (len_old - page * p.page_size)) * D;
        if (lane < 16)
          ((u32x4*)(p.k_pages_w + dst))[lane] = ((const u32x4*)(p.k_new + new_row))[lane];
        else
          ((u32x4*)(p.v_pages_w + dst))[lane - 16] =
              ((const u32x4*)(p.v_new + new_row))[lane - 16];
      }
    }

    u32x4 qb[4];
    if (head_ok) {
      const u32x4* qp = (const u32x4*)(p.q + (size_t)(q0 + n16) * D);
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

    // K/V of a 32-token block starting at t0 (a multiple of 32, so the block
    // lies in one page).  Rows past t_end repeat the last valid token and are
    // masked in the softmax.  With valid == false (the prefetch past a wave's
    // last block) every lane reads the first row of q instead: same
    // instructions and registers, a cache hit, no HBM traffic.
    // Physical page of the block at t0 (a scalar load; the ring below issues
    // it one block ahead, so its latency is not on the block's load path).
    auto page_id = [&](int t0) { return clamp_page(pt[t0 / p.page_size], p.num_pages); };
    auto load_block = [&](int t0, int pid, bool valid, u32x4 (&ka)[2][4], u32x4 (&vr)[8]) {
      const int page = t0 / p.page_size;
      const size_t tok0 =
          ((size_t)pid * p.Hkv + kvh) * p.page_size + (t0 - page * p.page_size);
      const uint16_t* kb = valid ? p.k_pages + tok0 * D : p.q;
      const uint16_t* vb = valid ? p.v_pages + tok0 * D : p.q;
      const int last = valid ? min(32, t_end - t0) - 1 : 0;
      const int new_r = (APPEND && valid) ? len_old - t0 : -1;  // block row of the new token
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int r = min(16 * tt + n16, last);
        const uint16_t* kr = (APPEND && r == new_r) ? p.k_new + new_row : kb + (size_t)r * D;
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[tt][s] = ld_stream(kr + 8 * (4 * s + j));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = min(pv_token(i, j), last);
        const uint16_t* vrow =
            (APPEND && r == new_r) ? p.v_new + new_row : vb + (size_t)r * D;
        vr[i] = ld_stream(vrow + 8 * n16);
      }
    };
    auto compute_block = [&](int t0, const u32x4 (&ka)[2][4], const u32x4 (&vr)[8]) {
      const int nt = min(32, t_end - t0);
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        s0 = mfma16x16x32(ka[0][s], qb[s], s0);
        s1 = mfma16x16x32(ka[1][s], qb[s], s1);
      }
      float alpha;
      const u32x4 pb = softmax_block(s0, s1, j, nt, p.scale_log2, m_run, l_run, alpha);
      pv_block(acc, vr, pb, alpha);
    };

    // Blocks of this wave: t_begin + 32 * (wave + W * i), i < nblk, through a
    // ring of S register stages: while block i is consumed, blocks
    // i + 1 .. i + S - 1 are in flight (past the last block the request is the
    // q-row dummy of load_block).  sched_barrier keeps the compiler from
    // sinking the loads below the math (which would serialise them again).
    const int first = t_begin + 32 * wave;
    const int nblk = first < t_end ? (t_end - first + 32 * W - 1) / (32 * W) : 0;
    if (nblk > 0) {
      auto tblk = [&](int k) { return first + 32 * W * min(k, nblk - 1); };
      u32x4 ka[S][2][4], vr[S][8];
#pragma unroll
      for (int st = 0; st < S - 1; ++st)
        load_block(tblk(st), page_id(tblk(st)), st < nblk, ka[st], vr[st]);
      int pid_next = page_id(tblk(S - 1));
      for (int i = 0; i < nblk; i += S) {
#pragma unroll
        for (int st = 0; st < S; ++st) {
          const int blk = i + st;
          if (blk >= nblk) break;
          const int nxt = blk + S - 1;
          load_block(tblk(nxt), pid_next, nxt < nblk, ka[(st + S - 1) % S],
                     vr[(st + S - 1) % S]);
          pid_next = page_id(tblk(nxt + 1));
          __builtin_amdgcn_sched_barrier(0);
          compute_block(first + 32 * W * blk, ka[st], vr[st]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }

    // Combine the waves: per head column, M = max m_w, L = sum l_w 2^(m_w - M).
    const float l_tot = wave_sum_xor16_32(l_run);
    __syncthreads();  // the previous segment is done with the LDS
    if (head_ok) {
      if (j == 0) {
        s_m[wave][n16] = m_run;
        s_l[wave][n16] = l_tot;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_acc[wave][n16][acc_col(j, i, e)] = acc[e][i];
    }
    __syncthreads();
    const int w_first = plan_owner(plan, row_start);
    const int nseg = plan_owner(plan, row_end - 1) - w_first + 1;
    const bool final_write = nseg == 1;
    float* dst_out = final_write ? p.out + (size_t)q0 * D
                                 : p.ws.part_out + (size_t)(g + row) * G * D;
    float* dst_lse = final_write ? p.lse + q0 : p.ws.part_lse + (size_t)(g + row) * G;
    for (int idx = tid; idx < G * D; idx += NT) {
      const int h = idx / D;
      const int d = idx - h * D;
      float M = neg_inf();
#pragma unroll
      for (int w = 0; w < W; ++w) M = fmaxf(M, s_m[w][h]);
      float L = 0.f, o = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float sc = __builtin_amdgcn_exp2f(s_m[w][h] - M);
        L += s_l[w][h] * sc;
        o += s_acc[w][h][d] * sc;
      }
      const float ov = o / L;
      const float lv = (M + __log2f(L)) * kLn2;
      if (final_write || !COMBINE) {
        dst_out[idx] = ov;
        if (d == 0) dst_lse[h] = lv;
      } else {  // read by the row's last workgroup, maybe on another XCD
        st_agent(dst_out + idx, ov);
        if (d == 0) st_agent(dst_lse + h, lv);
      }
    }
    if (COMBINE && !final_write && arrive_last(p.ws.counters + row, nseg, &s_flag)) {
      reduce_rows<NT>(p.ws.part_out + (size_t)(w_first + row) * G * D,
                      p.ws.part_lse + (size_t)(w_first + row) * G, G, G, D, nseg,
                      p.out + (size_t)q0 * D, p.lse + q0, s_w, s_red);
      if (tid == 0) p.ws.counters[row] = 0;
    }
    blk = seg_end;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace ws

using namespace ws;

// Workgroups of a GQA call: n_workgroups when given, else two per CU (the
// kernel's occupancy), at most what the blocks of the longest possible batch
// can feed with 8 blocks each, and no more than the in-kernel combine takes
// for G heads per row.
static int gqa_workgroups(int n_workgroups, int rows_kv, int G, int max_len) {
  if (n_workgroups > 0) return n_workgroups;
  const long long max_blocks = (long long)rows_kv * ((max_len + 31) / 32);
  const int n = choose_workgroups(0, kGqaStages <= 2 ? 2 : 1, max_blocks, 8);
  return std::min(n, kReduceMaxWeights / G);
}

static int gqa_launch(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                      uint16_t* k_pages, uint16_t* v_pages, const int32_t* page_table,
                      const int32_t* len_in, int32_t* len_out, int B, int Hq, int Hkv,
                      int D, int page_size, int max_pages, int num_pages, int max_len,
                      int n_workgroups, float scale, float* out, float* lse,
                      void* workspace, size_t workspace_bytes, void* stream,
                      bool combine, const char* name) {
  if (!q || !k_pages || !v_pages || !page_table || !len_in || !out || !lse)
    return set_error(WS_EINVAL, "%s: null pointer", name);
  if (B < 0 || B > kMaxSeqs || Hkv <= 0 || Hq <= 0 || Hq % Hkv)
    return set_error(WS_EINVAL, "%s: bad batch/heads B=%d Hq=%d Hkv=%d (B <= %d)", name,
                     B, Hq, Hkv, kMaxSeqs);
  const int G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16)
    return set_error(WS_EINVAL, "%s: group size %d unsupported (1,2,4,8,16)", name, G);
  if (D != kGqaD)
    return set_error(WS_EINVAL, "%s: head_dim %d unsupported (128)", name, D);
  if (page_size <= 0 || max_pages <= 0 || num_pages <= 0 || max_len < 0 ||
      (page_size % 32 && max_pages != 1) ||
      (long long)max_len > (long long)page_size * max_pages)
    return set_error(WS_EINVAL,
                     "%s: bad paging page_size=%d max_pages=%d num_pages=%d max_len=%d "
                     "(page_size must be a multiple of 32 unless max_pages == 1)",
                     name, page_size, max_pages, num_pages, max_len);
  if (n_workgroups < 0)
    return set_error(WS_EINVAL, "%s: n_workgroups %d < 0", name, n_workgroups);
  if (!aligned16(q) || !aligned16(k_pages) || !aligned16(v_pages) || !aligned16(out) ||
      (k_new && (!aligned16(k_new) || !aligned16(v_new))))
    return set_error(WS_EINVAL, "%s: buffers must be 16-byte aligned", name);
  if (k_new && !v_new) return set_error(WS_EINVAL, "%s: v_new is null", name);
  if (len_out && len_out == len_in)
    return set_error(WS_EINVAL, "%s: len_out must not alias len_in", name);
  if (B == 0) return WS_OK;
  const int rows_kv = B * Hkv;
  if (rows_kv > kCounterSlots)
    return set_error(WS_EINVAL, "%s: %d kv rows exceed the %d row counters", name, rows_kv,
                     kCounterSlots);
  if ((long long)rows_kv * ((max_len + 32) / 32) * 4096 >= (1LL << 31))
    return set_error(WS_EINVAL, "%s: %d kv rows of %d tokens exceed the block index range",
                     name, rows_kv, max_len);
  const int n = gqa_workgroups(n_workgroups, rows_kv, G, max_len);
  if ((long long)n * G > kReduceMaxWeights)
    return set_error(WS_EINVAL, "%s: %d workgroups of %d heads exceed the combine (%d)",
                     name, n, G, kReduceMaxWeights);
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
  prm.page_size = page_size;
  prm.max_pages = max_pages;
  prm.num_pages = num_pages;
  prm.cap = (int)std::min<long long>((long long)page_size * max_pages, 1LL << 30);
  prm.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(n), block(64 * kGqaWaves);
#define WS_GQA_CASE(GG)                                                                 \
  case GG:                                                                              \
    if (k_new && combine)                                                               \
      hipLaunchKernelGGL((gqa_decode_kernel<GG, true, true>), grid, block, 0, s, prm);  \
    else if (k_new)                                                                     \
      hipLaunchKernelGGL((gqa_decode_kernel<GG, true, false>), grid, block, 0, s, prm); \
    else if (combine)                                                                   \
      hipLaunchKernelGGL((gqa_decode_kernel<GG, false, true>), grid, block, 0, s, prm); \
    else                                                                                \
      hipLaunchKernelGGL((gqa_decode_kernel<GG, false, false>), grid, block, 0, s, prm); \
    break;
  switch (G) {
    WS_GQA_CASE(1)
    WS_GQA_CASE(2)
    WS_GQA_CASE(4)
    WS_GQA_CASE(8)
    WS_GQA_CASE(16)
  }
#undef WS_GQA_CASE
  return check_launch(name);
}

extern "C" int ws_decode_plan(int kind, int rows_kv, int heads, int max_len,
                              int n_workgroups, int* n_workgroups_out,
                              size_t* workspace_bytes_out) {
  if ((kind != 0 && kind != 1) || rows_kv < 0 || max_len < 0 || n_workgroups < 0 ||
      heads <= 0 || heads > 16)
    return set_error(WS_EINVAL, "ws_decode_plan: bad arguments");
  int n;
  size_t bytes;
  if (kind == 0) {
    n = gqa_workgroups(n_workgroups, rows_kv, heads, max_len);
    bytes = ws::workspace_bytes(rows_kv, heads, kGqaD, n);
  } else {
    n = mla_workgroups(n_workgroups, rows_kv, max_len);
    bytes = ws::workspace_bytes(rows_kv, heads, 512, n);
  }
  if (n_workgroups_out) *n_workgroups_out = n;
  if (workspace_bytes_out) *workspace_bytes_out = bytes;
  return WS_OK;
}

extern "C" int ws_gqa_decode_partial(
    const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
    const int32_t* page_table, const int32_t* gpu_len, int B, int Hq, int Hkv, int D,
    int page_size, int max_pages, int num_pages, int max_len, int n_workgroups,
    float scale, float* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  return gqa_launch(q, nullptr, nullptr, (uint16_t*)k_pages, (uint16_t*)v_pages,
                    page_table, gpu_len, nullptr, B, Hq, Hkv, D, page_size, max_pages,
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
                    Hq, Hkv, D, page_size, max_pages, num_pages, max_len, n_workgroups,
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
                    Hq, Hkv, D, page_size, max_pages, num_pages, max_len, n_workgroups,
                    scale, out, lse, workspace, workspace_bytes, stream, false,
                    "ws_gqa_append_decode_split");
}
