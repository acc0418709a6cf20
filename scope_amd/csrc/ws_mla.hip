// Split-KV absorbed-MLA decode attention over the HBM partition (gfx950),
// optionally fused with the append of the decode step's new latent.
//
// Work decomposition (ws_plan.h): the grid's 256-thread workgroups take equal
// shares of all 32-token blocks of all sequences; the 16 heads of sequence b
// share each token's 576-wide latent (512 c_kv followed by 64 k_pe).  The
// workgroup reads each 32-token block from HBM once, with coalesced 16-byte
// loads, keeps three blocks in flight in registers and stages the block being
// consumed in an LDS tile, from which all MFMA operands are read: wave w
// computes the QK partial of token tile (w & 1) over latent half (w >> 1)
// (9 k-steps), the four score tiles meet in LDS, every wave runs the same
// online softmax, and wave w accumulates output columns [128w, 128w + 128).
// A sequence held by one workgroup is written final (fp32 out / lse);
// otherwise each workgroup stores a bf16 piece (slot workgroup + sequence,
// 16 KB) and a later launch combines them: mla_reduce_kernel for the
// one-launch entry points, ws_merge_split / ws_mla_merge_split_uv for the
// split step.
//
// With c_new != nullptr, token len_in[b] is the new latent: the ring reads
// its row from c_new/pe_new, the workgroup whose segment holds it writes it
// from its LDS tile into its page slot at the segment's end, and
// len_out[b] = len_in[b] + 1.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "ws_attn.h"
#include "ws_plan.h"
#include "ws_reduce.h"

namespace ws {

constexpr int kMlaH = 16;
constexpr int kMlaL = 576;
constexpr int kMlaC = 512;

struct MlaParams {
  const uint16_t* q_nope;
  const uint16_t* q_pe;
  const uint16_t* latent;
  uint16_t* latent_w;
  const int32_t* page_table;
  const int32_t* len_in;
  int32_t* len_out;
  const uint16_t* c_new;  // [B] rows of 512 (row stride c_stride) or nullptr
  const uint16_t* pe_new;
  long long c_stride, pe_stride;
  float* out;
  float* lse;
  uint16_t* part_out;  // [slot][16][512] bf16
  float* part_lse;     // [slot][16]
  // B: plan sequences v = b * ng + g, one per (sequence b, 16-head group g);
  // rows of q / out are v * 16 + h, i.e. b * H + 16 g + h with H = 16 ng.
  // The wide kernel plans sequences (ng = 1) with 128-head rows.
  int B, ng, page_size, max_pages, num_pages, cap;
  int hp;  // heads of a piece (and of a plan sequence's rows): 16, or 128 (wide)
  float scale_log2;
};

// A wave's 128 output columns of head n16 from its accumulators: acc[e][i] of
// lane group j is column 16 e + 4 j + i.
__device__ __forceinline__ void store_cols(float* __restrict__ dst, const f32x4 (&acc)[8],
                                           int j, float inv_l) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    *(float4*)(dst + 16 * e + 4 * j) = make_float4(acc[e][0] * inv_l, acc[e][1] * inv_l,
                                                   acc[e][2] * inv_l, acc[e][3] * inv_l);
}

// The same columns as a bf16 piece.
__device__ __forceinline__ void store_cols_piece(uint16_t* __restrict__ dst,
                                                 const f32x4 (&acc)[8], int j, float inv_l) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint2 v;
    v.x = pack_bf16x2(acc[e][0] * inv_l, acc[e][1] * inv_l);
    v.y = pack_bf16x2(acc[e][2] * inv_l, acc[e][3] * inv_l);
    *(uint2*)(dst + 16 * e + 4 * j) = v;
  }
}

// LDS tile of one 32-token block: row-major latent rows of 72 16-byte chunks
// plus two pad chunks.  A row stride of 74 chunks leaves the QK reads (16
// rows x 4 chunks per ds_read_b128) conflict-free, measured with the LDS
// bank-conflict counters on an in-bounds probe of that pattern (73 and 76:
// 2-way).  The PV reads (ds_read_b64_tr_b16: per 32-lane pass, rows 4 a ..
// 4 a + 7, 32 bytes of each) hit 64 different banks at this stride: rows
// 74 chunks apart fall in different 64-byte quarters of a 256-byte bank
// cycle, and the second four rows fill the other half of each quarter.
constexpr int kRowChunks = 74;
constexpr int kTileChunks = 32 * kRowChunks;
// Blocks in flight in registers while one is consumed from LDS.
constexpr int kMlaDepth = 3;
// 16-byte chunks of a block each thread moves (32 rows x 72 chunks / 256).
constexpr int kChunksPerThread = 9;

template <bool APPEND>
__global__ __launch_bounds__(256) void mla_decode_kernel(const MlaParams p) {
  constexpr int NT = 256;
  constexpr int add = APPEND ? 1 : 0;
  __shared__ u32x4 s_lat[3][kTileChunks];  // block k (PV), k + 1 (QK), k + 2 (being written)
  __shared__ f32x4 sbuf[2][2][2][64];      // [block parity][latent half][token tile][lane]
  __shared__ int s_pref[kMaxSeqs + 1];
  __shared__ int s_len[kMaxSeqs];
  __shared__ int s_wpref[kSeqPlanMax + 1];
  __shared__ int s_scan[NT / 64 + 1];
  const int g = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n16 = lane & 15;
  const int j = lane >> 4;
  const int tt = wave & 1;
  const int kh = wave >> 1;
  const int col0 = 128 * wave;
  // byte offset in a tile of this lane's V^T reads (token row 4 j + n16 / 4,
  // columns col0 + 4 (n16 % 4) ..); the read of output tile e adds 32 e bytes
  // (16 columns), the second read of a tile 16 rows
  const uint32_t v_lane =
      (uint32_t)(((4 * j + (n16 >> 2)) * kRowChunks) * 16 + 2 * col0 + 8 * (n16 & 3));

  if (APPEND && p.len_out && g == 0)
    for (int b = tid; b < p.B / p.ng; b += NT)
      p.len_out[b] = step_len_out(p.len_in, b, add, p.cap);
  const Plan plan = plan_build<NT>(p.len_in, add, p.cap, p.B, 1, gridDim.x, s_pref, s_scan,
                                   s_len, s_wpref, g, p.ng);
  if (g == 0) {  // sequences without tokens: the empty partial (0, -inf), or
    for (int b = 0; b < p.B; ++b) {  // NaN for an invalid length
      if (s_pref[b + 1] != s_pref[b]) continue;
      const bool ok = len_ok(p.len_in[seq_of(b, p.ng)], add, p.cap);
      for (int idx = tid; idx < kMlaH * kMlaC; idx += NT)
        p.out[(size_t)b * kMlaH * kMlaC + idx] = ok ? 0.f : qnan();
      if (tid < kMlaH) p.lse[b * kMlaH + tid] = ok ? neg_inf() : qnan();
    }
  }
  if (!plan.has_work) return;
  const int blk_begin = uniform(plan.begin);  // (the compiler cannot tell on its own)
  const int blk_end = uniform(plan.end);
  int blk = blk_begin;
  const u32x4* dummy = (const u32x4*)p.q_nope;

  while (blk < blk_end) {
    const int b = uniform((blk == blk_begin && plan.b0 >= 0) ? plan.b0
                                                             : plan_seq(s_pref, p.B, blk));
    const int len = uniform(s_len[b]);
    const int len_old = len - add;
    const int row_start = uniform(s_pref[b]);
    const int row_end = uniform(s_pref[b + 1]);
    const int seg_end = min(blk_end, row_end);
    const int t_begin = (blk - row_start) * 32;
    const int t_end = min(len, (seg_end - row_start) * 32);
    const int nblk = seg_end - blk;
    const int orow = b * kMlaH + n16;  // b: plan sequence (sequence, head group)
    const int sb = uniform(seq_of(b, p.ng));  // the sequence whose latent it reads
    const int32_t* pt = p.page_table + (size_t)sb * p.max_pages;

    // Pool token index of the first row of each of the segment's blocks, 64
    // at a time (lane l: block pid_base + l), read with readlane: the ring
    // issues no load whose address waits on another load (a page-table read
    // per block would make every block wait for all loads in flight).  They
    // are requested first: the first KV requests wait for them.  A page id
    // outside the pool is kept clamped and marks the index with bit 31: the
    // loads read the clamped page, the append skips it.  (The clamp also
    // keeps the wait for the page-table load inside the refill branch: the
    // raw value flowing out of it would make the compiler wait for every
    // load in flight on each block.)  A block never crosses a page (page
    // sizes are multiples of 32, or the pool has one page per sequence).
    int pid_base = 0;
    int m_tok = 0;
    int seg_bad = 0;  // bit 31: a block of the segment had a page id outside the pool
    auto fetch_pids = [&]() {
      const int t0 = t_begin + 32 * min(pid_base + lane, nblk - 1);
      const int page = t0 / p.page_size;
      const int raw = pt[page];
      const int pid = clamp_page(raw, p.num_pages);
      m_tok = (pid * p.page_size + (t0 - page * p.page_size)) |
              (raw == pid ? 0 : (int)0x80000000u);
    };
    fetch_pids();

    // Q^T for this wave's 9 QK k-steps: k = 32 * (9 * kh + u) + 8 * j .. + 8.
    // Requested after the first KV block (the first QK needs it later).
    u32x4 qb[9];
    auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < 9; ++u) {
        const int k0 = 32 * (9 * kh + u) + 8 * j;
        if (k0 < kMlaC)
          qb[u] = ((const u32x4*)(p.q_nope + (size_t)orow * kMlaC))[k0 >> 3];
        else
          qb[u] = ((const u32x4*)(p.q_pe + (size_t)orow * 64))[(k0 - kMlaC) >> 3];
      }
    };

    f32x4 acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = neg_inf();
    float l_run = 0.f;

    // Block k of the segment, as this thread's 9 chunks: the 32 rows' c_kv
    // parts are 8 loads of 4 whole rows (1 KB per wave) and their k_pe parts
    // one load.  Rows past t_end repeat the last valid row (masked in the
    // softmax); past the segment's last block every lane reads the first 16
    // bytes of q_nope instead (a cache hit).
    // Addresses are selected as byte offsets from one global base (a pointer
    // select per chunk compiles to divergent branches, and an integer round
    // trip loses the address space, turning the loads into flat loads whose
    // completion the compiler can only wait for all at once).
    const char* g0 = (const char*)p.latent;
    const long long nc_off =
        APPEND ? (const char*)(p.c_new + (size_t)sb * p.c_stride) - g0 : 0;
    const long long npe_off =
        APPEND ? (const char*)(p.pe_new + (size_t)sb * p.pe_stride) - g0 - 16 * (kMlaC / 8) : 0;
    const long long dummy_off = (const char*)dummy - g0;
    const int pe_row = tid >> 3;
    const int pe_col = kMlaC / 8 + (tid & 7);
    // Byte offsets of a thread's chunks inside a block: chunk u at row
    // 4 u + wave, column `lane` (vo_row + u * 4 rows); chunk 8 at vo_pe.
    const uint32_t vo_row = (uint32_t)(wave * (kMlaL * 2) + 16 * lane);
    const uint32_t vo_pe = (uint32_t)(pe_row * (kMlaL * 2) + 16 * pe_col);
    auto gload = [&](int k, u32x4 (&dst)[kChunksPerThread]) {
      const bool valid = k < nblk;
      const int kc = min(k, nblk - 1);
      if (kc - pid_base >= 64) {
        pid_base += 64;
        fetch_pids();
      }
      const int t0 = t_begin + 32 * kc;
      const int tok_raw = __builtin_amdgcn_readlane(m_tok, kc - pid_base);
      seg_bad |= tok_raw;
      const long long lb = (long long)(uint32_t)(tok_raw & 0x7fffffff) * (kMlaL * 2);
      const int last = min(32, t_end - t0) - 1;
      const int new_r = (APPEND && valid) ? len_old - t0 : -1;
      if (valid && last == 31 && (unsigned)new_r > 31u) {
        // A full block without the appended token (all but a segment's last
        // few requests): one scalar base, fixed per-lane offsets.
        const char* bp = g0 + lb;
#pragma unroll
        for (int u = 0; u < 8; ++u) dst[u] = ld_stream(bp + u * (4 * kMlaL * 2) + vo_row);
        dst[8] = ld_stream(bp + vo_pe);
        return;
      }
      // Chunks 0..7 of a thread: row 4 u + wave, 16-byte column `lane` of
      // the row's c_kv part (each load reads whole rows, so its row, clamp
      // and new-token test are uniform); chunk 8: row tid / 8, k_pe column
      // tid % 8.
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int r = min(4 * u + wave, last);
        const long long row = (APPEND && r == new_r) ? nc_off : lb + r * (kMlaL * 2);
        const long long off = valid ? row + 16 * lane : dummy_off;
        dst[u] = ld_stream(g0 + off);
      }
      {
        const int r = min(pe_row, last);
        long long off = lb + r * (kMlaL * 2) + 16 * pe_col;
        if (APPEND) off = r == new_r ? npe_off + 16 * pe_col : off;
        off = valid ? off : dummy_off;
        dst[8] = ld_stream(g0 + off);
      }
    };
    auto lwrite = [&](u32x4* tile, const u32x4 (&src)[kChunksPerThread]) {
#pragma unroll
      for (int u = 0; u < 8; ++u) tile[(4 * u + wave) * kRowChunks + lane] = src[u];
      tile[pe_row * kRowChunks + pe_col] = src[8];
    };
    // QK partial of block k from its LDS tile: token tile tt over latent
    // half kh, into score buffer `par`.
    // All nine operand reads go out before the first MFMA (the MFMA chain
    // is serial; read by read, each would wait a full LDS round trip).
    auto qk_read = [&](const u32x4* tile, u32x4 (&kr)[9]) {
      const u32x4* krow = tile + (16 * tt + n16) * kRowChunks + j;
#pragma unroll
      for (int u = 0; u < 9; ++u) kr[u] = krow[4 * (9 * kh + u)];
    };
    auto qk_mfma = [&](const u32x4 (&kr)[9], int par) {
      f32x4 sp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 9; ++u) sp = mfma16x16x32(kr[u], qb[u], sp);
      sbuf[par][kh][tt][lane] = sp;
    };
    auto qk = [&](const u32x4* tile, int par) {
      u32x4 kr[9];
      qk_read(tile, kr);
      __builtin_amdgcn_sched_barrier(0);
      qk_mfma(kr, par);
    };
    // Softmax of block k from its four score partials sp (latent halves 0 and
    // 1 of token tile 0, then of token tile 1), then PV of this wave's 128
    // output columns from the block's tile.
    auto finish = [&](int k, const u32x4* tile, const f32x4 (&sp)[4]) {
      const int nt = min(32, t_end - (t_begin + 32 * k));
      const f32x4 s0 = sp[0] + sp[1];
      const f32x4 s1 = sp[2] + sp[3];
      float alpha;
      bool rescale;
      const u32x4 pb =
          softmax_block(s0, s1, j, nt, p.scale_log2, m_run, l_run, alpha, rescale);
      // V^T straight from LDS: for output tile e, lanes 4 e' + r of lane
      // group j address token rows 4 j + e' and 16 + 4 j + e' (the k-slots of
      // pb, pv_token) at columns col0 + 16 e + 4 r, so result lane m holds
      // four tokens of column col0 + 16 e + m (lds_read_tr_b64).
      if (rescale) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = acc[e] * alpha;
      }
      // (All sixteen reads go out before the first MFMA, as in the QK.)
      const uint32_t vt = (uint32_t)(uintptr_t)tile + v_lane;
      uint2 lo[8], hi[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lo[e] = lds_read_tr_b64(vt + 32 * e);
        hi[e] = lds_read_tr_b64(vt + 32 * e + 16 * 16 * kRowChunks);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        acc[e] = mfma16x16x32(u32x4{lo[e].x, lo[e].y, hi[e].x, hi[e].y}, pb, acc[e]);
    };

    // Pipeline over three LDS tiles (block m in tile m % 3) and three
    // register slots (block m in slot m % 3).  Step k, between two barriers:
    // block k + 2 from its register slot into its tile and the request of
    // block k + 5 into that slot (first, so the requests queue while the math
    // runs), softmax + PV of block k (its scores were exchanged before the
    // barrier), QK of block k + 1 into the other score buffer (independent of
    // block k's math, so the two overlap).  One
    // barrier per block; blocks k + 3 .. k + 5 are in flight meanwhile.  The
    // loop body is a whole turn of the ring with no early exit (the last
    // nblk % 3 blocks run after it): a path around part of the turn makes the
    // compiler assume the younger slots' loads may be the ones a slot write
    // waits for, and it then waits for every load in flight.
    u32x4 st[kMlaDepth][kChunksPerThread];
    gload(0, st[0]);
    load_q();
    gload(1, st[1]);
    gload(2, st[2]);
    __syncthreads();  // the previous segment is done with the tiles and sbuf
    lwrite(s_lat[0], st[0]);
    gload(3, st[0]);
    if (nblk > 1) lwrite(s_lat[1], st[1]);
    gload(4, st[1]);
    __syncthreads();
    qk(s_lat[0], 0);
    __syncthreads();
    auto step = [&](auto slot, int kk) {
      constexpr int s = decltype(slot)::value;  // kk % 3
      if (kk + 2 < nblk) lwrite(s_lat[(s + 2) % 3], st[(s + 2) % 3]);
      gload(kk + 5, st[(s + 2) % 3]);
      // block k's scores, then block k + 1's QK operands, requested before
      // block k's softmax, which does not need them (LDS reads complete in
      // order; past the segment's last block the QK reads see a stale tile
      // and go unused)
      const int par = kk & 1;
      const f32x4 sp[4] = {sbuf[par][0][0][lane], sbuf[par][1][0][lane], sbuf[par][0][1][lane],
                           sbuf[par][1][1][lane]};
      __builtin_amdgcn_sched_barrier(0);
      u32x4 kr[9];
      qk_read(s_lat[(s + 1) % 3], kr);
      __builtin_amdgcn_sched_barrier(0);
      finish(kk, s_lat[s], sp);
      if (kk + 1 < nblk) qk_mfma(kr, (kk + 1) & 1);
      __syncthreads();
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    static_assert(kMlaDepth == 3, "the ring turn below is written for three slots");
    int k = 0;
    for (; k + 3 <= nblk; k += 3) {
      step(S0{}, k);
      step(S1{}, k + 1);
      step(S2{}, k + 2);
    }
    if (k < nblk) step(S0{}, k);
    if (k + 1 < nblk) step(S1{}, k + 1);

    // The appended token is its sequence's last, so a segment that holds it
    // ends with its block, whose tile is still intact: row len_old - t0 of
    // tile (nblk - 1) % 3 holds its 72 chunks (read from c_new / pe_new by
    // the ring), which go from LDS into the token's page slot.  (Head group
    // 0 of the sequence writes it.)
    if (APPEND && len_old >= t_begin && len_old < t_end && b == sb * p.ng) {
      const int t0 = t_begin + 32 * (nblk - 1);
      const int tok = __builtin_amdgcn_readlane(m_tok, nblk - 1 - pid_base);
      if (tid < kMlaL / 8 && tok >= 0)  // bit 31: the page id is outside the pool
        ((u32x4*)(p.latent_w + ((size_t)tok + (len_old - t0)) * kMlaL))[tid] =
            s_lat[(nblk - 1) % 3][(len_old - t0) * kRowChunks + tid];
    }

    const float l_tot = wave_sum_xor16_32(l_run);
    const bool bad = seg_bad < 0;  // a bad page id was read (clamped): the piece is NaN
    const float inv_l = bad ? qnan() : 1.f / l_tot;
    const float lse_v = bad ? qnan() : (m_run + __log2f(l_tot)) * kLn2;
    if (row_start >= blk_begin && row_end <= blk_end) {  // the whole sequence is here
      store_cols(p.out + (size_t)orow * kMlaC + col0, acc, j, inv_l);
      if (wave == 0 && j == 0) p.lse[orow] = lse_v;
    } else {
      const size_t prow = (size_t)(g + b) * kMlaH + n16;
      store_cols_piece(p.part_out + prow * kMlaC + col0, acc, j, inv_l);
      if (wave == 0 && j == 0) p.part_lse[prow] = lse_v;
    }
    blk = seg_end;
  }
}

}  // namespace ws

#include "ws_mla_wide.h"

namespace ws {

// Combines the partials of sequences held by several workgroups: one 64-lane
// workgroup per (head row, 256-column chunk).  Recomputes the decode's plan
// to find the sequence's workgroups (slots w + b for w in its owner range).
// Runs after the decode kernel on the same stream, so plain loads see the
// partials.
__global__ __launch_bounds__(64) void mla_reduce_kernel(const MlaParams p, int grid) {
  __shared__ int s_pref[kMaxSeqs + 1];
  __shared__ int s_wpref[kSeqPlanMax + 1];
  __shared__ int s_scan[2];
  __shared__ float s_w[kReduceMaxWeights];
  const int hrow = blockIdx.x;  // b * hp + h
  const int chunk = blockIdx.y;
  const int t = threadIdx.x;
  const int b = hrow / p.hp;
  const int h = hrow - b * p.hp;
  const int add = p.c_new ? 1 : 0;
  const Plan plan = plan_build<64>(p.len_in, add, p.cap, p.B, 1, grid, s_pref, s_scan, nullptr,
                                   s_wpref, -1, p.ng);
  const int row_start = s_pref[b], row_end = s_pref[b + 1];
  if (row_end == row_start) return;
  int w_first, n;
  plan_row_splits(plan, b, row_start, row_end - row_start, s_wpref, w_first, n);
  if (n == 1) return;
  const size_t slot0 = (size_t)(w_first + b) * p.hp + h;  // partial row of split 0
  const int c = chunk * 64 + t;  // float4 column
  // the pieces' columns are requested with their lse values
  uint2 pv[8];
  if (n <= 8) preload_pieces(p.part_out + slot0 * kMlaC + 4 * c, (size_t)p.hp * kMlaC, n, pv);
  float mx = neg_inf();
  for (int s = t; s < n; s += 64) {
    const float v = p.part_lse[slot0 + (size_t)s * p.hp];
    s_w[s] = v;
    mx = max_nan(mx, v);
  }
  for (int o = 1; o < 64; o <<= 1) mx = max_nan(mx, __shfl_xor(mx, o));
  float sum = 0.f;
  for (int s = t; s < n; s += 64) {
    const float w = __expf(s_w[s] - mx);
    s_w[s] = w;
    sum += w;
  }
  for (int o = 1; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
  __syncthreads();
  if (chunk == 0 && t == 0) p.lse[hrow] = mx + __logf(sum);
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n <= 8)
    accum_preloaded(pv, n, s_w, a);
  else
    accum_pieces(p.part_out + slot0 * kMlaC + 4 * c, (size_t)p.hp * kMlaC, n, s_w, a);
  const float inv = 1.f / sum;
  ((float4*)(p.out + (size_t)hrow * kMlaC))[c] =
      make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Workgroups of an MLA call: n_workgroups when given, else one per CU (the
// kernel's occupancy), at most what the blocks of the longest possible batch
// can feed with 4 blocks each, and no more than the reduction's weights hold.
int mla_workgroups(int n_workgroups, int B, int max_len) {
  if (n_workgroups > 0) return n_workgroups;
  const long long max_blocks = (long long)B * ((max_len + 31) / 32);
  const int n = choose_workgroups(0, 1, max_blocks, 4);
  return std::min(n, kReduceMaxWeights);
}

static int mla_launch(const uint16_t* q_nope, const uint16_t* q_pe,
                      const uint16_t* c_new, long long c_stride, const uint16_t* pe_new,
                      long long pe_stride, uint16_t* latent_pages,
                      const int32_t* page_table, const int32_t* len_in,
                      int32_t* len_out, int B, int H, int page_size, int max_pages,
                      int num_pages, int max_len, int n_workgroups, float scale,
                      float* out, float* lse, void* workspace, size_t workspace_bytes,
                      void* stream, bool combine, const char* name) {
  if (!q_nope || !q_pe || !latent_pages || !page_table || !len_in || !out || !lse)
    return set_error(WS_EINVAL, "%s: null pointer", name);
  // H = 16 ng: each 16-head group is its own plan sequence over the shared latent
  if (B < 0 || H < kMlaH || H % kMlaH || (long long)B * (H / kMlaH) > kMaxSeqs)
    return set_error(WS_EINVAL,
                     "%s: B=%d H=%d unsupported (H a multiple of 16, B * H / 16 <= %d)", name, B,
                     H, kMaxSeqs);
  // 128 heads over at most 64 sequences: the wide kernel, one plan sequence
  // per sequence and 128-head pieces (ws_reduce.h mla_layout)
  const MlaLayout lay = mla_layout(B, H);
  const int ng = lay.ng;
  if (page_size <= 0 || max_pages <= 0 || num_pages <= 0 || max_len < 0 ||
      (page_size % 32 && max_pages != 1) ||
      (long long)max_len > (long long)page_size * max_pages)
    return set_error(WS_EINVAL,
                     "%s: bad paging page_size=%d max_pages=%d num_pages=%d max_len=%d",
                     name, page_size, max_pages, num_pages, max_len);
  if (n_workgroups < 0 || n_workgroups > kReduceMaxWeights)
    return set_error(WS_EINVAL, "%s: n_workgroups %d outside [0, %d]", name, n_workgroups,
                     kReduceMaxWeights);
  if (!aligned16(q_nope) || !aligned16(q_pe) || !aligned16(latent_pages) ||
      !aligned16(out))
    return set_error(WS_EINVAL, "%s: buffers must be 16-byte aligned", name);
  if (c_new && (!pe_new || !aligned16(c_new) || !aligned16(pe_new) || c_stride < 512 ||
                pe_stride < 64 || c_stride % 8 || pe_stride % 8))
    return set_error(WS_EINVAL, "%s: bad new-latent buffers", name);
  if (len_out && len_out == len_in)
    return set_error(WS_EINVAL, "%s: len_out must not alias len_in", name);
  if (B == 0) return WS_OK;
  const int Bv = lay.plan_seqs;  // plan sequences (sequence, head group)
  const int hp = lay.piece_heads;
  if ((long long)Bv * ((max_len + 32) / 32) * 4096 >= (1LL << 31))
    return set_error(WS_EINVAL, "%s: %d sequences of %d tokens exceed the block index range",
                     name, Bv, max_len);
  if ((long long)num_pages * page_size >= (1LL << 31))  // bit 31 marks bad page ids
    return set_error(WS_EINVAL, "%s: pools of %lld tokens exceed the 31-bit token index", name,
                     (long long)num_pages * page_size);
  const int n = mla_workgroups(n_workgroups, Bv, max_len);
  const size_t need = ws::workspace_bytes(Bv, hp, kMlaC, n);
  if (!workspace || workspace_bytes < need)
    return set_error(WS_EWORKSPACE, "%s: workspace %zu < %zu bytes", name, workspace_bytes,
                     need);
  if (((uintptr_t)workspace & 255u) != 0)
    return set_error(WS_EINVAL, "%s: workspace must be 256-byte aligned", name);
  const SplitWorkspace w = carve_workspace(workspace, Bv, hp, n);
  MlaParams prm;
  prm.q_nope = q_nope;
  prm.q_pe = q_pe;
  prm.latent = latent_pages;
  prm.latent_w = latent_pages;
  prm.page_table = page_table;
  prm.len_in = len_in;
  prm.len_out = len_out;
  prm.c_new = c_new;
  prm.pe_new = pe_new;
  prm.c_stride = c_stride;
  prm.pe_stride = pe_stride;
  prm.out = out;
  prm.lse = lse;
  prm.part_out = w.part_out;
  prm.part_lse = w.part_lse;
  prm.B = Bv;
  prm.ng = ng;
  prm.hp = hp;
  prm.page_size = page_size;
  prm.max_pages = max_pages;
  prm.num_pages = num_pages;
  prm.cap = (int)std::min<long long>((long long)page_size * max_pages, 1LL << 30);
  prm.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  if (lay.wide) {
    if (c_new)
      hipLaunchKernelGGL(mla_wide_kernel<true>, dim3(n), dim3(256), 0, s, prm);
    else
      hipLaunchKernelGGL(mla_wide_kernel<false>, dim3(n), dim3(256), 0, s, prm);
  } else if (c_new) {
    hipLaunchKernelGGL(mla_decode_kernel<true>, dim3(n), dim3(256), 0, s, prm);
  } else {
    hipLaunchKernelGGL(mla_decode_kernel<false>, dim3(n), dim3(256), 0, s, prm);
  }
  int rc = check_launch(name);
  if (rc || n == 1 || !combine) return rc;
  hipLaunchKernelGGL(mla_reduce_kernel, dim3(Bv * hp, kMlaC / 256), dim3(64), 0, s, prm, n);
  return check_launch(name);
}

}  // namespace ws

using namespace ws;

extern "C" int ws_mla_decode_partial(const uint16_t* q_nope, const uint16_t* q_pe,
                                     const uint16_t* latent_pages,
                                     const int32_t* page_table, const int32_t* gpu_len,
                                     int B, int H, int page_size, int max_pages,
                                     int num_pages, int max_len, int n_workgroups,
                                     float scale, float* out, float* lse, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return mla_launch(q_nope, q_pe, nullptr, 0, nullptr, 0, (uint16_t*)latent_pages,
                    page_table, gpu_len, nullptr, B, H, page_size, max_pages, num_pages,
                    max_len, n_workgroups, scale, out, lse, workspace, workspace_bytes,
                    stream, true, "ws_mla_decode_partial");
}

extern "C" int ws_mla_append_decode_partial(
    const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_new,
    int64_t c_stride, const uint16_t* pe_new, int64_t pe_stride, uint16_t* latent_pages,
    const int32_t* page_table, const int32_t* len_in, int32_t* len_out, int B, int H,
    int page_size, int max_pages, int num_pages, int max_len, int n_workgroups,
    float scale, float* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  if (!c_new) return set_error(WS_EINVAL, "ws_mla_append_decode_partial: c_new is null");
  return mla_launch(q_nope, q_pe, c_new, c_stride, pe_new, pe_stride, latent_pages,
                    page_table, len_in, len_out, B, H, page_size, max_pages, num_pages,
                    max_len, n_workgroups, scale, out, lse, workspace, workspace_bytes,
                    stream, true, "ws_mla_append_decode_partial");
}

extern "C" int ws_mla_append_decode_split(
    const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_new,
    int64_t c_stride, const uint16_t* pe_new, int64_t pe_stride, uint16_t* latent_pages,
    const int32_t* page_table, const int32_t* len_in, int32_t* len_out, int B, int H,
    int page_size, int max_pages, int num_pages, int max_len, int n_workgroups,
    float scale, float* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  if (!c_new) return set_error(WS_EINVAL, "ws_mla_append_decode_split: c_new is null");
  return mla_launch(q_nope, q_pe, c_new, c_stride, pe_new, pe_stride, latent_pages,
                    page_table, len_in, len_out, B, H, page_size, max_pages, num_pages,
                    max_len, n_workgroups, scale, out, lse, workspace, workspace_bytes,
                    stream, false, "ws_mla_append_decode_split");
}
