// Split-KV absorbed-MLA decode attention with 128 query heads (DeepSeek-V2)
// over the HBM partition (gfx950), optionally fused with the append of the
// decode step's new latent.  Included by ws_mla.hip, which dispatches calls
// whose layout is wide (ws_reduce.h mla_layout) here.
//
// The 16-head kernel would stream the shared latent once per 16-head group.
// Here every 32-token latent block is read from HBM once per workgroup and
// feeds all 128 heads: wave w owns heads [32w, 32w + 32), with its queries in
// registers (the B operand of v_mfma_f32_32x32x16_bf16 for the 36 16-wide
// k-steps of the 576-wide score: 144 VGPRs) and its 32 x 512 fp32 output in
// 256 accumulator registers.  Per block and wave:
//   QK       S^T[token][head] over 576 dims: 36 MFMAs, A = the block's latent
//            rows read from LDS (lane = token row, 8 dims)
//   softmax  lanes l and l ^ 32 hold 16 tokens each of head l % 32, in the
//            log2 domain against a reference max that stays fixed for the
//            segment (below)
//   PV       O^T[column][head] += V^T P^T: two 16-token k-steps x 16 column
//            tiles = 32 MFMAs.  P^T is the QK accumulator as it is: the
//            k-slots follow the accumulator rows (k-slot 8 j + 4 a + c of
//            k-step s is token 16 s + 8 a + 4 j + c, lane half j).  V^T comes
//            from 16-byte LDS reads of eight token rows per lane, paired into
//            dwords by v_perm; column tile (set, e) holds the columns
//            256 set + 8 m + e, so one read of 8 columns feeds 8 tiles.
// The waves never exchange data: they share the LDS tile and one barrier per
// block.  Blocks come from HBM straight into LDS (global_load_lds_dwordx4, no
// register staging): four tiles, block k consumed while k + 1 .. k + 3 are in
// flight (108 KB per CU).  A tile's rows are 72 16-byte chunks plus one pad
// chunk (row stride 73 chunks), so the 16 lanes of an LDS read phase hit 16
// different 4-bank groups both for the QK reads (one chunk of 16 rows:
// 73 m mod 16 is a permutation) and the PV reads (16 chunks of one row), and
// every operand read is one per-lane base plus an immediate offset.  A
// tile's 2336 chunks take 37 load instructions of 64 lanes; each wave issues
// 10 per block, the last 3 of them into a small sink, so every wave's
// outstanding-load count is the same.
//
// No rescaling: the output accumulators feed only MFMAs and the final stores,
// so they stay in AGPRs (a VALU rescale merged back into them makes the
// compiler keep them in VGPRs and copy them at every block).  The reference
// max m_ref of a head is its largest score in the segment's first block;
// probabilities 2^(x - m_ref) of later blocks may exceed 1 by up to 2^64
// (kWideHeadroomLog2), which fp32 sums and bf16 probabilities hold with their
// usual relative precision (both reach 2^127).  A segment whose scores climb
// further above m_ref runs again with the true maximum as the reference.
//
// Plan (ws_plan.h) over sequences (at most 64); a sequence held by one
// workgroup is written final (fp32 out / lse), otherwise each workgroup
// leaves a bf16 piece of all 128 heads in slot workgroup + sequence, which
// mla_reduce_kernel or the merges combine.
#pragma once

namespace ws {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWideRowChunks = 73;                      // 576 bf16 = 72 x 16 B, + 1 pad
constexpr int kWideTileChunks = 32 * kWideRowChunks;    // one 32-token block: 2336
constexpr int kWideTileDma = 37;                        // instructions of 64 chunks per tile
constexpr int kWideTileAlloc = kWideTileDma * 64;       // 2368 chunks
constexpr int kWideTiles = 4;
constexpr int kWideDmaPerWave = 10;                     // 4 x 10 = 37 + 3 into the sink
constexpr int kWideSinkDma = 4 * kWideDmaPerWave - kWideTileDma;
constexpr float kWideHeadroomLog2 = 64.f;
static_assert(kWideTileAlloc >= kWideTileChunks, "a tile holds its 37 instructions");

__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b,
                                               const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// The QK MFMAs with their 32 x 32 accumulator in VGPRs.  The output
// accumulators take all 256 AGPRs, and the compiler gives every MFMA of a
// function that uses AGPRs an AGPR accumulator: the scores would then
// compete with the outputs for AGPRs and be shuttled between the register
// files.  qk_first starts a chain (accumulator 0), qk_next continues it
// (back-to-back accumulation into the same registers needs no wait states),
// qk_last ends it with the wait states a VALU read of an XDL result needs
// (19 for a 16-pass MFMA, plus one on gfx950: 21 here), which the compiler's
// hazard tracking does not know about for inline assembly.
__device__ __forceinline__ void qk_first(f32x16& c, const u32x4& a, const u32x4& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void qk_next(f32x16& c, const u32x4& a, const u32x4& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void qk_last(f32x16& c, const u32x4& a, const u32x4& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 4"
               : "+v"(c)
               : "v"(a), "v"(b));
}

// One 16-byte chunk from global memory into LDS: lane i of the wave writes
// lds_base + 16 i (lds_base wave-uniform, in bytes).  Written as inline
// assembly: the compiler then does not see an LDS write whose completion it
// would wait for (vmcnt(0)) before every later LDS read, which would drain
// the blocks in flight; the kernel waits for completion itself
// (wide_wait_barrier).  Vector memory loads complete in issue order, so the
// waits the compiler computes for its own loads stay sufficient.
__device__ __forceinline__ void wide_dma16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(gptr), "s"(lds_base)
               : "memory");
}

// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// byte offset (no per-lane 64-bit address arithmetic).
__device__ __forceinline__ void wide_dma16_s(uint32_t off, const void* sbase,
                                             uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(sbase), "s"(lds_base)
               : "memory");
}

// Waits until at most N vector memory operations of this wave are in flight
// and its LDS reads are done, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void wide_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

template <bool APPEND>
__global__ __launch_bounds__(256) void mla_wide_kernel(const MlaParams p) {
  constexpr int NT = 256;
  constexpr int H = kWideHeads;
  constexpr int add = APPEND ? 1 : 0;
  __shared__ u32x4 s_tile[kWideTiles][kWideTileAlloc];
  __shared__ u32x4 s_sink[kWideSinkDma * 64];
  __shared__ int s_pref[kWideMaxSeqs + 1];
  __shared__ int s_len[kWideMaxSeqs];
  __shared__ int s_wpref[kSeqPlanMax + 1];
  __shared__ int s_scan[NT / 64 + 1];
  __shared__ int s_redo;
  const int g = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n32 = lane & 31;  // head (QK B, PV B, output) or row (A operands)
  const int j2 = lane >> 5;   // k-slot half
  const int head = 32 * wave + n32;
  // Byte offsets, within a block of 32 consecutive rows, of the chunks this
  // lane loads with its kWideDmaPerWave instructions (tile chunk c is row
  // c / 73, chunk c % 73 of the row, i.e. row-major chunk c - c / 73; pad
  // chunks and the sink read a chunk of the block), two 16-bit offsets per
  // register.
  uint32_t offp[kWideDmaPerWave / 2];
#pragma unroll
  for (int j = 0; j < kWideDmaPerWave / 2; ++j) {
    uint32_t v = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 64 * (kWideDmaPerWave * wave + 2 * j + h) + lane;
      const int off = min(16 * (c - c / kWideRowChunks), 32 * kMlaL * 2 - 16);
      v |= (uint32_t)off << (16 * h);
    }
    offp[j] = v;
  }

  if (APPEND && p.len_out && g == 0)
    for (int b = tid; b < p.B; b += NT) p.len_out[b] = step_len_out(p.len_in, b, add, p.cap);
  const Plan plan = plan_build<NT>(p.len_in, add, p.cap, p.B, 1, gridDim.x, s_pref, s_scan,
                                   s_len, s_wpref, g, 1);
  if (g == 0) {  // sequences without tokens: the empty partial (0, -inf), or
    for (int b = 0; b < p.B; ++b) {  // NaN for an invalid length
      if (s_pref[b + 1] != s_pref[b]) continue;
      const bool ok = len_ok(p.len_in[b], add, p.cap);
      for (int idx = tid; idx < H * kMlaC; idx += NT)
        p.out[(size_t)b * H * kMlaC + idx] = ok ? 0.f : qnan();
      if (tid < H) p.lse[b * H + tid] = ok ? neg_inf() : qnan();
    }
  }
  if (!plan.has_work) return;
  const int blk_begin = uniform(plan.begin);
  const int blk_end = uniform(plan.end);
  int blk = blk_begin;
  const char* g0 = (const char*)p.latent;
  const uint32_t tile_base0 = uniform((int)(uint32_t)(uintptr_t)&s_tile[0][0]);
  const uint32_t sink_base = uniform((int)(uint32_t)(uintptr_t)&s_sink[0]);

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
    const int32_t* pt = p.page_table + (size_t)b * p.max_pages;

    // Page ids of the segment's blocks, 64 at a time (lane l: block
    // pid_base + l), read with readlane; an id outside the pool is kept
    // clamped with bit 31 set (the loads read the clamped page, the piece is
    // NaN and the append skips it).
    int pid_base = 0;
    int m_pid = 0;
    int seg_bad = 0;
    auto fetch_pids = [&]() __attribute__((always_inline)) {
      const int t0 = t_begin + 32 * min(pid_base + lane, nblk - 1);
      const int raw = pt[t0 / p.page_size];
      const int pid = clamp_page(raw, p.num_pages);
      m_pid = pid | (raw == pid ? 0 : (int)0x80000000u);
    };
    fetch_pids();
    // Q^T of this wave's 32 heads: k-step u holds dims 16 u + 8 j2 .. + 8.
    u32x4 qb[36];
    {
      const size_t qrow = (size_t)b * H + head;
#pragma unroll
      for (int u = 0; u < 32; ++u)
        qb[u] = ((const u32x4*)(p.q_nope + qrow * kMlaC))[2 * u + j2];
#pragma unroll
      for (int u = 32; u < 36; ++u)
        qb[u] = ((const u32x4*)(p.q_pe + qrow * 64))[2 * (u - 32) + j2];
    }
    // The queries are needed from the first block on: have them in registers
    // before the block loads go out (the compiler's wait for them would
    // otherwise also wait for every block load in flight).
#pragma unroll
    for (int u = 0; u < 36; ++u) asm volatile("" : : "v"(qb[u]));

    const long long nc_off =
        APPEND ? (const char*)(p.c_new + (size_t)b * p.c_stride) - g0 : 0;
    const long long npe_off =
        APPEND ? (const char*)(p.pe_new + (size_t)b * p.pe_stride) - g0 : 0;
    // Block k of the segment into tile `slot`: this wave's 10 instructions
    // of 64 chunks (chunks 64 I .. 64 I + 63 of the tile, I = 10 wave + i,
    // the last three of wave 3 into the sink).  Rows past t_end repeat the
    // last valid row (masked in the softmax); a block past the segment's end
    // goes into a tile no later block of the segment uses.
    auto issue = [&](int k, int slot) __attribute__((always_inline)) {
      const bool valid = k < nblk;
      const int kc = min(k, nblk - 1);
      if (kc - pid_base >= 64) {
        pid_base += 64;
        fetch_pids();
      }
      const int t0 = t_begin + 32 * kc;
      const int page = t0 / p.page_size;
      const int pid_raw = __builtin_amdgcn_readlane(m_pid, kc - pid_base);
      seg_bad |= pid_raw;
      const int pid = pid_raw & 0x7fffffff;
      const long long lb =
          (long long)((size_t)pid * p.page_size + (t0 - page * p.page_size)) * (kMlaL * 2);
      const int last = min(32, t_end - t0) - 1;
      const int new_r = (APPEND && valid) ? len_old - t0 : -1;
      // LDS destinations: scalar, recomputed per block (not hoisted)
      uint32_t dst0 = tile_base0 + (uint32_t)slot * (kWideTileAlloc * 16) +
                      1024 * kWideDmaPerWave * wave;
      uint32_t sink0 = sink_base;
      asm volatile("" : "+s"(dst0), "+s"(sink0));
      if (!valid || (last == 31 && (unsigned)new_r >= 32u)) {
        // all 32 rows are tokens of the segment (or, past the segment's
        // end, the loads only have to stay in bounds: they read q_nope,
        // at least 128 KB): a scalar base and the precomputed offsets
        const char* sb = valid ? g0 + lb : (const char*)p.q_nope;
#pragma unroll
        for (int i = 0; i < kWideDmaPerWave; ++i) {
          const int I = kWideDmaPerWave * wave + i;
          const uint32_t off = (i & 1) ? offp[i >> 1] >> 16 : offp[i >> 1] & 0xffffu;
          const uint32_t dst = I < kWideTileDma ? dst0 + 1024 * i
                                                : sink0 + 1024 * (I - kWideTileDma);
          wide_dma16_s(off, sb, dst);
        }
        return;
      }
      // the segment's last block when partial or holding the appended
      // token: instruction I = 10 wave + i loads tile chunks 64 I .. 64 I +
      // 63 (row c / 73, chunk c % 73; the pad chunks and the sink take any
      // valid row), rows past t_end repeat the last valid row, the appended
      // token's row comes from c_new / pe_new
      int lane_v = lane;
      asm volatile("" : "+v"(lane_v));
#pragma unroll
      for (int i = 0; i < kWideDmaPerWave; ++i) {
        const int I = kWideDmaPerWave * wave + i;
        const int c = 64 * I + lane_v;
        const int r = min(c / kWideRowChunks, 31);
        const int x = min(c - (c / kWideRowChunks) * kWideRowChunks, 71);
        const int rr = min(r, last);
        long long off = lb + rr * (kMlaL * 2) + 16 * x;
        if (APPEND && rr == new_r) off = x < 64 ? nc_off + 16 * x : npe_off + 16 * (x - 64);
        const uint32_t dst = I < kWideTileDma ? dst0 + 1024 * i
                                              : sink0 + 1024 * (I - kWideTileDma);
        wide_dma16(g0 + off, dst);
      }
    };

    f32x16 acc[16];
    float m_run = neg_inf();  // reference max (m_ref); -inf until the first block
    float m_max = neg_inf();  // the segment's largest score so far
    float l_run = 0.f;

    // QK of one block into sc, two k-steps at a time (batch g: k-steps
    // 2 g, 2 g + 1): A = row n32 of the tile, k-step u = chunk 2 u + j2.
    auto qk_batch = [&](const u32x4* tile, int g, f32x16& sc) __attribute__((always_inline)) {
      const u32x4* arow = tile + n32 * kWideRowChunks + j2;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ku = 2 * g + u;
        const u32x4 kr = arow[2 * ku];
        if (ku == 0)
          qk_first(sc, kr, qb[ku]);
        else if (ku == 35)
          qk_last(sc, kr, qb[ku]);
        else
          qk_next(sc, kr, qb[ku]);
      }
    };
    // Softmax of block k from its scores: accumulator i is token
    // 8 (i / 4) + 4 j2 + i % 4 of head n32 (valid when below nt, the lane's
    // part moved to the right).  Writes P^T for the two PV k-steps.
    auto softmax = [&](int k, const f32x16& sc, u32x4 (&pb)[2]) __attribute__((always_inline)) {
      const int nt = min(32, t_end - (t_begin + 32 * k));
      const int lim = nt - 4 * j2;
      float x[16];
      float bm = neg_inf();
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x[i] = 8 * (i >> 2) + (i & 3) < lim ? sc[i] * p.scale_log2 : neg_inf();
        bm = fmaxf(bm, x[i]);
      }
      {
        float lo, hi;
        pair_xor32(bm, lo, hi);
        bm = fmaxf(lo, hi);
      }
      m_run = m_run == neg_inf() ? bm : m_run;
      m_max = fmaxf(m_max, bm);
      float ps = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float pa = __builtin_amdgcn_exp2f(x[8 * s + 2 * d] - m_run);
          const float pc = __builtin_amdgcn_exp2f(x[8 * s + 2 * d + 1] - m_run);
          ps += pa + pc;
          pb[s][d] = pack_bf16x2(pa, pc);
        }
      }
      l_run += ps;
    };
    // PV group g of a block (k-step s = g / 2, column set g % 2): lane
    // (n32, j2) reads the 16 bytes of columns 256 set + 8 n32 .. + 8 of tokens
    // 16 s + 8 (q >> 2) + 4 j2 + (q & 3) (16 lanes of one token read 16
    // consecutive chunks: no bank conflicts), one read feeding 8 tiles.
    auto pv_group = [&](const u32x4* tile, int g, const u32x4 (&pb)[2])
        __attribute__((always_inline)) {
      const int s = g >> 1, set = g & 1;
      const u32x4* vrow = tile + 4 * j2 * kWideRowChunks + n32 + 32 * set;
      u32x4 vr[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) vr[q] = vrow[(16 * s + 8 * (q >> 2) + (q & 3)) * kWideRowChunks];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        u32x4 va;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          va[d] = (e & 1) ? pair_hi(vr[2 * d][w], vr[2 * d + 1][w])
                          : pair_lo(vr[2 * d][w], vr[2 * d + 1][w]);
        acc[8 * set + e] = mfma32x32x16(va, pb[s], acc[8 * set + e]);
      }
    };

    // Ring over the four tiles (block m in tile m % 4).  Step k: wait for
    // block k (this wave's loads of blocks k + 1 and k + 2 may still be in
    // flight), the barrier (every wave's part of block k is in, every wave is
    // done with block k - 1's tile), block k + 3 into that tile, then block
    // k's QK, softmax and PV.  The tile of a block is picked at run time (its
    // LDS address is one scalar add).
    auto step = [&](int kk) __attribute__((always_inline)) {
      const int s = kk & (kWideTiles - 1);
      wide_wait_barrier<2 * kWideDmaPerWave>();
      // the pass's first barrier: every wave has read the previous decision
      if (kk == 0 && tid == 0) s_redo = 0;
      issue(kk + 3, (s + 3) & (kWideTiles - 1));
      __builtin_amdgcn_sched_barrier(0);
      const u32x4* tile = s_tile[s];
      f32x16 sc;
#pragma unroll
      for (int g = 0; g < 18; ++g) qk_batch(tile, g, sc);
      __builtin_amdgcn_sched_barrier(0);
      u32x4 pb[2];
      softmax(kk, sc, pb);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < 4; ++g) pv_group(tile, g, pb);
    };
    for (int pass = 0;; ++pass) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[e][i] = 0.f;
      l_run = 0.f;
      if (pid_base != 0) {
        pid_base = 0;
        fetch_pids();
      }
      issue(0, 0);
      issue(1, 1);
      issue(2, 2);
      for (int k = 0; k < nblk; ++k) step(k);
      // every load of the pass has landed and every wave is done with the
      // tiles (a second pass, or the next segment, overwrites them)
      const bool climbed = __builtin_amdgcn_ballot_w64(m_max > m_run + kWideHeadroomLog2) != 0;
      if (climbed && lane == 0) s_redo = 1;
      wide_wait_barrier<0>();
      const bool redo = s_redo != 0;
      if (pass > 0 || !redo) break;
      // scores climbed out of the reference's headroom: again, with the
      // segment's maximum as the reference (no score exceeds it)
      m_run = m_max;
      wide_wait_barrier<0>();  // every wave has read s_redo
    }

    // The appended token is its sequence's last, so a segment that holds it
    // ends with its block, whose tile is intact: row len_old - t0 of tile
    // (nblk - 1) % 4 holds its 72 chunks (read from c_new / pe_new), which go
    // into the token's page slot.
    if (APPEND && len_old >= t_begin && len_old < t_end) {
      const int t0 = t_begin + 32 * (nblk - 1);
      const int pid = __builtin_amdgcn_readlane(m_pid, nblk - 1 - pid_base);
      const int page = t0 / p.page_size;
      const int r = len_old - t0;
      if (tid < kWideRowChunks && pid >= 0)  // bit 31: the page id is outside the pool
        ((u32x4*)(p.latent_w +
                  ((size_t)pid * p.page_size + (len_old - page * p.page_size)) * kMlaL))[tid] =
            s_tile[(nblk - 1) % kWideTiles][r * kWideRowChunks + tid];
    }

    float lo, hi;
    pair_xor32(l_run, lo, hi);
    const float l_tot = lo + hi;
    const bool bad = seg_bad < 0;  // a bad page id was read (clamped): the piece is NaN
    const float inv_l = bad ? qnan() : 1.f / l_tot;
    const float lse_v = bad ? qnan() : (m_run + __log2f(l_tot)) * kLn2;
    const size_t orow = (size_t)b * H + head;
    // accumulator (set, e) value i is column 256 set + 64 (i / 4) + 32 j2 +
    // 8 (i % 4) + e: eight consecutive columns per (set, i)
    if (row_start >= blk_begin && row_end <= blk_end) {  // the whole sequence is here
      float* dst = p.out + orow * kMlaC;
#pragma unroll
      for (int set = 0; set < 2; ++set)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float4* o = (float4*)(dst + 256 * set + 64 * (i >> 2) + 32 * j2 + 8 * (i & 3));
          o[0] = make_float4(acc[8 * set + 0][i] * inv_l, acc[8 * set + 1][i] * inv_l,
                             acc[8 * set + 2][i] * inv_l, acc[8 * set + 3][i] * inv_l);
          o[1] = make_float4(acc[8 * set + 4][i] * inv_l, acc[8 * set + 5][i] * inv_l,
                             acc[8 * set + 6][i] * inv_l, acc[8 * set + 7][i] * inv_l);
        }
      if (j2 == 0) p.lse[orow] = lse_v;
    } else {
      const size_t prow = (size_t)(g + b) * H + head;
      uint16_t* dst = p.part_out + prow * kMlaC;
#pragma unroll
      for (int set = 0; set < 2; ++set)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          store_piece8(dst + 256 * set + 64 * (i >> 2) + 32 * j2 + 8 * (i & 3),
                       acc[8 * set + 0][i] * inv_l, acc[8 * set + 1][i] * inv_l,
                       acc[8 * set + 2][i] * inv_l, acc[8 * set + 3][i] * inv_l,
                       acc[8 * set + 4][i] * inv_l, acc[8 * set + 5][i] * inv_l,
                       acc[8 * set + 6][i] * inv_l, acc[8 * set + 7][i] * inv_l);
      if (j2 == 0) p.part_lse[prow] = lse_v;
    }
    blk = seg_end;
  }
}

}  // namespace ws
