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
//   PV       O^T[column][head] += V^T P^T: two 16-token k-steps x 16 tiles of
//            32 columns = 32 MFMAs.  P^T is the QK accumulator as it is: the
//            k-slots follow the accumulator rows (k-slot 8 j + 4 a + c of
//            k-step s is token 16 s + 8 a + 4 j + c, lane half j).  V^T comes
//            straight from LDS with ds_read_b64_tr_b16 (two per MFMA): in each
//            16-lane group, result lane 4 r + j, element e is element j of the
//            8 bytes that lane 4 e + r addresses, so lanes 4 e + r pointing at
//            token row e, columns 4 r .. 4 r + 3 deliver four tokens of one
//            column per lane.
// The waves never exchange data: they share the LDS tile and one barrier per
// block.  Blocks come from HBM straight into LDS (global_load_lds_dwordx4, no
// register staging): four tiles, block k consumed while k + 1 .. k + 3 are in
// flight (148 KB per CU), each wave's ten load instructions of a block spread
// over its MFMAs (a burst stalls the wave while the memory pipeline drains).
//
// Tile layout.  gfx950's LDS serves 256 bytes per pass, 64 banks of 4 bytes
// (as the bank-conflict counter measures it): a 64-lane ds_read_b128 takes
// four passes of 16 lanes, ds_read_b64_tr_b16 two passes of 32 lanes, and a
// pass whose lanes hit one bank twice takes a cycle more per repeat.  Row r
// of a tile (72 chunks of 16 bytes) starts at chunk
// wide_row_off(r) = 72 r + 5 (r / 4) + 4 ((r / 2) % 2), so that
//   - the QK reads (16 rows, one chunk each per pass) hit 16 different
//     chunk slots mod 16: the offsets of rows 0 .. 15, and of 16 .. 31, are
//     distinct mod 16;
//   - the PV transposed reads (rows 4 a .. 4 a + 3, 64 bytes of each row per
//     pass) hit 64 different banks: within each aligned 4-row group the
//     offsets are c, c + 4, c + 8, c + 12 mod 16.
// Every operand read is one per-lane base plus an immediate offset.  A tile's
// 2368 chunks (2343 used) take 37 load instructions of 64 lanes: instruction
// i of wave w fills chunks 64 I .. 64 I + 63, I = w + 4 i, and the waves
// other than wave 0 send their tenth (I = 37 .. 39) into a 1 KB sink, so
// every wave's outstanding-load count is the same (ten per block).
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

constexpr int kWideRowData = 72;  // 576 bf16 = 72 x 16 B
// LDS chunk offset of row r of a tile.
__host__ __device__ constexpr int wide_row_off(int r) {
  return kWideRowData * r + 5 * (r >> 2) + 4 * ((r >> 1) & 1);
}
constexpr int kWideTileChunks = wide_row_off(31) + kWideRowData;  // 2343
constexpr int kWideTileDma = (kWideTileChunks + 63) / 64;         // 37 instructions of 64 chunks
constexpr int kWideTileAlloc = kWideTileDma * 64;                 // 2368 chunks
constexpr int kWideTiles = 4;
constexpr int kWideDmaPerWave = 10;  // 4 x 10 = 37 + 3 into the sink
constexpr float kWideHeadroomLog2 = 64.f;
// chunk offsets of rows 16 s + 8 t + q (q < 8) are wide_row_off(q) + 1172 s + 586 t
constexpr int kWideRowsS = 1172, kWideRowsT = 586;
static_assert(wide_row_off(16) == kWideRowsS * 1 + 0 && wide_row_off(8) == kWideRowsT &&
                  wide_row_off(24 + 7) == wide_row_off(7) + kWideRowsS + kWideRowsT,
              "row offsets split into a row-group part and a per-lane part");
static_assert(kWideTileDma == 37 && 4 * (kWideDmaPerWave - 1) == kWideTileDma - 1,
              "instructions 0-8 of every wave and instruction 9 of wave 0 fill the tile");

// Row of tile chunk c (the pad chunks after a row count as that row's; c past
// the tile gives row 31).
__device__ __forceinline__ int wide_row_of(int c) {
  int r = min(c / 74, 31);  // 72 r <= wide_row_off(r) <= 74 r: the row is r or r + 1
  if (r < 31 && wide_row_off(r + 1) <= c) ++r;
  return r;
}

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
// hazard tracking does not know about for inline assembly.  The memory
// clobber keeps LDS reads on the side of each MFMA where the source puts
// them (the kernel places its reads a few MFMAs ahead of their use).
__device__ __forceinline__ void qk_first(f32x16& c, const u32x4& a, const u32x4& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b) : "memory");
}
__device__ __forceinline__ void qk_next(f32x16& c, const u32x4& a, const u32x4& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b) : "memory");
}
__device__ __forceinline__ void qk_last(f32x16& c, const u32x4& a, const u32x4& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 4"
               : "+v"(c)
               : "v"(a), "v"(b)
               : "memory");
}

// One 16-byte chunk per lane from global memory into LDS, from the
// wave-uniform 64-bit base `sbase` (SGPRs) plus the lane's 32-bit byte offset:
// lane i of the wave writes lds_base + 16 i (lds_base wave-uniform, in
// bytes).  Written as inline assembly: the compiler then does not see an LDS
// write whose completion it would wait for (vmcnt(0)) before every later LDS
// read, which would drain the blocks in flight; the kernel waits for
// completion itself (wide_wait_barrier).  Vector memory loads complete in
// issue order, so the waits the compiler computes for its own loads stay
// sufficient.
__device__ __forceinline__ void wide_dma16_s(uint32_t off, const void* sbase,
                                             uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(sbase), "s"(lds_base)
               : "memory");
}

// The same with the LDS destination lds_base + imm, imm a constant once the
// caller's loop is unrolled (one scalar add into M0).
__device__ __forceinline__ void wide_dma16_add(uint32_t off, const void* sbase,
                                               uint32_t lds_base, int imm) {
  asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(sbase), "s"(lds_base), "i"(imm)
               : "memory", "scc");
}

// Waits until at most N vector memory operations of this wave are in flight
// and its LDS reads are done, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void wide_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Waits for this wave's LDS operations and joins the workgroup barrier.
__device__ __forceinline__ void wide_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}
// Waits for this wave's LDS operations (its own LDS writes before it reads
// other lanes' values back).
__device__ __forceinline__ void wide_lds_wait() {
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
}

// Stores 32 staged 1 KB rows (row h at src + 260 h dwords, lane part at
// src) to dst + h * row_bytes + col_byte, eight rows' LDS reads in flight
// before their stores.
__device__ __forceinline__ void wide_store_rows(char* dst, int row_bytes, const uint32_t* src,
                                                int col_byte) {
#pragma unroll
  for (int h0 = 0; h0 < 32; h0 += 8) {
    u32x4 v[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) v[h] = *(const u32x4*)(src + (h0 + h) * 260);
#pragma unroll
    for (int h = 0; h < 8; ++h)
      *(u32x4*)(dst + (size_t)(h0 + h) * row_bytes + col_byte) = v[h];
  }
}

template <bool APPEND>
__global__ __launch_bounds__(256) void mla_wide_kernel(const MlaParams p) {
  constexpr int NT = 256;
  constexpr int H = kWideHeads;
  constexpr int add = APPEND ? 1 : 0;
  __shared__ u32x4 s_tile[kWideTiles][kWideTileAlloc];
  __shared__ u32x4 s_sink[64];
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
  // Byte offsets, within a block of 32 consecutive token rows in HBM, of the
  // chunks this lane loads with its kWideDmaPerWave instructions (tile chunk
  // c of row r = wide_row_of(c) is chunk c - wide_row_off(r) of the row; pad
  // chunks and the sink read a chunk of the block), two 16-bit offsets per
  // register (the largest is 31 * 1152 + 1136).
  uint32_t offp[kWideDmaPerWave / 2];
#pragma unroll
  for (int j = 0; j < kWideDmaPerWave / 2; ++j) {
    uint32_t v = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 64 * min(wave + 4 * (2 * j + h), kWideTileDma - 1) + lane;
      const int r = wide_row_of(c);
      const int x = min(c - wide_row_off(r), kWideRowData - 1);
      v |= (uint32_t)(r * (kMlaL * 2) + 16 * x) << (16 * h);
    }
    offp[j] = v;
  }
  // Per-lane part of the PV transposed reads: 16-lane group G = lane / 16
  // (k-slot half j2 = G / 2, column half ch = G % 2), lane 4 e + r of the
  // group addresses token row 4 j2 + e, columns 16 ch + 4 r .. + 3.
  const uint32_t v_lane = [&] {
    const int G = lane >> 4, e = (lane >> 2) & 3, r = lane & 3;
    return (uint32_t)(16 * wide_row_off(4 * (G >> 1) + e) + 2 * (16 * (G & 1) + 4 * r));
  }();

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
  if (tid == 0) s_redo = 0;  // read after the ring's barriers
  if (!plan.has_work) return;
  // The scores enter the softmax as q.k * sx with sx > 0: a negative scale
  // negates the queries instead (exact in bf16), and a zero scale becomes the
  // smallest normal float, whose products round every finite score to the
  // same probability while masked tokens stay -inf.
  const bool q_neg = p.scale_log2 < 0.f;
  const float sx = q_neg ? -p.scale_log2 : p.scale_log2 > 0.f ? p.scale_log2 : 1.17549435e-38f;
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

    // Pool token index of the first row of each of the segment's blocks, 64
    // at a time (lane l: block pid_base + l), read with readlane; a page id
    // outside the pool is clamped and marks the index with bit 31 (the loads
    // read the clamped page and the piece is NaN).
    int pid_base = 0;
    int m_tok = 0;
    int seg_bad = 0;
    auto fetch_pids = [&]() __attribute__((always_inline)) {
      const int t0 = t_begin + 32 * min(pid_base + lane, nblk - 1);
      const int page = t0 / p.page_size;
      const int raw = pt[page];
      const int pid = clamp_page(raw, p.num_pages);
      m_tok = (pid * p.page_size + (t0 - page * p.page_size)) |
              (raw == pid ? 0 : (int)0x80000000u);
    };
    fetch_pids();
    // The appended token is its sequence's last, so one segment holds it: that
    // segment's workgroup writes its row (c_new, pe_new) into the token's page
    // slot first, and every block then loads from the pool alike.
    const bool owner = APPEND && len_old >= t_begin && len_old < t_end;
    u32x4 new_chunk = {0u, 0u, 0u, 0u};
    int new_dst = -1;  // the row's pool token index, -1: not written here
    if (owner && tid < kWideRowData) {
      const int page = len_old / p.page_size;
      const int raw = pt[page];
      new_dst = clamp_page(raw, p.num_pages) == raw
                    ? raw * p.page_size + (len_old - page * p.page_size)
                    : -1;
      new_chunk = tid < kMlaC / 8
                      ? ((const u32x4*)(p.c_new + (size_t)b * p.c_stride))[tid]
                      : ((const u32x4*)(p.pe_new + (size_t)b * p.pe_stride))[tid - kMlaC / 8];
    }
    // Q^T of this wave's 32 heads: k-step u holds dims 16 u + 8 j2 .. + 8.
    // The q_nope rows come through LDS (the tiles are free here): one 1 KB
    // load instruction per row into a 65-chunk row slot (the read-back of
    // chunk 2 u + j2 of 32 rows then hits distinct banks), where per-lane
    // global loads would fetch 32 separate 32-byte pieces per instruction;
    // the q_pe chunks are loaded straight into registers.
    u32x4 qb[36];
    {
      const size_t qrow0 = (size_t)b * H + 32 * wave;
      const uint32_t qst = tile_base0 + (uint32_t)(32 * wave * 65 * 16);
#pragma unroll 8
      for (int h = 0; h < 32; ++h)
        wide_dma16_s(16 * lane, p.q_nope + (qrow0 + h) * kMlaC, qst + (uint32_t)(h * 65 * 16));
#pragma unroll
      for (int u = 32; u < 36; ++u)
        qb[u] = ((const u32x4*)(p.q_pe + (qrow0 + n32) * 64))[2 * (u - 32) + j2];
      asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
      if (new_dst >= 0) ((u32x4*)(p.latent_w + (size_t)new_dst * kMlaL))[tid] = new_chunk;
      const u32x4* qs = &s_tile[0][0] + (32 * wave + n32) * 65 + j2;
#pragma unroll
      for (int u = 0; u < 32; ++u) qb[u] = qs[2 * u];
      if (q_neg) {
#pragma unroll
        for (int u = 0; u < 36; ++u) qb[u] ^= 0x80008000u;
      }
    }
    // The queries are needed from the first block on: have them in registers
    // before the block loads go out (a wait the compiler placed at their
    // first use would also wait for every block load in flight), and every
    // wave done reading its rows before the loads overwrite them.
#pragma unroll
    for (int u = 0; u < 36; ++u) asm volatile("" : : "v"(qb[u]));
    // the appended row is in its page before any wave's loads of the block
    // go out (this wave's store done, then the barrier)
    if (owner) asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    wide_lds_barrier();

    // Block k of the segment into tile `slot`: this wave's 10 instructions
    // of 64 chunks.  Rows past t_end read the last valid row's last chunk
    // (each lane's offset clamped: finite values whose probabilities are 0);
    // a block past the segment's end reads q_nope (at least 128 KB) into a
    // tile no later block of the segment uses.
    struct Dma {
      const char* sb;   // the block's first row
      uint32_t wbase;   // this wave's part of the tile (LDS bytes)
      uint32_t d9;      // instruction 9's destination (tile or sink)
      uint32_t lim;     // offset clamp
    };
    auto issue_begin = [&](int k, int slot) __attribute__((always_inline)) {
      const bool valid = k < nblk;
      const int kc = min(k, nblk - 1);
      if (kc - pid_base >= 64) {
        pid_base += 64;
        fetch_pids();
      }
      const int tok_raw = __builtin_amdgcn_readlane(m_tok, kc - pid_base);
      seg_bad |= tok_raw;
      const uint32_t tok = (uint32_t)tok_raw & 0x7fffffffu;
      const int nt = t_end - (t_begin + 32 * kc);
      const uint32_t lim =
          nt >= 32 ? 0xffffu : (uint32_t)((nt - 1) * (kMlaL * 2) + 16 * (kWideRowData - 1));
      Dma d;
      d.sb = valid ? g0 + (size_t)tok * (kMlaL * 2) : (const char*)p.q_nope;
      d.lim = lim;
      const uint32_t tb = tile_base0 + (uint32_t)slot * (kWideTileAlloc * 16);
      d.wbase = tb + 1024 * wave;
      // a scalar select (the compiler makes a branch of the conditional)
      asm("s_cmp_eq_u32 %1, 0\n\ts_cselect_b32 %0, %2, %3"
          : "=s"(d.d9)
          : "s"(wave), "s"(tb + 1024 * (kWideTileDma - 1)), "s"(sink_base)
          : "scc");
      // recomputed per block (not hoisted)
      asm volatile("" : "+s"(d.wbase), "+s"(d.d9));
      return d;
    };
    // The offset pair of instructions 2 j and 2 j + 1 (offp[j]).
    auto dma_pair = [&](int j) __attribute__((always_inline)) {
      asm volatile("" : "+v"(offp[j]));  // unpacked at each use: five live registers
      return offp[j];
    };
    // Instruction i of a block (i a constant after unrolling), pr =
    // dma_pair(i / 2), its offset clamped.
    auto dma_one = [&](const Dma& d, uint32_t pr, int i) __attribute__((always_inline)) {
      const uint32_t off = min((i & 1) ? pr >> 16 : pr & 0xffffu, d.lim);
      if (i < kWideDmaPerWave - 1)
        wide_dma16_add(off, d.sb, d.wbase, 4 * 1024 * i);
      else
        wide_dma16_s(off, d.sb, d.d9);
    };
    auto issue = [&](int k, int slot) __attribute__((always_inline)) {
      const Dma d = issue_begin(k, slot);
      uint32_t pr = 0;
#pragma unroll
      for (int i = 0; i < kWideDmaPerWave; ++i) {
        if ((i & 1) == 0) pr = dma_pair(i >> 1);
        dma_one(d, pr, i);
      }
    };

    f32x16 acc[16];
    float m_run = neg_inf();  // reference max (m_ref) of the lane's head
    float m_max = neg_inf();  // the lane's largest score of the segment so far
    float l_run = 0.f;

    // Pieces of the ring (block k in tile k % 4):
    //   QK(k)    36 MFMAs into sc; A = row n32 of the tile, k-step u = chunk
    //            2 u + j2, each read four MFMAs ahead
    //   soft_x   log2-domain scores of a block (xa: the first PV k-step's,
    //            xh: the second's) and the lane's running max, which only
    //            feeds the headroom check, so no lanes are combined except to
    //            set m_run at the pass's first block
    //   soft_p   one dword of a k-step's P^T from its scores (two exp2
    //            against m_run)
    //   PV(k)    MFMA m (k-step m / 16, columns 32 (m % 16) ..) into
    //            accumulator m % 16, its V^T operand from two transposed reads
    //            (tokens 16 s + 8 t + 4 j2 + e, t = 0, 1) three MFMAs ahead
    const u32x4* arow0 = &s_tile[0][0] + wide_row_off(n32) + j2;
    auto qk_read = [&](int tile, int u) __attribute__((always_inline)) {
      return arow0[tile * kWideTileAlloc + 2 * u];
    };
    auto qk_mfma = [&](f32x16& sc, const u32x4& kr, int u) __attribute__((always_inline)) {
      if (u == 0)
        qk_first(sc, kr, qb[0]);
      else if (u == 35)
        qk_last(sc, kr, qb[35]);
      else
        qk_next(sc, kr, qb[u]);
    };
    // lane's V^T base in tile `tile`, opaque to the compiler (which would
    // otherwise keep a register per read offset instead of using the
    // instruction's offset field)
    auto vbase = [&](int tile) __attribute__((always_inline)) {
      uint32_t vl = v_lane;
      asm volatile("" : "+v"(vl));
      return tile_base0 + (uint32_t)tile * (kWideTileAlloc * 16) + vl;
    };
    auto vread = [&](uint32_t vt, int m) __attribute__((always_inline)) {
      const int sv = m >> 4, ct = m & 15;
      const uint32_t a = vt + 16 * kWideRowsS * sv + 64 * ct;
      const uint2 lo = lds_read_tr_b64(a);
      const uint2 hi = lds_read_tr_b64(a + 16 * kWideRowsT);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    };
    // the memory clobber keeps the operand reads where the source puts them
    auto pv_mfma = [&](const u32x4& va, const u32x4& pbs, int m) __attribute__((always_inline)) {
      f32x16& a = acc[m & 15];
      a = mfma32x32x16(va, pbs, a);
      asm volatile("" : "+a"(a));
      asm volatile("" : : : "memory");
    };
    // soft_x: the scores of a block as x = q.k * sx - m_run (xa: the first PV
    // k-step's, xh: the second's).  With sx > 0 the block's largest score is
    // sx times the largest raw score (v_max3 over the accumulator) and x is
    // one FMA per score; tokens past the end of a partial block are raw -inf.
    auto soft_x = [&](int kb, const f32x16& sc, float (&xa)[8], float (&xh)[8], bool first)
        __attribute__((always_inline)) {
      const int nt = min(32, t_end - (t_begin + 32 * kb));
      f32x16 v = sc;
      if (nt < 32) {  // accumulator i is token 8 (i / 4) + 4 j2 + i % 4
        int l = lane;  // recomputed here rather than kept live
        asm volatile("" : "+v"(l));
        const int lim = nt - 4 * (l >> 5);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 8 * (i >> 2) + (i & 3) < lim ? v[i] : neg_inf();
      }
      float r = v[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) r = fmaxf(r, v[i]);
      const float bm = r * sx;
      m_max = fmaxf(m_max, bm);
      // The pass's first block (first): m_run, unless a second pass set it,
      // becomes the head's largest score.  That block holds at least one
      // token, so for finite inputs m_run is finite from then on and later
      // blocks need not look.
      if (first) {
        float lo, hi;
        pair_xor32(bm, lo, hi);
        m_run = m_run == neg_inf() ? fmaxf(lo, hi) : m_run;
      }
      const float nm = -m_run;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        xa[i] = __builtin_fmaf(v[i], sx, nm);
        xh[i] = __builtin_fmaf(v[8 + i], sx, nm);
      }
    };
    // soft_p: one dword of a k-step's P^T (two exp2), its two probabilities
    // added to the row sum as rounded (the PV MFMAs see the same values)
    auto soft_p = [&](const float (&xs)[8], u32x4& pbs, int dd) __attribute__((always_inline)) {
      typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
      const uint32_t pk = pack_bf16x2(__builtin_amdgcn_exp2f(xs[2 * dd]),
                                      __builtin_amdgcn_exp2f(xs[2 * dd + 1]));
      pbs[dd] = pk;
      l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk),
                                              __builtin_bit_cast(bf16x2_t, 0x3f803f80u), l_run,
                                              false);
    };

    // Step kk of the ring, software-pipelined.  Block kk's scores (xa, xh)
    // come from the previous step.  The QK chain of block kk + 1 (36
    // MFMAs) runs with PV(kk) between its links: its first four links beside
    // the first k-step's probabilities (soft_p from xa), then 24 PV MFMAs,
    // three to every four links (the XDL unit alternates between the
    // independent PV MFMAs and the dependent QK chain), the second k-step's
    // probabilities beside PV's first k-step; soft_x of block kk + 1 runs
    // beside the last 8 PV MFMAs.  Block kk + 3's ten load instructions go
    // out over the chain into tile (kk + 3) % 4.  The step waits for block
    // kk + 1 (block kk + 2 may be in flight) and the barrier (every wave's
    // part of block kk + 1 is in, every wave is done with step kk - 1 and so
    // with tile (kk - 1) % 4 = (kk + 3) % 4).
    auto step = [&](int kk, float (&xa)[8], float (&xh)[8]) __attribute__((always_inline)) {
      const int tp = kk & (kWideTiles - 1), tq = (kk + 1) & (kWideTiles - 1);
      wide_wait_barrier<kWideDmaPerWave>();
      const Dma d = issue_begin(kk + 3, (kk + 3) & (kWideTiles - 1));
      f32x16 sc;
      u32x4 kr[5], va[4], pb[2];
      uint32_t pr = 0;
      const uint32_t vt = vbase(tp);
#pragma unroll
      for (int u = 0; u < 4; ++u) kr[u] = qk_read(tq, u);
#pragma unroll
      for (int m = 0; m < 3; ++m) va[m] = vread(vt, m);
#pragma unroll
      for (int u = 0; u < 36; ++u) {
        if (u + 4 < 36) kr[(u + 4) % 5] = qk_read(tq, u + 4);
        qk_mfma(sc, kr[u % 5], u);
        if (u < 4) {
          soft_p(xa, pb[0], u);
        } else if ((u - 4) % 4 != 3) {
          const int m = 3 * ((u - 4) / 4) + (u - 4) % 4;
          va[(m + 3) & 3] = vread(vt, m + 3);
          pv_mfma(va[m & 3], pb[m >> 4], m);
          if (m < 16 && (m & 3) == 1) soft_p(xh, pb[1], m >> 2);
        }
        if (u % 4 == 2) {  // instructions 0-8
          if ((u / 4) % 2 == 0) pr = dma_pair(u / 8);
          dma_one(d, pr, u / 4);
        }
      }
      soft_x(kk + 1, sc, xa, xh, false);
#pragma unroll
      for (int m = 24; m < 32; ++m) {
        if (m + 3 < 32) va[(m + 3) & 3] = vread(vt, m + 3);
        pv_mfma(va[m & 3], pb[1], m);
        if (m == 27) dma_one(d, pr, 9);
      }
    };
    // The pass's last block: PV only (its tile is in and synchronised).
    auto step_last = [&](int kk, const float (&xa)[8], const float (&xh)[8])
        __attribute__((always_inline)) {
      const uint32_t vt = vbase(kk & (kWideTiles - 1));
      u32x4 va[4], pb[2];
#pragma unroll
      for (int dd = 0; dd < 4; ++dd) soft_p(xa, pb[0], dd);
#pragma unroll
      for (int m = 0; m < 3; ++m) va[m] = vread(vt, m);
#pragma unroll
      for (int m = 0; m < 32; ++m) {
        if (m + 3 < 32) va[(m + 3) & 3] = vread(vt, m + 3);
        pv_mfma(va[m & 3], pb[m >> 4], m);
        if (m < 16 && (m & 3) == 1) soft_p(xh, pb[1], m >> 2);
      }
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
      float xa[8], xh[8];
      {  // QK and soft_x of block 0
        wide_wait_barrier<2 * kWideDmaPerWave>();
        f32x16 sc;
        u32x4 kr[5];
#pragma unroll
        for (int u = 0; u < 4; ++u) kr[u] = qk_read(0, u);
#pragma unroll
        for (int u = 0; u < 36; ++u) {
          if (u + 4 < 36) kr[(u + 4) % 5] = qk_read(0, u + 4);
          qk_mfma(sc, kr[u % 5], u);
        }
        soft_x(0, sc, xa, xh, true);
      }
#pragma clang loop unroll(disable)
      for (int k = 0; k + 1 < nblk; ++k) step(k, xa, xh);
      step_last(nblk - 1, xa, xh);
      {  // the head's largest score (both lanes of the head)
        float lo, hi;
        pair_xor32(m_max, lo, hi);
        m_max = fmaxf(lo, hi);
      }
      // every load of the pass has landed and every wave is done with the
      // tiles (a second pass, or the next segment, overwrites them)
      const bool climbed = __builtin_amdgcn_ballot_w64(m_max > m_run + kWideHeadroomLog2) != 0;
      if (climbed && lane == 0) s_redo = 1;
      wide_wait_barrier<0>();
      const bool redo = s_redo != 0;
      wide_wait_barrier<0>();  // every wave has read s_redo
      if (tid == 0) s_redo = 0;  // before the next vote, past the ring's barriers
      if (pass > 0 || !redo) break;
      // scores climbed out of the reference's headroom: again, with the
      // segment's maximum as the reference (no score exceeds it)
      m_run = m_max;
    }

    float lo, hi;
    pair_xor32(l_run, lo, hi);
    const float l_tot = lo + hi;
    const bool bad = seg_bad < 0;  // a bad page id was read (clamped): the piece is NaN
    const float inv_l = bad ? qnan() : 1.f / l_tot;
    const float lse_v = bad ? qnan() : (m_run + __log2f(l_tot)) * kLn2;
    const bool whole = row_start >= blk_begin && row_end <= blk_end;  // final, fp32
    if (j2 == 0) {
      if (whole)
        p.lse[(size_t)b * H + head] = lse_v;
      else
        p.part_lse[(size_t)(g + b) * H + head] = lse_v;
    }
    // The outputs leave through LDS (the tiles are free: every wave is past
    // the pass's last barrier), so that each store instruction writes one
    // contiguous 1 KB row: wave w stages its 32 rows (row stride 260 dwords:
    // the row reads and the fp32 writes hit distinct banks, the bf16 writes
    // two lanes per bank pair) and stores them itself.  Accumulator ct value
    // i is column 32 ct + 8 (i / 4) + 4 j2 + i % 4.
    uint32_t* stage = (uint32_t*)&s_tile[0][0] + (size_t)(32 * wave) * 260;
    if (!whole) {  // bf16 piece: all 512 columns at once
#pragma unroll
      for (int ct = 0; ct < 16; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *(uint2*)(stage + n32 * 260 + 16 * ct + 4 * q + 2 * j2) =
              make_uint2(pack_bf16x2(acc[ct][4 * q] * inv_l, acc[ct][4 * q + 1] * inv_l),
                         pack_bf16x2(acc[ct][4 * q + 2] * inv_l, acc[ct][4 * q + 3] * inv_l));
      wide_lds_wait();  // this wave's rows are in LDS
      char* dst = (char*)(p.part_out + ((size_t)(g + b) * H + 32 * wave) * kMlaC);
      wide_store_rows(dst, kMlaC * 2, stage + 4 * lane, 16 * lane);
    } else {  // fp32 final: two halves of 256 columns
      char* dst = (char*)(p.out + ((size_t)b * H + 32 * wave) * kMlaC);
#pragma unroll
      for (int hc = 0; hc < 2; ++hc) {
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int ct = 8 * hc + c8;
            *(float4*)(stage + n32 * 260 + 32 * c8 + 8 * q + 4 * j2) =
                make_float4(acc[ct][4 * q] * inv_l, acc[ct][4 * q + 1] * inv_l,
                            acc[ct][4 * q + 2] * inv_l, acc[ct][4 * q + 3] * inv_l);
          }
        wide_lds_wait();
        wide_store_rows(dst, kMlaC * 4, stage + 4 * lane, 1024 * hc + 16 * lane);
        wide_lds_wait();  // the next half overwrites the rows
      }
    }
    // the next segment's loads overwrite the tiles: every wave's stores
    // have read their rows
    wide_lds_barrier();
    blk = seg_end;
  }
}

}  // namespace ws
