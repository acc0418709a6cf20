/*
 * wsgpu.h — C ABI of the MI355X (gfx950) GPU partition of a physically
 * partitioned decode KV cache.
 *
 * The library (scope_amd/lib/libwsgpu.so) holds the GPU side of a decode step
 * whose KV tokens are split between host memory and HBM:
 *
 *   ws_kv_append / ws_latent_append   write the new token(s) of every sequence
 *                                     into its HBM page (bit copies)
 *   ws_gqa_decode_partial             split-KV GQA decode attention over the
 *                                     HBM tokens -> (out, lse) per query head
 *   ws_mla_decode_partial             the same for the absorbed MLA layout
 *                                     (576-wide shared latent, 512-wide out)
 *   ws_split_reduce                   LSE-combine per-split partials
 *   ws_lse_merge                      combine the GPU partial with the host
 *                                     partial (any of the reference's partial
 *                                     formats) and normalise
 *
 * Conventions
 *   - bf16 tensors are passed as uint16_t bit patterns; fp32 as float.
 *   - A "partial" is (out, lse): out is the softmax-normalised attention
 *     output over the partition's tokens, lse = max + log(sum) in natural log.
 *     An empty partition is (0, -inf).  The reference triple
 *     (o_unnormalised, max, sum) maps to it by out = o / sum,
 *     lse = max + log(sum).
 *   - Paged layout: a page holds page_size consecutive tokens of one sequence.
 *       GQA pools  k_pages, v_pages : [num_pages][Hkv][page_size][D]  bf16
 *       MLA pool   latent_pages     : [num_pages][page_size][576]     bf16
 *                                     (512 latent c_kv followed by 64 rope k_pe)
 *     page_table : [B][max_pages] int32 physical page ids,
 *     gpu_len    : [B] int32 number of tokens of sequence b in the pool.
 *     Token t of sequence b lives in page page_table[b][t / page_size] at
 *     offset t % page_size.  A contiguous [N][S][D] buffer is the special
 *     case Hkv = 1, page_size = S, num_pages = N, page_table[n][0] = n.
 *   - Row order follows the reference: GQA query head h = kvh * G + g,
 *     out index [b][h][d]; MLA row b * H + h.
 *   - Every entry point is stream-ordered on `stream` (a hipStream_t; NULL is
 *     the default stream) and allocates nothing.  None keeps global mutable
 *     state except ws_gqa_append_decode_partial_noalloc (its static scratch).
 *     Device pointers are not dereferenced on the host.
 *   - Return value: 0 on success, a negative WS_E* code on a bad argument or a
 *     failed launch; ws_last_error() then describes it (thread-local string).
 */
#ifndef WSGPU_H
#define WSGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WS_OK 0
#define WS_EINVAL (-1)   /* argument out of range / null pointer           */
#define WS_ELAUNCH (-2)  /* kernel launch failed                            */
#define WS_EWORKSPACE (-3) /* workspace too small                           */

/* Formats of the second operand of ws_lse_merge (the host partial). */
#define WS_PARTIAL_LSE_F32 0      /* (out normalised fp32, lse fp32)               */
#define WS_TRIPLE_UNNORM_F32 1    /* (out unnormalised fp32, max fp32, sum fp32):
                                     fused_cpu_attn_mla / _mla_compressed / the
                                     fp32 path of fused_cpu_attn without normalise */
#define WS_TRIPLE_NORM_BF16 2     /* (out normalised bf16, max bf16, sum bf16):
                                     bf16 path of fused_cpu_attn                 */
#define WS_TRIPLE_NORM_F32 3      /* (out normalised fp32, max fp32, sum fp32):
                                     fp32 path of fused_cpu_attn                 */
#define WS_PARTIAL_LSE_BF16 4     /* (out normalised bf16, lse fp32): the native
                                     host partial's bf16 output (wshost.h
                                     wh_*_partial_bf16), half the bytes for a
                                     merge that reads it across the host link */

const char* ws_last_error(void);
const char* ws_version(void);

/*
 * Copy `bytes` (a multiple of 4) from src to dst with a copy kernel on
 * `stream`; either side may be device memory or pinned host memory
 * (hipHostMalloc, mapped into the device's address space), so it moves a
 * decode step's query to the host partial without a DMA copy's set-up
 * latency.  16-byte aligned pointers, no overlap.  Replaces the query's
 * .cpu() of the two-sided layer (system/deepseek.py:345-346,
 * system/mixoffload.py:1328).  (The host partial needs no copy back: the
 * merges read their host operand from pinned host memory in place.)
 */
int ws_copy(void* dst, const void* src, size_t bytes, void* stream);

/*
 * Page copies of a boundary move, every layer at once: for l < n_layers and
 * i < n_pages, page dst_ids[i] of dst + l * dst_layer_stride = page
 * src_ids[i] of src + l * src_layer_stride (pages of page_bytes, a multiple
 * of 16; strides in bytes).  Either pool may be HBM or pinned host memory:
 * the kernel reads and writes across the host link itself, with no host-side
 * gather and no staging copy.  dst_ids / src_ids: n_pages int32 each in
 * device-accessible memory, inside [0, dst_num_pages) / [0, src_num_pages)
 * (an id outside moves nothing).  Replaces the reference's movement of
 * tokens across the split: the host-segment tokens past the GPU share that
 * every step copies to the GPU (system/deepseek.py:368-371) and the GPU
 * segment's .to(device) (system/mixoffload.py:1369-1370); here a share change
 * moves whole pages once.  max_workgroups bounds the grid (0: a default of
 * 2048); a copy across the host link is bound by the link, and a few dozen
 * workgroups keep it busy while leaving the CUs to kernels that run beside
 * it on another stream.
 */
int ws_copy_pages(void* dst, long long dst_layer_stride, const int32_t* dst_ids,
                  int dst_num_pages, const void* src, long long src_layer_stride,
                  const int32_t* src_ids, int src_num_pages, int n_pages, int n_layers,
                  long long page_bytes, int max_workgroups, void* stream);

/*
 * Append n_new tokens per sequence to the GQA pools at positions
 * gpu_len[b] .. gpu_len[b] + n_new - 1, then (if update_len) gpu_len[b] += n_new.
 * k_new, v_new: [B][Hkv][n_new][D] bf16 (the reference's k4d/v4d layout).
 * Pages for the new positions must already be in page_table.
 * Replaces InplaceKVCache.append_4d (system/qwenoffload.py:100-118,
 * system/mixoffload.py:85-104) and the slot copy of _resident_layer
 * (roofline/bench_resident_kv.py:268-269) for the HBM partition.
 */
int ws_kv_append(const uint16_t* k_new, const uint16_t* v_new,
                 uint16_t* k_pages, uint16_t* v_pages,
                 const int32_t* page_table, int32_t* gpu_len,
                 int B, int Hkv, int D, int n_new,
                 int page_size, int max_pages, int num_pages,
                 int update_len, void* stream);

/*
 * Append n_new latent tokens per sequence to the MLA pool.
 * c_new: [B][n_new][512] bf16 (row stride c_stride elements),
 * pe_new: [B][n_new][64] bf16 (row stride pe_stride elements).
 * Replaces the GPU-segment half of InplaceKVCacheCompressed.append
 * (system/deepseek.py:171-192; boundary arithmetic 181-188 stays on the host).
 */
int ws_latent_append(const uint16_t* c_new, int64_t c_stride,
                     const uint16_t* pe_new, int64_t pe_stride,
                     uint16_t* latent_pages,
                     const int32_t* page_table, int32_t* gpu_len,
                     int B, int n_new, int page_size, int max_pages,
                     int num_pages, int update_len, void* stream);

/*
 * Plan of a decode call: kind 0 (GQA: rows_kv = B * Hkv, heads = the group
 * size G) or 1 (MLA: rows_kv = B, heads = H, a multiple of 16; H = 128 with B <= 64
 * plans sequences with 128-head pieces, other H 16-head groups), over sequences of at most
 * max_len tokens.  n_splits is the number of pieces the call cuts its work
 * into: one per wave for GQA (two per workgroup, each streaming on its
 * own), one per workgroup for MLA.  0 = the library's choice for the current
 * device: two GQA waves (one workgroup) or one MLA workgroup per CU, fewer
 * when the batch is small (a GQA split keeps at least two 32-token blocks).  Writes the resolved split count and the
 * workspace bytes the call needs; the same count goes to ws_merge_split.
 *
 * Splits take equal shares of all 32-token blocks of all rows, so ragged
 * batches stay balanced; a row shared by several splits is combined from
 * their partials.  Workspace layout: [partial lse fp32, padded to 256
 * bytes][partial out bf16], one partial slot per (split, row) pair.  The
 * workspace must be 256-byte aligned; it needs no initial contents (every
 * call writes the slots it reads back).  Calls that share a workspace must
 * be ordered on one stream.  At most 2048 sequences and 4096 splits per
 * call.
 */
int ws_decode_plan(int kind, int rows_kv, int heads, int max_len,
                   int n_splits, int* n_splits_out,
                   size_t* workspace_bytes_out);

/*
 * ws_decode_plan kind 0 for key width Dk and value width Dv (the widths
 * ws_attn_decode_partial takes; kind 0 sizes the workspace for Dv = 128):
 * rows_kv = B * Hkv, heads = the group size G.  The reference sizes nothing
 * here (its GPU partial is a torch bmm with allocated outputs,
 * roofline/bench_resident_kv.py:150-157); this is the workspace query of
 * the calls below at widths other than 128.
 */
int ws_attn_decode_plan(int rows_kv, int heads, int Dk, int Dv, int max_len,
                        int n_splits, int* n_splits_out,
                        size_t* workspace_bytes_out);

/*
 * Split-KV GQA decode attention over the pooled tokens of every sequence.
 * q: [B][Hq][D] bf16, Hq = Hkv * G, G from 1 to 16, D a multiple of 16 up
 * to 256 (the reference's bmm takes any width; its CPU kernel any multiple of
 * 16, kernel/cpu_attn.cpp:583).  Workspace: ws_decode_plan kind 0 for
 * D = 128, ws_attn_decode_plan for any D.
 * n_splits: waves of the plan (0 = choose, see ws_decode_plan); max_len:
 * upper bound of gpu_len[] (must be >= every gpu_len[b]).  Rows held by one
 * wave are written final by the streaming launch; rows spread over several
 * waves are combined from their workspace partials by a second, small launch
 * on the same stream (the split merge of ws_merge_split without a host
 * partial).
 * Outputs out: [B][Hq][D] fp32 normalised, lse: [B][Hq] fp32.
 * Replaces _local_bmm_softmax / _resident_layer
 * (roofline/bench_resident_kv.py:150-157, 261-271) and the GPU side of
 * _compute_pipelined_attention (system/mixoffload.py:1389-1447).
 */
int ws_gqa_decode_partial(const uint16_t* q,
                          const uint16_t* k_pages, const uint16_t* v_pages,
                          const int32_t* page_table, const int32_t* gpu_len,
                          int B, int Hq, int Hkv, int D,
                          int page_size, int max_pages, int num_pages,
                          int max_len, int n_splits, float scale,
                          float* out, float* lse,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * One decode step of the GPU partition in one launch: append the new token of
 * every sequence and attend over the partition including it.
 * k_new, v_new: [B][Hkv][1][D] bf16.  Token len_in[b] of sequence b is the new
 * one: it is written into its page slot (page_table must already hold that
 * page) and attended from k_new/v_new directly; len_out[b] = len_in[b] + 1
 * when len_out is not NULL (len_out must not alias len_in: a cache keeps two
 * length arrays and swaps them each step).  max_len must be >= every
 * len_in[b] + 1.  Other arguments and outputs as ws_gqa_decode_partial.
 * Replaces _resident_layer (roofline/bench_resident_kv.py:261-271): slot copy
 * + attention over the resident buffer; equivalent to ws_kv_append followed by
 * ws_gqa_decode_partial.
 */
int ws_gqa_append_decode_partial(const uint16_t* q, const uint16_t* k_new,
                                 const uint16_t* v_new, uint16_t* k_pages,
                                 uint16_t* v_pages, const int32_t* page_table,
                                 const int32_t* len_in, int32_t* len_out,
                                 int B, int Hq, int Hkv, int D,
                                 int page_size, int max_pages, int num_pages,
                                 int max_len, int n_splits, float scale,
                                 float* out, float* lse,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/*
 * The whole decode step of a GPU partition that holds every token (share
 * r = 1, no host partial): ws_gqa_append_decode_partial that also writes the
 * normalised output in bf16 (its combine launch writes both).  out_bf16
 * [B][Hq][D] bf16, out [B][Hq][D] fp32 and lse [B][Hq] fp32 are all
 * required.
 * Replaces _resident_layer followed by the final o / sum and bf16 cast when
 * the host share is empty (roofline/bench_resident_kv.py:261-271, 350;
 * system/mixoffload.py:1477-1480).
 */
int ws_gqa_append_decode_full(const uint16_t* q, const uint16_t* k_new,
                              const uint16_t* v_new, uint16_t* k_pages,
                              uint16_t* v_pages, const int32_t* page_table,
                              const int32_t* len_in, int32_t* len_out,
                              int B, int Hq, int Hkv, int D,
                              int page_size, int max_pages, int num_pages,
                              int max_len, int n_splits, float scale,
                              uint16_t* out_bf16, float* out, float* lse,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * Deferred-combine form of ws_gqa_append_decode_partial, for a step whose
 * partial is merged with a host partial anyway: one launch, the streaming
 * one.  Rows that one wave held are written final to out/lse, rows spread
 * over several waves leave their partials in the workspace, and
 * ws_merge_split combines them with the host partial in the merge launch.
 * The workspace must not be reused until the matching ws_merge_split ran.
 */
int ws_gqa_append_decode_split(const uint16_t* q, const uint16_t* k_new,
                               const uint16_t* v_new, uint16_t* k_pages,
                               uint16_t* v_pages, const int32_t* page_table,
                               const int32_t* len_in, int32_t* len_out,
                               int B, int Hq, int Hkv, int D,
                               int page_size, int max_pages, int num_pages,
                               int max_len, int n_splits, float scale,
                               float* out, float* lse,
                               void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * ws_gqa_decode_partial / ws_gqa_append_decode_partial with separate key and
 * value widths: k_pages [num_pages][Hkv][page_size][Dk], v_pages
 * [num_pages][Hkv][page_size][Dv], q [B][Hq][Dk], k_new [B][Hkv][1][Dk],
 * v_new [B][Hkv][1][Dv], out [B][Hq][Dv].  Dk == Dv, a multiple of 16 up
 * to 256, is the GQA call; (192, 128) with group size 1 is the decompressed
 * DeepSeek-V2 attention (128 nope + 64 rope key columns, 128 value columns,
 * 16 heads).  Workspace from ws_attn_decode_plan.
 * Replaces _local_bmm_softmax / _resident_layer with the reference's ds2
 * model entry, QHD 192 / VHD 128 / GROUPS 1 (roofline/bench_resident_kv.py:10,
 * 150-157, 261-271), the GPU side of the fused_cpu_attn_mla split
 * (kernel/cpu_attn.cpp:638-672).
 */
int ws_attn_decode_partial(const uint16_t* q, const uint16_t* k_pages,
                           const uint16_t* v_pages, const int32_t* page_table,
                           const int32_t* gpu_len, int B, int Hq, int Hkv,
                           int Dk, int Dv, int page_size, int max_pages,
                           int num_pages, int max_len, int n_splits, float scale,
                           float* out, float* lse, void* workspace,
                           size_t workspace_bytes, void* stream);
int ws_attn_append_decode_partial(const uint16_t* q, const uint16_t* k_new,
                                  const uint16_t* v_new, uint16_t* k_pages,
                                  uint16_t* v_pages, const int32_t* page_table,
                                  const int32_t* len_in, int32_t* len_out,
                                  int B, int Hq, int Hkv, int Dk, int Dv,
                                  int page_size, int max_pages, int num_pages,
                                  int max_len, int n_splits, float scale,
                                  float* out, float* lse, void* workspace,
                                  size_t workspace_bytes, void* stream);

/*
 * Split-KV absorbed-MLA decode attention.
 * q_nope: [B*H][512] bf16 (q_nope already multiplied by W_UK), q_pe: [B*H][64].
 * score = (q_nope . c + q_pe . pe) * scale over the shared 576-wide latent,
 * out = softmax . c (512-wide).  H: any multiple of 16 (16 for
 * DeepSeek-V2-Lite, 128 for DeepSeek-V2; nH = q rows / B as in
 * kernel/cpu_attn.cpp:860).  H = 128 with B <= 64 runs one pass over each
 * latent block for all 128 heads (a workgroup of four 32-head waves, pieces of
 * 128 heads); other H plan each group of 16 heads as a sequence of its own
 * over the shared latent.  A sequence's new latent is written once.
 * Outputs out: [B*H][512] fp32 normalised, lse: [B*H] fp32.
 * Replaces the GPU partial of _mla_compressed_forward
 * (system/deepseek.py:364-392; also roofline/bench_rstar_revalidate_ds2.py:74-86).
 */
int ws_mla_decode_partial(const uint16_t* q_nope, const uint16_t* q_pe,
                          const uint16_t* latent_pages,
                          const int32_t* page_table, const int32_t* gpu_len,
                          int B, int H, int page_size, int max_pages,
                          int num_pages, int max_len, int n_workgroups,
                          float scale, float* out, float* lse,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * One absorbed-MLA decode step of the GPU partition in one call: append the
 * new latent of every sequence (c_new [B] rows of 512, row stride c_stride;
 * pe_new [B] rows of 64, row stride pe_stride; bf16) at position len_in[b]
 * and attend over the partition including it; len_out[b] = len_in[b] + 1
 * when len_out is not NULL (must not alias len_in).  max_len must be >= every
 * len_in[b] + 1.  Replaces the GPU-segment append of
 * InplaceKVCacheCompressed.append (system/deepseek.py:171-192) followed by
 * the GPU partial of _mla_compressed_forward (system/deepseek.py:364-392).
 */
int ws_mla_append_decode_partial(const uint16_t* q_nope, const uint16_t* q_pe,
                                 const uint16_t* c_new, int64_t c_stride,
                                 const uint16_t* pe_new, int64_t pe_stride,
                                 uint16_t* latent_pages,
                                 const int32_t* page_table,
                                 const int32_t* len_in, int32_t* len_out,
                                 int B, int H, int page_size, int max_pages,
                                 int num_pages, int max_len,
                                 int n_workgroups, float scale,
                                 float* out, float* lse,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Deferred-combine form of ws_mla_append_decode_partial (see
 * ws_gqa_append_decode_split); finish with ws_merge_split. */
int ws_mla_append_decode_split(const uint16_t* q_nope, const uint16_t* q_pe,
                               const uint16_t* c_new, int64_t c_stride,
                               const uint16_t* pe_new, int64_t pe_stride,
                               uint16_t* latent_pages,
                               const int32_t* page_table,
                               const int32_t* len_in, int32_t* len_out,
                               int B, int H, int page_size, int max_pages,
                               int num_pages, int max_len,
                               int n_workgroups, float scale,
                               float* out, float* lse,
                               void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * Finish a deferred-combine step: for every output row, LSE-combine the GPU
 * pieces the step left (its final out/lse, or the partials of the
 * splits that shared the row) with the host partial, normalise, and
 * write out_bf16 and/or out_f32 [rows][Dv] and lse_out [rows] (any may be
 * NULL but not both outputs).
 *   gpu_len          the lengths after the step (the step's len_out)
 *   rows_per_seq     Hkv (GQA) or 1 (MLA); heads: G (GQA) or H (MLA, a
 *                    multiple of 16)
 *   Dv               128 (GQA) or 512 (MLA)
 *   page_capacity    page_size * max_pages of the step
 *   n_splits         the split count the step ran with (ws_decode_plan)
 *   out_g, lse_g     the step's out / lse; workspace as given to the step
 *   b_*, fmt_b       host partial as in ws_lse_merge, or b_out = NULL for none
 * rows = B * rows_per_seq * heads, ordered as the step's out.
 * Replaces the merge of the CPU and GPU partials after a decode step
 * (system/deepseek.py:394-403, system/mixoffload.py:1452-1464,
 * roofline/bench_resident_kv.py:339-350) together with the split combine.
 */
int ws_merge_split(const int32_t* gpu_len, int B, int rows_per_seq, int heads,
                   int Dv, int page_capacity, int n_splits,
                   const float* out_g, const float* lse_g,
                   const void* workspace, size_t workspace_bytes,
                   const void* b_out, const void* b_aux0, const void* b_aux1,
                   int fmt_b, uint16_t* out_bf16, float* out_f32,
                   float* lse_out, void* stream);

/*
 * ws_merge_split for an absorbed-MLA step (rows_per_seq 1, Dv 512) fused with
 * the W_UV epilogue: each merged row (b, h) is normalised, rounded to bf16
 * and multiplied by W_UV[h]^T, giving out_v [B][heads * Dout] bf16, the
 * attention output in the layout o_proj takes.
 *   w_uv       [heads][Dout][512] bf16 (the value half of kv_b_proj's weight,
 *              system/deepseek.py:256-260); Dout a multiple of 32, <= 512
 *   out_latent [B * heads][512] bf16 merged latent, or NULL
 *   lse_out    [B * heads] or NULL
 * Other arguments as ws_merge_split (rows_per_seq 1, Dv 512).
 * Replaces the merge + normalise + bf16 cast + W_UV bmm of the MLA decode
 * branch (system/deepseek.py:397-407) in one launch.
 */
int ws_mla_merge_split_uv(const int32_t* gpu_len, int B, int heads, int page_capacity,
                          int n_splits, const float* out_g, const float* lse_g,
                          const void* workspace, size_t workspace_bytes,
                          const void* b_out, const void* b_aux0, const void* b_aux1,
                          int fmt_b, const uint16_t* w_uv, int Dout, uint16_t* out_latent,
                          uint16_t* out_v, float* lse_out, void* stream);

/*
 * LSE-combine per-split partials: part_out [n_splits][rows][Dv],
 * part_lse [n_splits][rows] -> out [rows][Dv], lse [rows].  Split s of a row
 * takes part in the merge iff s < n_valid[row / heads_per_len] where
 * n_valid = ceil(len / tokens_per_split) for len = gpu_len[row / heads_per_len].
 * Rows with n_valid <= 1 are left untouched unless n_valid == 0, which writes
 * (0, -inf).  Used internally by the decode entry points; exported for callers
 * that schedule their own splits.
 * Replaces the running merge of _pingpong_stream
 * (roofline/bench_resident_kv.py:188-201).
 */
int ws_split_reduce(const float* part_out, const float* part_lse,
                    const int32_t* gpu_len, int rows, int heads_per_len,
                    int Dv, int n_splits, int tokens_per_split,
                    float* out, float* lse, void* stream);

/*
 * Merge the GPU partial (out_g, lse_g) with a second partial in format fmt_b
 * (WS_PARTIAL_LSE_F32 / _BF16: b_out fp32 / bf16, b_aux0 = lse fp32;
 * WS_TRIPLE_*: b_aux0 = max, b_aux1 = sum, dtype per format), over rows x Dv.  The b_* operands
 * may be in pinned host memory (hipHostMalloc): the kernel reads them over
 * the host link in place, so a host partial needs no copy to HBM first
 * (the same holds for ws_merge_split and ws_mla_merge_split_uv).
 * Writes any non-null of out_bf16 [rows][Dv], out_f32 [rows][Dv], lse_out
 * [rows].  Empty + empty gives out 0, lse -inf.
 * Replaces _pairwise_merge + the final normalise
 * (roofline/bench_resident_kv.py:141-148, 345-350), the MLA merge
 * (system/deepseek.py:394-403) and the GQA token-split merge with its CPU
 * un-normalise (system/mixoffload.py:1334, 1452-1464).
 */
int ws_lse_merge(const float* out_g, const float* lse_g,
                 const void* b_out, const void* b_aux0, const void* b_aux1,
                 int fmt_b, uint16_t* out_bf16, float* out_f32,
                 float* lse_out, int rows, int Dv, void* stream);

/*
 * ws_gqa_append_decode_partial for callers that cannot allocate device
 * memory: no counterpart in the reference (its decode step allocates through
 * torch); it is for code under HIP graph capture and serving loops that
 * forbid hipMalloc.  Same arguments and results as
 * ws_gqa_append_decode_partial without the workspace: the split pieces live
 * in a static device array of ws_noalloc_scratch_bytes() (8 MiB) per GPU,
 * held until the process ends.  A call whose plan needs more returns
 * WS_EWORKSPACE before launching anything.  The call allocates nothing (no
 * hipMalloc, no library allocation); its first call on a device looks up the
 * array's address there (hipGetSymbolAddress, which is not a capturable
 * operation), so that first call must come before any graph capture on the
 * device; later calls capture as plain kernel nodes.  Every call on one GPU
 * shares that GPU's array:
 * calls that overlap on one GPU (other streams, unordered threads) race;
 * calls ordered on one stream do not.  The array needs no initial contents.
 */
size_t ws_noalloc_scratch_bytes(void);
int ws_gqa_append_decode_partial_noalloc(const uint16_t* q, const uint16_t* k_new,
                                         const uint16_t* v_new, uint16_t* k_pages,
                                         uint16_t* v_pages, const int32_t* page_table,
                                         const int32_t* len_in, int32_t* len_out,
                                         int B, int Hq, int Hkv, int D,
                                         int page_size, int max_pages, int num_pages,
                                         int max_len, int n_splits, float scale,
                                         float* out, float* lse, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WSGPU_H */
