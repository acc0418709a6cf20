/* wshost.h - C ABI of libwshost.so, the host partial of the partitioned
 * decode KV cache: attention over the host segment of every sequence,
 * computed on the CPU while the GPU partition attends its own share.
 *
 * The host segment is paged exactly like the GPU partition (include/wsgpu.h):
 * the same pool layouts, page table and lengths, so moving the partition
 * boundary is a copy of whole pages between the two pools.  The reference's
 * dense host caches ([B*Hkv, S, D] for GQA, [B, S, 512] + [B, S, 64] for MLA,
 * system/qwenoffload.py:100-132, system/deepseek.py:161-166) are the case of
 * one page per sequence: page_size = S, max_pages = 1, page_table[b] = b.
 *
 * Outputs are the normalised fp32 partial and its natural-log LSE, the
 * (out, lse) form that ws_lse_merge / ws_merge_split take as format
 * WS_PARTIAL_LSE_F32, so no un-normalise step sits between the two.  An empty
 * host segment gives out = 0, lse = -inf (the merge identity).
 *
 * Unlike the reference CPU kernels, which take one length for every row of a
 * call (kernel/cpu_attn.cpp:590, 861), every sequence here has its own
 * length, so a ragged batch is one call (no per-sequence loop, no padding).
 * All 32-token blocks of all rows are split evenly over the threads; a row
 * split across threads is combined by LSE after a barrier.
 *
 * Page size: a multiple of 32, or any size when max_pages is 1.  Every page
 * id a length reaches must lie in [0, num_pages): it is checked before any
 * work and a bad id is an error (nothing is clamped).  Calls are
 * synchronous, allocate only per-call scratch and keep no state between
 * calls; concurrent calls from different threads are safe.  Python callers
 * via ctypes release the GIL for the duration of a call.
 */
#ifndef WSHOST_H
#define WSHOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WH_OK 0
#define WH_EINVAL (-1)  /* bad argument: see wh_last_error() */
#define WH_ENOTSUP (-2) /* this CPU lacks AVX-512 F/BW/BF16 */

/* Message of the last failed call on this thread ("" when none). */
const char* wh_last_error(void);

/* Library version string. */
const char* wh_version(void);

/* 1 when this CPU runs the kernels (AVX-512 F, BW and BF16), else 0. */
int wh_isa_supported(void);

/* GQA host partial.
 * Replaces the per-sequence calls of fused_cpu_attn / fused_cpu_attn_mla
 * (kernel/cpu_attn.cpp:572-672) made by the token-split decode flows
 * (system/mixoffload.py:1324-1335, roofline/bench_resident_kv.py:129-133).
 *   q          [B, Hq, D] bf16; query head kvh*G + g (G = Hq / Hkv) reads
 *              KV head kvh, the row order of system/qwenoffload.py:1367
 *   k_pages,   [num_pages, Hkv, page_size, D] bf16 pools
 *   v_pages
 *   page_table [B, max_pages] int32; token t of sequence b is in page
 *              page_table[b][t / page_size] at offset t % page_size
 *   lens       [B] int32 host tokens, 0 <= lens[b] <= max_pages * page_size
 *   out        [B, Hq, D] fp32 normalised partial; lse [B, Hq] fp32
 * D: a multiple of 16 up to 256; G: 1..16.  n_threads <= 0: the OpenMP
 * default.  Returns WH_OK or a negative WH_E* code. */
int wh_gqa_partial(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                   const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                   int D, int page_size, int max_pages, int num_pages, float scale,
                   float* out, float* lse, int n_threads);

/* wh_gqa_partial writing out as bf16 (rounded to nearest even), lse fp32:
 * the (out, lse) pair the GPU merges take as WS_PARTIAL_LSE_BF16, half the
 * bytes of the fp32 out for a merge that reads it across the host link.
 * (fused_cpu_attn's own bf16 path, kernel/cpu_attn.cpp:631-634, rounds max
 * and sum to bf16 as well; here the lse stays fp32.) */
int wh_gqa_partial_bf16(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                        const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                        int D, int page_size, int max_pages, int num_pages, float scale,
                        uint16_t* out, float* lse, int n_threads);

/* wh_gqa_partial with separate key and value widths: q [B, Hq, Dk],
 * k_pages [num_pages, Hkv, page_size, Dk], v_pages [num_pages, Hkv,
 * page_size, Dv], out [B, Hq, Dv].  (Dk, Dv): equal multiples of 16 up to 256,
 * or (192, 128), the decompressed DeepSeek-V2 layout (128 nope + 64 rope key
 * columns, 128 value columns; the reference's ds2 model entry,
 * roofline/bench_resident_kv.py:10).
 * Replaces fused_cpu_attn_mla with Dk != Dv (kernel/cpu_attn.cpp:638-672),
 * returning (out, lse) instead of its unnormalised triple. */
int wh_attn_partial(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                    const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                    int Dk, int Dv, int page_size, int max_pages, int num_pages, float scale,
                    float* out, float* lse, int n_threads);

/* wh_attn_partial over fp32 q and K / V pools (same shapes, float), fp32
 * FMAs with fp32 probabilities.  (Dk, Dv): equal multiples of 16 up to 256,
 * or (192, 128).
 * Replaces the float32 path of fused_cpu_attn (kernel/cpu_attn.cpp:572-636)
 * and fused_cpu_attn_fp32 (kernel/cpu_attn.cpp:817-848), both of which
 * return the normalised out with (max, sum); returns (out, lse). */
int wh_attn_partial_f32(const float* q, const float* k_pages, const float* v_pages,
                        const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                        int Dk, int Dv, int page_size, int max_pages, int num_pages,
                        float scale, float* out, float* lse, int n_threads);

/* The reference CPU kernel's own triple: wh_attn_partial / _f32 returning
 * fp32 (out [B, Hq, Dv], row_max [B, Hq], row_sum [B, Hq]) instead of
 * (out, lse).  row_max is the largest scaled score q.k * scale of the row,
 * row_sum the sum of exp(q.k * scale - row_max), and out is divided by
 * row_sum when `normalize` is nonzero, else left as the weighted sum.  These
 * are the outputs of fused_cpu_attn (normalised; kernel/cpu_attn.cpp:540-567,
 * 628-635), fused_cpu_attn_fp32 (normalised; :817-848) and
 * fused_cpu_attn_mla (unnormalised; :638-672).  An empty row gives out = 0,
 * row_max = -inf, row_sum = 0. */
int wh_attn_triple(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                   const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                   int Dk, int Dv, int page_size, int max_pages, int num_pages, float scale,
                   int normalize, float* out, float* row_max, float* row_sum, int n_threads);
int wh_attn_triple_f32(const float* q, const float* k_pages, const float* v_pages,
                       const int32_t* page_table, const int32_t* lens, int B, int Hq, int Hkv,
                       int Dk, int Dv, int page_size, int max_pages, int num_pages, float scale,
                       int normalize, float* out, float* row_max, float* row_sum,
                       int n_threads);

/* Absorbed-MLA host partial (H heads, a multiple of 16: 16 for
 * DeepSeek-V2-Lite, 128 for DeepSeek-V2; 512-wide latent + 64-wide rope key).
 * Replaces fused_cpu_attn_mla_compressed (kernel/cpu_attn.cpp:852-1022, nH =
 * q_proj rows / B at 860) as called by the decode branch of
 * _mla_compressed_forward (system/deepseek.py:355).
 *   q_nope [B*H, 512], q_pe [B*H, 64] bf16 (row b*H + h, the order of
 *          system/deepseek.py:337-338)
 *   c_pages, pe_pages: latent (also the value, 512 wide) and rope key (64
 *          wide) of token i of page p at c_pages + (p*page_size + i)*c_stride
 *          and pe_pages + (p*page_size + i)*pe_stride; the GPU pool layout
 *          [num_pages, page_size, 576] is c_stride = pe_stride = 576 with
 *          pe_pages = c_pages + 512, the reference's separate arrays are
 *          c_stride = 512, pe_stride = 64
 *   page_table, lens: as for GQA
 *   out    [B*H, 512] fp32 normalised partial; lse [B*H] fp32
 * Returns WH_OK or a negative WH_E* code. */
int wh_mla_partial(const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_pages,
                   int c_stride, const uint16_t* pe_pages, int pe_stride,
                   const int32_t* page_table, const int32_t* lens, int B, int H, int page_size,
                   int max_pages, int num_pages, float scale, float* out, float* lse,
                   int n_threads);

/* wh_mla_partial writing out as bf16 (rounded to nearest even), lse fp32
 * (WS_PARTIAL_LSE_BF16 for the GPU merges). */
int wh_mla_partial_bf16(const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_pages,
                        int c_stride, const uint16_t* pe_pages, int pe_stride,
                        const int32_t* page_table, const int32_t* lens, int B, int H,
                        int page_size, int max_pages, int num_pages, float scale,
                        uint16_t* out, float* lse, int n_threads);

/* wh_mla_partial returning the reference's triple: fp32 out [B*H, 512]
 * (unnormalised unless `normalize`), row_max [B*H] and row_sum [B*H] as for
 * wh_attn_triple.  Replaces fused_cpu_attn_mla_compressed's outputs
 * (kernel/cpu_attn.cpp:1001-1021: unnormalised out, max, sum). */
int wh_mla_triple(const uint16_t* q_nope, const uint16_t* q_pe, const uint16_t* c_pages,
                  int c_stride, const uint16_t* pe_pages, int pe_stride,
                  const int32_t* page_table, const int32_t* lens, int B, int H, int page_size,
                  int max_pages, int num_pages, float scale, int normalize, float* out,
                  float* row_max, float* row_sum, int n_threads);

/* Streaming read bandwidth of the host memory in GB/s (the host side's
 * roofline for the share scheduler): n_threads OpenMP threads (<= 0: the
 * default) sum a buffer of `bytes` (>= 1 MiB) that they first touched, best
 * of `reps` passes after one warm-up.  No counterpart in the reference (its
 * share tables are calibrated offline).  Returns 0 on bad arguments or a CPU
 * without AVX-512. */
double wh_host_read_gbs(size_t bytes, int n_threads, int reps);

#ifdef __cplusplus
}
#endif

#endif /* WSHOST_H */
