/*
 * wslayer.h — one decode step of one attention layer over a two-sided
 * (host + HBM) paged KV cache in a single native call.
 *
 * The library (scope_amd/lib/libwslayer.so) strings together what the
 * reference's layer does in Python around its CPU thread
 * (system/deepseek.py:323-403 for absorbed MLA, system/mixoffload.py:
 * 1324-1464 for GQA): the query to pinned host memory (ws_copy), the GPU
 * split step with the fused append (ws_*_append_decode_split), the wait for
 * the query on the host, the host partial over the host pages
 * (wh_*_partial_bf16, OpenMP), and the merge, which reads the host partial
 * from pinned memory in place (ws_merge_split, or ws_mla_merge_split_uv
 * with the W_UV epilogue).  The calling thread runs it without Python in
 * between (ctypes releases the GIL for the whole call).  No counterpart in
 * the reference as one function; each piece cites its own in wsgpu.h /
 * wshost.h.
 *
 * Conventions: device pointers for the GPU side and the merge outputs;
 * pinned host memory (hipHostMalloc) for q_*_h, out_h, lse_h; host memory for
 * the host pools, page table and lengths.  A layer with no host tokens
 * (every host_lens[b] == 0) skips the copy, the wait and the host partial and
 * merges with no host operand.  Returns 0 or a negative error code
 * (WS_E*, or WH_E* from the host partial); wl_last_error() is the message.
 * The output field `stage` tells how far the call got: 0 nothing launched,
 * 1 the split step launched (so the device lengths advanced), 2 the merge
 * launched.
 */
#ifndef WSLAYER_H
#define WSLAYER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  /* GPU split step (ws_mla_append_decode_split): q rows b*H + h */
  const uint16_t* q_nope;  /* [B*H][512] bf16, device */
  const uint16_t* q_pe;    /* [B*H][64] */
  const uint16_t* c_new;   /* [B] rows of 512 at stride c_stride */
  int64_t c_stride;
  const uint16_t* pe_new;  /* [B] rows of 64 at stride pe_stride */
  int64_t pe_stride;
  uint16_t* latent_pages;  /* [num_pages][page_size][576] */
  const int32_t* page_table;
  const int32_t* len_in;
  int32_t* len_out;
  int B, H, page_size, max_pages, num_pages, max_len, n_splits;
  float scale;
  float* out_g;            /* [B*H][512] fp32 scratch of the step */
  float* lse_g;            /* [B*H] */
  void* workspace;
  size_t workspace_bytes;
  void* ev_step_begin;     /* optional hipEvent_t recorded around the step */
  void* ev_step_end;
  /* host partial (wh_mla_partial_bf16) over the host segment */
  uint16_t* q_nope_h;      /* pinned [B*H][512] */
  uint16_t* q_pe_h;        /* pinned [B*H][64] */
  const uint16_t* host_latent;  /* [host_num_pages][host_page_size][576] */
  const int32_t* host_table;    /* [B][host_max_pages] */
  const int32_t* host_lens;     /* [B] */
  int host_page_size, host_max_pages, host_num_pages, host_threads;
  uint16_t* out_h;         /* pinned bf16 [B*H][512] */
  float* lse_h;            /* pinned fp32 [B*H] */
  /* merge outputs (device); with w_uv the W_UV epilogue instead of out */
  uint16_t* out;           /* bf16 [B*H][512], or NULL with w_uv */
  float* lse_out;          /* fp32 [B*H] or NULL */
  const uint16_t* w_uv;    /* [H][Dout][512] bf16 or NULL */
  int Dout;
  uint16_t* out_v;         /* [B][H*Dout] bf16 with w_uv */
  /* results */
  double host_seconds;     /* out: the host partial's wall time */
  int stage;               /* out: see above */
} WlMlaLayer;

int wl_mla_layer(WlMlaLayer* a, void* stream);

typedef struct {
  /* GPU split step (ws_gqa_append_decode_split) */
  const uint16_t* q;       /* [B][Hq][D] bf16, device */
  const uint16_t* k_new;   /* [B][Hkv][1][D] */
  const uint16_t* v_new;
  uint16_t* k_pages;       /* [num_pages][Hkv][page_size][D] */
  uint16_t* v_pages;
  const int32_t* page_table;
  const int32_t* len_in;
  int32_t* len_out;
  int B, Hq, Hkv, D, page_size, max_pages, num_pages, max_len, n_splits;
  float scale;
  float* out_g;            /* [B][Hq][D] fp32 scratch of the step */
  float* lse_g;
  void* workspace;
  size_t workspace_bytes;
  void* ev_step_begin;
  void* ev_step_end;
  /* host partial (wh_gqa_partial_bf16) */
  uint16_t* q_h;           /* pinned [B][Hq][D] */
  const uint16_t* host_k;  /* [host_num_pages][Hkv][host_page_size][D] */
  const uint16_t* host_v;
  const int32_t* host_table;
  const int32_t* host_lens;
  int host_page_size, host_max_pages, host_num_pages, host_threads;
  uint16_t* out_h;         /* pinned bf16 [B][Hq][D] */
  float* lse_h;            /* pinned fp32 [B][Hq] */
  /* merge outputs (device) */
  uint16_t* out;           /* bf16 [B][Hq][D] */
  float* lse_out;          /* fp32 [B][Hq] or NULL */
  double host_seconds;
  int stage;
} WlGqaLayer;

int wl_gqa_layer(WlGqaLayer* a, void* stream);

const char* wl_last_error(void);

/* sizeof(WlMlaLayer) for which == 0, sizeof(WlGqaLayer) for 1 (bindings check
 * their struct layouts against it). */
size_t wl_struct_size(int which);

#ifdef __cplusplus
}
#endif

#endif /* WSLAYER_H */
