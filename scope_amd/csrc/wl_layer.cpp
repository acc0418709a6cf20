// One decode step of one attention layer over a two-sided paged KV cache in
// a single native call (include/wslayer.h): the query to pinned host memory,
// the GPU split step, the host partial over the host pages once the query
// has arrived, and the merge that reads the host partial in place.  Host
// code only; it calls libwsgpu.so (the launches) and libwshost.so (the host
// partial) through their C ABIs.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstdio>

#include "../../include/wsgpu.h"
#include "../../include/wshost.h"
#include "../../include/wslayer.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int gpu_fail(int rc, const char* what) {
  return fail(rc, "%s: %s", what, ws_last_error());
}

// The event the host waits on for the query copy: one per thread and
// device, created on first use (an event records only on streams of the
// device it was created on).  It keeps the default system-scope release, so
// the copy's writes to host memory are visible once it has completed.
constexpr int kMaxDevices = 64;

int query_event(hipStream_t s, hipEvent_t* ev) {
  thread_local hipEvent_t e[kMaxDevices] = {};
  int dev = 0, cur = 0;
  if (hipStreamGetDevice(s, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(WS_ELAUNCH, "wl: the stream's device is unknown");
  if (!e[dev]) {
    if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(dev) != hipSuccess)
      return fail(WS_ELAUNCH, "wl: cannot select device %d", dev);
    const hipError_t rc = hipEventCreateWithFlags(&e[dev], hipEventDisableTiming);
    hipSetDevice(cur);
    if (rc != hipSuccess) {
      e[dev] = nullptr;
      return fail(WS_ELAUNCH, "wl: hipEventCreateWithFlags failed");
    }
  }
  *ev = e[dev];
  return WS_OK;
}

bool any_host_tokens(const int32_t* lens, int B) {
  for (int b = 0; b < B; ++b)
    if (lens[b] != 0) return true;
  return false;
}

// Records ev (a caller's timing event) on the stream, if given.
int record(void* ev, hipStream_t s) {
  if (ev && hipEventRecord((hipEvent_t)ev, s) != hipSuccess)
    return fail(WS_ELAUNCH, "wl: hipEventRecord failed");
  return WS_OK;
}

// Copies `n` query buffers to the host and records the wait event.
int query_to_host(void* const* dst, const void* const* src, const size_t* bytes, int n,
                  hipStream_t s, hipEvent_t* ev) {
  for (int i = 0; i < n; ++i)
    if (int rc = ws_copy(dst[i], src[i], bytes[i], s)) return gpu_fail(rc, "wl: query copy");
  if (int rc = query_event(s, ev)) return rc;
  if (hipEventRecord(*ev, s) != hipSuccess) return fail(WS_ELAUNCH, "wl: hipEventRecord failed");
  return WS_OK;
}

int wait_query(hipEvent_t ev) {
  if (hipEventSynchronize(ev) != hipSuccess)
    return fail(WS_ELAUNCH, "wl: waiting for the query copy failed");
  return WS_OK;
}

}  // namespace

extern "C" const char* wl_last_error(void) { return g_err; }

extern "C" size_t wl_struct_size(int which) {
  return which == 0 ? sizeof(WlMlaLayer) : which == 1 ? sizeof(WlGqaLayer) : 0;
}

extern "C" int wl_mla_layer(WlMlaLayer* a, void* stream) {
  g_err[0] = '\0';
  if (!a) return fail(WS_EINVAL, "wl_mla_layer: null arguments");
  a->stage = 0;
  a->host_seconds = 0.0;
  if (a->B <= 0 || a->H <= 0 || !a->host_lens)
    return fail(WS_EINVAL, "wl_mla_layer: bad batch B=%d H=%d", a->B, a->H);
  if (!a->w_uv && !a->out) return fail(WS_EINVAL, "wl_mla_layer: no output");
  hipStream_t s = (hipStream_t)stream;
  const bool host = any_host_tokens(a->host_lens, a->B);
  const size_t rows = (size_t)a->B * a->H;
  hipEvent_t ev = nullptr;
  if (host) {
    if (!a->q_nope_h || !a->q_pe_h || !a->out_h || !a->lse_h)
      return fail(WS_EINVAL, "wl_mla_layer: host buffers missing");
    void* dst[2] = {a->q_nope_h, a->q_pe_h};
    const void* src[2] = {a->q_nope, a->q_pe};
    const size_t bytes[2] = {rows * 512 * 2, rows * 64 * 2};
    if (int rc = query_to_host(dst, src, bytes, 2, s, &ev)) return rc;
  }
  if (int rc = record(a->ev_step_begin, s)) return rc;
  if (int rc = ws_mla_append_decode_split(
          a->q_nope, a->q_pe, a->c_new, a->c_stride, a->pe_new, a->pe_stride, a->latent_pages,
          a->page_table, a->len_in, a->len_out, a->B, a->H, a->page_size, a->max_pages,
          a->num_pages, a->max_len, a->n_splits, a->scale, a->out_g, a->lse_g, a->workspace,
          a->workspace_bytes, s))
    return gpu_fail(rc, "wl_mla_layer: split step");
  a->stage = 1;
  if (int rc = record(a->ev_step_end, s)) return rc;
  const void* b_out = nullptr;
  const void* b_lse = nullptr;
  if (host) {
    if (int rc = wait_query(ev)) return rc;
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = wh_mla_partial_bf16(
        a->q_nope_h, a->q_pe_h, a->host_latent, 576, a->host_latent + 512, 576, a->host_table,
        a->host_lens, a->B, a->H, a->host_page_size, a->host_max_pages, a->host_num_pages,
        a->scale, a->out_h, a->lse_h, a->host_threads);
    a->host_seconds =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (rc) return fail(rc, "wl_mla_layer: host partial: %s", wh_last_error());
    b_out = a->out_h;
    b_lse = a->lse_h;
  }
  const int cap = a->page_size * a->max_pages;
  int rc;
  if (a->w_uv)
    rc = ws_mla_merge_split_uv(a->len_out, a->B, a->H, cap, a->n_splits, a->out_g, a->lse_g,
                               a->workspace, a->workspace_bytes, b_out, b_lse, nullptr,
                               WS_PARTIAL_LSE_BF16, a->w_uv, a->Dout, nullptr, a->out_v,
                               a->lse_out, s);
  else
    rc = ws_merge_split(a->len_out, a->B, 1, a->H, 512, cap, a->n_splits, a->out_g, a->lse_g,
                        a->workspace, a->workspace_bytes, b_out, b_lse, nullptr,
                        WS_PARTIAL_LSE_BF16, a->out, nullptr, a->lse_out, s);
  if (rc) return gpu_fail(rc, "wl_mla_layer: merge");
  a->stage = 2;
  return WS_OK;
}

extern "C" int wl_gqa_layer(WlGqaLayer* a, void* stream) {
  g_err[0] = '\0';
  if (!a) return fail(WS_EINVAL, "wl_gqa_layer: null arguments");
  a->stage = 0;
  a->host_seconds = 0.0;
  if (a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Hq % a->Hkv || !a->host_lens || !a->out)
    return fail(WS_EINVAL, "wl_gqa_layer: bad shape B=%d Hq=%d Hkv=%d", a->B, a->Hq, a->Hkv);
  hipStream_t s = (hipStream_t)stream;
  const bool host = any_host_tokens(a->host_lens, a->B);
  const size_t rows = (size_t)a->B * a->Hq;
  hipEvent_t ev = nullptr;
  if (host) {
    if (!a->q_h || !a->out_h || !a->lse_h)
      return fail(WS_EINVAL, "wl_gqa_layer: host buffers missing");
    void* dst[1] = {a->q_h};
    const void* src[1] = {a->q};
    const size_t bytes[1] = {rows * (size_t)a->D * 2};
    if (int rc = query_to_host(dst, src, bytes, 1, s, &ev)) return rc;
  }
  if (int rc = record(a->ev_step_begin, s)) return rc;
  if (int rc = ws_gqa_append_decode_split(
          a->q, a->k_new, a->v_new, a->k_pages, a->v_pages, a->page_table, a->len_in,
          a->len_out, a->B, a->Hq, a->Hkv, a->D, a->page_size, a->max_pages, a->num_pages,
          a->max_len, a->n_splits, a->scale, a->out_g, a->lse_g, a->workspace,
          a->workspace_bytes, s))
    return gpu_fail(rc, "wl_gqa_layer: split step");
  a->stage = 1;
  if (int rc = record(a->ev_step_end, s)) return rc;
  const void* b_out = nullptr;
  const void* b_lse = nullptr;
  if (host) {
    if (int rc = wait_query(ev)) return rc;
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = wh_gqa_partial_bf16(a->q_h, a->host_k, a->host_v, a->host_table,
                                       a->host_lens, a->B, a->Hq, a->Hkv, a->D,
                                       a->host_page_size, a->host_max_pages,
                                       a->host_num_pages, a->scale, a->out_h, a->lse_h,
                                       a->host_threads);
    a->host_seconds =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (rc) return fail(rc, "wl_gqa_layer: host partial: %s", wh_last_error());
    b_out = a->out_h;
    b_lse = a->lse_h;
  }
  const int rc = ws_merge_split(a->len_out, a->B, a->Hkv, a->Hq / a->Hkv, a->D,
                                a->page_size * a->max_pages, a->n_splits, a->out_g, a->lse_g,
                                a->workspace, a->workspace_bytes, b_out, b_lse, nullptr,
                                WS_PARTIAL_LSE_BF16, a->out, nullptr, a->lse_out, s);
  if (rc) return gpu_fail(rc, "wl_gqa_layer: merge");
  a->stage = 2;
  return WS_OK;
}
