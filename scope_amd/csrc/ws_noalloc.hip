// ws_gqa_append_decode_partial without a caller workspace: for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops
// that forbid hipMalloc).  The split pieces of the step live in a file-scope
// device array, `scratch`, of kNoAllocScratchBytes; every GPU the library runs
// on holds its own copy until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address is taken once per device with hipGetSymbolAddress (with that
// device current) and only that address is passed to the kernels.  Every call
// on one GPU shares the array, so calls that overlap on one GPU (different
// streams, or threads without ordering) race; calls ordered on one stream do
// not.  The array needs no initial contents: a call writes every slot it or
// its combine launch reads back.
#include <mutex>

#include "ws_reduce.h"

namespace ws {

constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kNoAllocMaxDevices];

// Device address of `scratch` on device `dev`, looked up on the first call
// for that device (made current for the lookup) and kept.
static int scratch_address(int dev, void** out, const char* name) {
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(WS_EINVAL, "%s: device %d outside [0, %d)", name, dev, kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess)
      return set_error(WS_ELAUNCH, "%s: hipGetDevice failed", name);
    if (cur != dev && hipSetDevice(dev) != hipSuccess)
      return set_error(WS_ELAUNCH, "%s: hipSetDevice(%d) failed", name, dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return set_error(WS_ELAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", name,
                       dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WS_OK;
}

}  // namespace ws

using namespace ws;

extern "C" size_t ws_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int ws_gqa_append_decode_partial_noalloc(
    const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_pages,
    uint16_t* v_pages, const int32_t* page_table, const int32_t* len_in, int32_t* len_out,
    int B, int Hq, int Hkv, int D, int page_size, int max_pages, int num_pages, int max_len,
    int n_workgroups, float scale, float* out, float* lse, void* stream) {
  static const char* name = "ws_gqa_append_decode_partial_noalloc";
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv || B < 0)
    return set_error(WS_EINVAL, "%s: bad batch/heads B=%d Hq=%d Hkv=%d", name, B, Hq, Hkv);
  int n = 0;
  size_t need = 0;
  int rc = ws_attn_decode_plan(B * Hkv, Hq / Hkv, D, D, max_len, n_workgroups, &n, &need);
  if (rc != WS_OK) return rc;
  if (need > kNoAllocScratchBytes)
    return set_error(WS_EWORKSPACE,
                     "%s: the step needs %zu bytes of split scratch, above the static %zu "
                     "(fewer splits, rows or heads, or ws_gqa_append_decode_partial with a "
                     "workspace)",
                     name, need, kNoAllocScratchBytes);
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice((hipStream_t)stream, &dev) != hipSuccess)
      return set_error(WS_EINVAL, "%s: cannot query the stream's device", name);
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return set_error(WS_ELAUNCH, "%s: hipGetDevice failed", name);
  }
  void* ptr = nullptr;
  rc = scratch_address(dev, &ptr, name);
  if (rc != WS_OK) return rc;
  return ws_gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, page_table, len_in,
                                      len_out, B, Hq, Hkv, D, page_size, max_pages, num_pages,
                                      max_len, n, scale, out, lse, ptr, kNoAllocScratchBytes,
                                      stream);
}
