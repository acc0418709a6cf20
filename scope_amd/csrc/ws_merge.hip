// LSE merge of the GPU partial with a second (host) partial, fused with the
// final normalisation and the bf16 cast.  One workgroup per row, one float4
// of the output per thread.  The second operand may arrive in any of the
// reference CPU kernels' output conventions, so no conversion launch is
// needed after its host-to-device copy.
#include <math.h>

#include "ws_common.h"

namespace ws {

template <int FMT>
__device__ __forceinline__ void load_b(const void* b_out, const void* aux0,
                                       const void* aux1, int row, int Dv, int c,
                                       float& lse_b, float4& o_b) {
  if (FMT == WS_PARTIAL_LSE_F32) {
    lse_b = ((const float*)aux0)[row];
    o_b = ((const float4*)((const float*)b_out + (size_t)row * Dv))[c];
  } else if (FMT == WS_TRIPLE_UNNORM_F32 || FMT == WS_TRIPLE_NORM_F32) {
    const float m = ((const float*)aux0)[row];
    const float s = ((const float*)aux1)[row];
    lse_b = (s > 0.f) ? m + __logf(s) : neg_inf();
    o_b = ((const float4*)((const float*)b_out + (size_t)row * Dv))[c];
    if (FMT == WS_TRIPLE_UNNORM_F32) {
      const float inv = (s > 0.f) ? 1.f / s : 0.f;
      o_b.x *= inv;
      o_b.y *= inv;
      o_b.z *= inv;
      o_b.w *= inv;
    }
  } else {  // WS_TRIPLE_NORM_BF16
    const float m = bf16_to_f32(((const uint16_t*)aux0)[row]);
    const float s = bf16_to_f32(((const uint16_t*)aux1)[row]);
    lse_b = (s > 0.f) ? m + __logf(s) : neg_inf();
    const uint2 raw =
        ((const uint2*)((const uint16_t*)b_out + (size_t)row * Dv))[c];
    o_b = make_float4(bf16_to_f32(raw.x & 0xffffu), bf16_to_f32(raw.x >> 16),
                      bf16_to_f32(raw.y & 0xffffu), bf16_to_f32(raw.y >> 16));
  }
}

template <int FMT>
__global__ __launch_bounds__(128) void lse_merge_kernel(
    const float* __restrict__ out_g, const float* __restrict__ lse_g,
    const void* __restrict__ b_out, const void* __restrict__ b_aux0,
    const void* __restrict__ b_aux1, uint16_t* __restrict__ out_bf16,
    float* __restrict__ out_f32, float* __restrict__ lse_out, int Dv) {
  const int row = blockIdx.x;
  const int c = threadIdx.x;
  if (c >= Dv / 4) return;
  const float la = lse_g[row];
  float lb;
  float4 ob;
  load_b<FMT>(b_out, b_aux0, b_aux1, row, Dv, c, lb, ob);
  const float M = fmaxf(la, lb);
  float4 r;
  float lse_r;
  if (M == neg_inf()) {
    r = make_float4(0.f, 0.f, 0.f, 0.f);
    lse_r = neg_inf();
  } else {
    const float wa = __expf(la - M);
    const float wb = __expf(lb - M);
    const float inv = 1.f / (wa + wb);
    const float4 oa = ((const float4*)(out_g + (size_t)row * Dv))[c];
    // An empty side has weight 0; its (0) output must not turn into NaN.
    const float fa = wa * inv, fb = wb * inv;
    r = make_float4(fa * oa.x + fb * ob.x, fa * oa.y + fb * ob.y,
                    fa * oa.z + fb * ob.z, fa * oa.w + fb * ob.w);
    lse_r = M + __logf(wa + wb);
  }
  if (out_f32) ((float4*)(out_f32 + (size_t)row * Dv))[c] = r;
  if (out_bf16) {
    uint2 packed;
    packed.x = pack_bf16x2(r.x, r.y);
    packed.y = pack_bf16x2(r.z, r.w);
    ((uint2*)(out_bf16 + (size_t)row * Dv))[c] = packed;
  }
  if (lse_out && c == 0) lse_out[row] = lse_r;
}

}  // namespace ws

using namespace ws;

extern "C" int ws_lse_merge(const float* out_g, const float* lse_g,
                            const void* b_out, const void* b_aux0,
                            const void* b_aux1, int fmt_b, uint16_t* out_bf16,
                            float* out_f32, float* lse_out, int rows, int Dv,
                            void* stream) {
  if (!out_g || !lse_g || !b_out || !b_aux0)
    return set_error(WS_EINVAL, "ws_lse_merge: null input pointer");
  if (fmt_b != WS_PARTIAL_LSE_F32 && !b_aux1)
    return set_error(WS_EINVAL, "ws_lse_merge: triple format needs b_aux1 (sum)");
  if (rows < 0 || Dv <= 0 || Dv % 4 || Dv > 512)
    return set_error(WS_EINVAL, "ws_lse_merge: bad sizes rows=%d Dv=%d", rows, Dv);
  if (((uintptr_t)out_g | (uintptr_t)b_out | (uintptr_t)out_f32) & 15u ||
      ((uintptr_t)out_bf16 & 7u))
    return set_error(WS_EINVAL, "ws_lse_merge: misaligned buffer");
  if (rows == 0) return WS_OK;
  const int threads = ((Dv / 4 + 63) / 64) * 64;
  hipStream_t s = (hipStream_t)stream;
  switch (fmt_b) {
#define WS_MERGE_CASE(F)                                                         \
  case F:                                                                        \
    hipLaunchKernelGGL(lse_merge_kernel<F>, dim3(rows), dim3(threads), 0, s,     \
                       out_g, lse_g, b_out, b_aux0, b_aux1, out_bf16, out_f32,   \
                       lse_out, Dv);                                             \
    break;
    WS_MERGE_CASE(WS_PARTIAL_LSE_F32)
    WS_MERGE_CASE(WS_TRIPLE_UNNORM_F32)
    WS_MERGE_CASE(WS_TRIPLE_NORM_BF16)
    WS_MERGE_CASE(WS_TRIPLE_NORM_F32)
#undef WS_MERGE_CASE
    default:
      return set_error(WS_EINVAL, "ws_lse_merge: unknown format %d", fmt_b);
  }
  return check_launch("ws_lse_merge");
}
