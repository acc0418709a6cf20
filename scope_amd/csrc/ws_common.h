// Shared definitions of the gfx950 kernels of the GPU KV partition.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/wsgpu.h"

namespace ws {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Records a thread-local error message for ws_last_error() and returns code.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }
__device__ __forceinline__ float qnan() { return __builtin_nanf(""); }

// max that keeps a NaN: a partial poisoned by a bad page id or length stays
// NaN through every merge (fmaxf would drop it and hide the error).
__device__ __forceinline__ float max_nan(float a, float b) {
  return (a != a || b != b) ? qnan() : fmaxf(a, b);
}

// v_perm_b32 pairing of two bf16 words: low halves or high halves of (lo, hi)
// into one dword [lo_part | hi_part << 16].
__device__ __forceinline__ uint32_t pair_lo(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

// Round-to-nearest-even fp32 -> bf16 of two values packed in one dword (a
// in the low half): one v_cvt_pk_bf16_f32 (converting the values one at a
// time costs a shift and a merge per pair).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// Round-to-nearest-even fp32 -> bf16 bits.
__device__ __forceinline__ uint16_t f32_to_bf16(float a) {
  return __builtin_bit_cast(uint16_t, (__bf16)a);
}

// Streaming 16-byte load: the KV pages are read once per call, so the
// non-temporal hint keeps them from displacing reused lines in the caches
// (and measurably raises the HBM read rate on gfx950).
__device__ __forceinline__ u32x4 ld_stream(const void* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}

// ds_read_b64_tr_b16 at LDS byte address `addr`.  In each 16-lane group,
// result lane 4 r + j, element e is element j of the four 16-bit values lane
// 4 e + r addresses (measured with an in-bounds probe on gfx950).
__device__ __forceinline__ uint2 lds_read_tr_b64(uint32_t addr) {
  typedef short i16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(uintptr_t)addr);
  return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}

__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b,
                                              const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Lane l's value and lane l ^ 16's (l ^ 32's) value, from gfx950's
// v_permlane16_swap (v_permlane32_swap): plain VALU exchanges, where a
// shuffle would be an LDS-crossbar round trip on the softmax's critical path.
// With both operands v, the swap leaves, in every lane, the lower-row (lower-
// half) value in the first result and the upper one in the second.
__device__ __forceinline__ void pair_xor16(float v, float& lo, float& hi) {
  const uint32_t a = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(a, a, false, false);
  lo = __builtin_bit_cast(float, (uint32_t)r[0]);
  hi = __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ void pair_xor32(float v, float& lo, float& hi) {
  const uint32_t a = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
  lo = __builtin_bit_cast(float, (uint32_t)r[0]);
  hi = __builtin_bit_cast(float, (uint32_t)r[1]);
}
// Max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lanes of a head
// column), every lane of the wave active.
__device__ __forceinline__ float wave_max_xor16_32(float v) {
  float lo, hi;
  pair_xor16(v, lo, hi);
  pair_xor32(fmaxf(lo, hi), lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float wave_sum_xor16_32(float v) {
  float lo, hi;
  pair_xor16(v, lo, hi);
  pair_xor32(lo + hi, lo, hi);
  return lo + hi;
}

}  // namespace ws
