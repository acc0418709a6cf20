// Split pieces shared by the decode kernels and the merges.
//
// A decode call cuts every row's blocks between its splits (ws_plan.h).  A
// split that holds a whole row writes the row's final partial (out
// normalised fp32, lse natural log) straight to the caller's out / lse; a
// row spread over several splits leaves one piece per split in the
// workspace, and a later launch on the same stream (merge_split_kernel,
// merge_split_uv_kernel, mla_reduce_kernel) rebuilds the plan to find and
// LSE-combine them.
//
// Workspace layout (ws_decode_plan), for a call over rows_kv rows of `heads`
// output rows each, run by n splits:
//   [slot lse f32 x (n + rows_kv) x heads, padded to 256 B]
//   [slot out bf16 x (n + rows_kv) x heads x Dv]
// (slot = split + row, ws_plan.h).  Pieces are normalised and rounded to
// bf16 (their weights stay fp32): a 32-token block carries 36 KB of latent
// and an MLA piece 16 x 512 outputs, so at 256 splits fp32 pieces cost
// 8 MB of writes and reads per call.  Every call writes the slots it reads
// back, so the workspace needs no initial contents.
#pragma once

#include "ws_common.h"

namespace ws {

// Most (partial, row) weights one reduction keeps in LDS.
constexpr int kReduceMaxWeights = 4096;

__host__ __device__ inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct SplitWorkspace {
  float* part_lse;
  uint16_t* part_out;  // bf16
};

__host__ __device__ inline size_t workspace_bytes(int rows_kv, int heads, int Dv, int n) {
  const size_t slots = (size_t)n + rows_kv;
  return align256(slots * heads * 4) + slots * heads * Dv * 2;
}

__host__ __device__ inline SplitWorkspace carve_workspace(void* base, int rows_kv,
                                                          int heads, int n) {
  SplitWorkspace w;
  char* p = (char*)base;
  const size_t slots = (size_t)n + rows_kv;
  w.part_lse = (float*)p;
  p += align256(slots * heads * 4);
  w.part_out = (uint16_t*)p;
  return w;
}

// Layout of an absorbed-MLA call with B sequences of H heads (H a multiple
// of 16).  H = 128 over at most 64 sequences (DeepSeek-V2) runs the wide
// kernel (ws_mla_wide.h): its plan sequences are the sequences and a piece
// holds all 128 heads.  Other head counts plan (sequence, 16-head group)
// pairs with 16-head pieces.  The step, the merges and the workspace query of
// a call all take their layout from here, so they agree.
constexpr int kWideHeads = 128;
constexpr int kWideMaxSeqs = 64;
struct MlaLayout {
  bool wide;
  int ng;           // plan sequences per sequence
  int piece_heads;  // heads of one piece
  int plan_seqs;    // B * ng
};
__host__ __device__ inline MlaLayout mla_layout(int B, int H) {
  MlaLayout l;
  l.wide = H == kWideHeads && B >= 1 && B <= kWideMaxSeqs;
  l.ng = l.wide ? 1 : H / 16;
  l.piece_heads = l.wide ? H : 16;
  l.plan_seqs = B * l.ng;
  return l;
}

// Workgroups of a decode call: n_workgroups, or the library's choice (0):
// `per_cu` resident workgroups on every CU of the current device, but no more
// than the call's 32-token blocks can feed with `min_blocks` each.
int choose_workgroups(int n_workgroups, int per_cu, long long max_blocks, int min_blocks);
// Workgroups of an MLA call (ws_mla.hip).
int mla_workgroups(int n_workgroups, int B, int max_len);
// Combines the pieces of a split decode step with no host partial: rows held
// by several splits are LSE-combined from the workspace, the others copied;
// lengths are len[b] + len_add; out/lse may alias out_g/lse_g (Dv <= 256);
// out_bf16, when not null, also receives the output in bf16.  Launches on
// `stream`; returns WS_OK or an error code (ws_merge.hip).
int merge_split_pieces(const int32_t* len, int len_add, int B, int R, int heads, int Dv,
                       int cap, int n, const float* out_g, const float* lse_g,
                       const SplitWorkspace& w, float* out, float* lse, uint16_t* out_bf16,
                       hipStream_t stream);

// Eight outputs of a piece, rounded to bf16, as one 16-byte store.
__device__ __forceinline__ void store_piece8(uint16_t* dst, float a0, float a1, float a2,
                                             float a3, float a4, float a5, float a6,
                                             float a7) {
  u32x4 v;
  v[0] = pack_bf16x2(a0, a1);
  v[1] = pack_bf16x2(a2, a3);
  v[2] = pack_bf16x2(a4, a5);
  v[3] = pack_bf16x2(a6, a7);
  *(u32x4*)dst = v;
}

// Four bf16 piece outputs (8 bytes) as floats.
__device__ __forceinline__ float4 piece4_f32(uint2 v) {
  return make_float4(__builtin_bit_cast(float, v.x << 16),
                     __builtin_bit_cast(float, v.x & 0xffff0000u),
                     __builtin_bit_cast(float, v.y << 16),
                     __builtin_bit_cast(float, v.y & 0xffff0000u));
}

// a += ws * (four outputs of one piece).
__device__ __forceinline__ void accum_piece(float4& a, float ws, uint2 raw) {
  const float4 v = piece4_f32(raw);
  a.x += ws * v.x; a.y += ws * v.y; a.z += ws * v.z; a.w += ws * v.w;
}

// a += sum_s w[s] * (four bf16 outputs of piece s at src + s * stride), in
// order of s, with sixteen pieces' loads in flight per round while sixteen
// remain, then eight (the last n % 8 pieces' loads also go out together).
__device__ __forceinline__ void accum_pieces(const uint16_t* src, size_t stride, int n,
                                             const float* w, float4& a) {
  int s = 0;
  for (; s + 16 <= n; s += 16) {
    uint2 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = *(const uint2*)(src + (size_t)(s + u) * stride);
#pragma unroll
    for (int u = 0; u < 16; ++u) accum_piece(a, w[s + u], v[u]);
  }
  for (; s + 8 <= n; s += 8) {
    uint2 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *(const uint2*)(src + (size_t)(s + u) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) accum_piece(a, w[s + u], v[u]);
  }
  if (s < n) {
    uint2 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = *(const uint2*)(src + (size_t)min(s + u, n - 1) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s + u < n) accum_piece(a, w[s + u], v[u]);
  }
}

// The raw bytes of a row's pieces when it has at most eight (a row with
// fewer repeats its last one), requested before the weights are known: the
// piece loads share their round trip with the lse loads, and nothing waits
// for them until the accumulation.
__device__ __forceinline__ void preload_pieces(const uint16_t* src, size_t stride, int n,
                                               uint2 (&v)[8]) {
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = *(const uint2*)(src + (size_t)min(u, n - 1) * stride);
}

// accum_pieces over the n <= 8 pieces preload_pieces fetched: the same terms
// in the same order, so the result is bit-identical to accum_pieces.
__device__ __forceinline__ void accum_preloaded(const uint2 (&v)[8], int n, const float* w,
                                                float4& a) {
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (u < n) accum_piece(a, w[u], v[u]);
}

}  // namespace ws
