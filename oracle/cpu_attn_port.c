/*
 * C restatement of the reference CPU partial-attention kernels.
 * ORACLE — test infrastructure and CPU baseline only; never product code.
 *
 * Follows kernel/cpu_attn.cpp:
 *   ws_oracle_gqa            fused_cpu_attn (572-636) and fused_cpu_attn_mla
 *                            (638-672): run_kernel (193-570) = tiling
 *                            (205-222), per-tile online softmax over 8-token
 *                            blocks with fp32 accumulation (230-531), tile
 *                            merge (533-569), optional normalisation.
 *   ws_oracle_mla_compressed fused_cpu_attn_mla_compressed (852-1022):
 *                            n_tiles = max(1, threads / B) sequence tiles per
 *                            batch row (886-888), 8-token blocks over the 16
 *                            heads sharing one latent (905-971), serial merge
 *                            (1001-1020).
 * Written in plain C from the math (no intrinsics); the compiler vectorises
 * the d-loops.  Differences from the reference: S == 0 returns the empty
 * partial (out 0, max -inf, sum 0) where the reference divides by zero
 * (kernel/cpu_attn.cpp:217-222, 887-888); exp is libm expf (the reference
 * builds with -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Load one row of `n` elements as fp32 (bf16 widened or fp32 copied). */
static inline void load_row(float* dst, const void* src, int64_t off, int n,
                            int is_bf16) {
  if (is_bf16) {
    const uint16_t* s = (const uint16_t*)src + off;
    for (int i = 0; i < n; ++i) dst[i] = bf(s[i]);
  } else {
    memcpy(dst, (const float*)src + off, sizeof(float) * (size_t)n);
  }
}

static int tile_len_gqa(int seq, int rows, int n_threads) {
  int target = 1;
  if (rows < n_threads) {
    target = (n_threads + rows - 1) / rows;
    if (target < 2) target = 2;
  }
  int tile = (seq + target - 1) / target;
  tile = ((tile + 15) / 16) * 16;
  if (tile < 256) tile = 256;
  if (tile > seq) tile = seq;
  return tile;
}

/* Online softmax of G query rows over tokens [t0, t1) of one K/V row.
 * qf [G][Dk] fp32; o [G][Dv], m [G], s [G] updated in place. */
__attribute__((target_clones("avx512f", "avx2", "default")))
static void gqa_tile(const float* qf, const void* k, const void* v, int is_bf16,
                     int64_t k_row, int64_t k_si, int64_t v_row, int64_t v_si,
                     int G, int Dk, int Dv, int t0, int t1, float scale,
                     float* o, float* m, float* s, float* kbuf, float* vbuf) {
  enum { BLK = 8 };
  float sc[BLK];
  for (int t = t0; t < t1; t += BLK) {
    const int nb = (t1 - t) < BLK ? (t1 - t) : BLK;
    for (int r = 0; r < nb; ++r) {
      load_row(kbuf + (size_t)r * Dk, k, k_row + (int64_t)(t + r) * k_si, Dk, is_bf16);
      load_row(vbuf + (size_t)r * Dv, v, v_row + (int64_t)(t + r) * v_si, Dv, is_bf16);
    }
    for (int g = 0; g < G; ++g) {
      const float* qg = qf + (size_t)g * Dk;
      float m_new = m[g];
      for (int r = 0; r < nb; ++r) {
        const float* kr = kbuf + (size_t)r * Dk;
        float acc = 0.f;
#pragma omp simd reduction(+ : acc)
        for (int d = 0; d < Dk; ++d) acc += qg[d] * kr[d];
        sc[r] = acc * scale;
        if (sc[r] > m_new) m_new = sc[r];
      }
      const float decay = expf(m[g] - m_new);
      float blk_sum = 0.f;
      float* og = o + (size_t)g * Dv;
#pragma omp simd
      for (int d = 0; d < Dv; ++d) og[d] *= decay;
      for (int r = 0; r < nb; ++r) {
        const float e = expf(sc[r] - m_new);
        blk_sum += e;
        const float* vr = vbuf + (size_t)r * Dv;
#pragma omp simd
        for (int d = 0; d < Dv; ++d) og[d] += e * vr[d];
      }
      s[g] = decay * s[g] + blk_sum;
      m[g] = m_new;
    }
  }
}

/*
 * q [B_kv][G][Dk] contiguous; k row b token i at k + b*k_sb + i*k_si (elements),
 * likewise v.  is_bf16 selects bf16 or fp32 for q, k, v.
 * out [B_kv][G][Dv], mx [B_kv][G], sm [B_kv][G] fp32.
 * normalize = 1: out = o / sum (fused_cpu_attn); 0: unnormalised
 * (fused_cpu_attn_mla).  n_threads <= 0 uses the OpenMP default.
 */
void ws_oracle_gqa(const void* q, const void* k, const void* v, int is_bf16,
                   int B_kv, int G, int Dk, int Dv, int S, int64_t k_sb,
                   int64_t k_si, int64_t v_sb, int64_t v_si, float scale,
                   int normalize, int n_threads, float* out, float* mx,
                   float* sm) {
#ifdef _OPENMP
  if (n_threads <= 0) n_threads = omp_get_max_threads();
#else
  n_threads = 1;
#endif
  for (int64_t i = 0; i < (int64_t)B_kv * G; ++i) {
    mx[i] = -INFINITY;
    sm[i] = 0.f;
  }
  memset(out, 0, sizeof(float) * (size_t)B_kv * G * Dv);
  if (S <= 0 || B_kv <= 0) return;
  const int tile = tile_len_gqa(S, B_kv, n_threads);
  const int n_tiles = (S + tile - 1) / tile;
  const int tasks = B_kv * n_tiles;
  float* t_o = (float*)calloc((size_t)tasks * G * Dv, sizeof(float));
  float* t_m = (float*)malloc(sizeof(float) * (size_t)tasks * G);
  float* t_s = (float*)calloc((size_t)tasks * G, sizeof(float));
  for (int64_t i = 0; i < (int64_t)tasks * G; ++i) t_m[i] = -INFINITY;

#pragma omp parallel num_threads(n_threads)
  {
    float* qf = (float*)malloc(sizeof(float) * (size_t)G * Dk);
    float* kbuf = (float*)malloc(sizeof(float) * 8 * (size_t)Dk);
    float* vbuf = (float*)malloc(sizeof(float) * 8 * (size_t)Dv);
#pragma omp for schedule(static)
    for (int task = 0; task < tasks; ++task) {
      const int b = task / n_tiles, ti = task % n_tiles;
      const int t0 = ti * tile;
      const int t1 = (t0 + tile < S) ? t0 + tile : S;
      load_row(qf, q, (int64_t)b * G * Dk, G * Dk, is_bf16);
      gqa_tile(qf, k, v, is_bf16, (int64_t)b * k_sb, k_si, (int64_t)b * v_sb,
               v_si, G, Dk, Dv, t0, t1, scale, t_o + (size_t)task * G * Dv,
               t_m + (size_t)task * G, t_s + (size_t)task * G, kbuf, vbuf);
    }
    free(qf);
    free(kbuf);
    free(vbuf);
  }

#pragma omp parallel for schedule(static) num_threads(n_threads)
  for (int b = 0; b < B_kv; ++b) {
    for (int g = 0; g < G; ++g) {
      float row_max = -INFINITY;
      for (int ti = 0; ti < n_tiles; ++ti) {
        const float tm = t_m[((size_t)b * n_tiles + ti) * G + g];
        if (tm > row_max) row_max = tm;
      }
      float row_sum = 0.f;
      float* og = out + ((size_t)b * G + g) * Dv;
      for (int ti = 0; ti < n_tiles; ++ti) {
        const size_t tk = (size_t)b * n_tiles + ti;
        const float w = expf(t_m[tk * G + g] - row_max);
        row_sum += w * t_s[tk * G + g];
        const float* to = t_o + (tk * G + g) * Dv;
        for (int d = 0; d < Dv; ++d) og[d] += w * to[d];
      }
      if (normalize) {
        const float inv = 1.f / row_sum;
        for (int d = 0; d < Dv; ++d) og[d] *= inv;
      }
      mx[(size_t)b * G + g] = row_max;
      sm[(size_t)b * G + g] = row_sum;
    }
  }
  free(t_o);
  free(t_m);
  free(t_s);
}

enum { LATENT_W = 512, ROPE_W = 64 };

__attribute__((target_clones("avx512f", "avx2", "default")))
static void mla_tile(const float* qn, const float* qp, const uint16_t* c,
                     const uint16_t* pe, int H, int s0, int s1, float scale,
                     float* o, float* m, float* s, float* cbuf, float* pbuf) {
  enum { BLK = 8 };
  float sc[BLK];
  for (int t = s0; t < s1; t += BLK) {
    const int nb = (s1 - t) < BLK ? (s1 - t) : BLK;
    for (int r = 0; r < nb; ++r) {
      for (int d = 0; d < LATENT_W; ++d) cbuf[r * LATENT_W + d] = bf(c[(size_t)(t + r) * LATENT_W + d]);
      for (int d = 0; d < ROPE_W; ++d) pbuf[r * ROPE_W + d] = bf(pe[(size_t)(t + r) * ROPE_W + d]);
    }
    for (int h = 0; h < H; ++h) {
      const float* qh = qn + (size_t)h * LATENT_W;
      const float* qph = qp + (size_t)h * ROPE_W;
      float m_new = m[h];
      for (int r = 0; r < nb; ++r) {
        float acc = 0.f;
        const float* cr = cbuf + r * LATENT_W;
        const float* pr = pbuf + r * ROPE_W;
#pragma omp simd reduction(+ : acc)
        for (int d = 0; d < LATENT_W; ++d) acc += qh[d] * cr[d];
#pragma omp simd reduction(+ : acc)
        for (int d = 0; d < ROPE_W; ++d) acc += qph[d] * pr[d];
        sc[r] = acc * scale;
        if (sc[r] > m_new) m_new = sc[r];
      }
      const float decay = expf(m[h] - m_new);
      float blk_sum = 0.f;
      float* oh = o + (size_t)h * LATENT_W;
#pragma omp simd
      for (int d = 0; d < LATENT_W; ++d) oh[d] *= decay;
      for (int r = 0; r < nb; ++r) {
        const float e = expf(sc[r] - m_new);
        blk_sum += e;
        const float* cr = cbuf + r * LATENT_W;
#pragma omp simd
        for (int d = 0; d < LATENT_W; ++d) oh[d] += e * cr[d];
      }
      s[h] = decay * s[h] + blk_sum;
      m[h] = m_new;
    }
  }
}

/*
 * q_proj [B*H][512], q_pe [B*H][64], c_kv [B][S][512], k_pe [B][S][64] bf16
 * (contiguous).  out [B*H][512] unnormalised fp32, mx/sm [B*H] fp32.
 */
void ws_oracle_mla_compressed(const uint16_t* q_proj, const uint16_t* q_pe,
                              const uint16_t* c_kv, const uint16_t* k_pe,
                              int B, int H, int S, float scale, int n_threads,
                              float* out, float* mx, float* sm) {
#ifdef _OPENMP
  if (n_threads <= 0) n_threads = omp_get_max_threads();
#else
  n_threads = 1;
#endif
  for (int64_t i = 0; i < (int64_t)B * H; ++i) {
    mx[i] = -INFINITY;
    sm[i] = 0.f;
  }
  memset(out, 0, sizeof(float) * (size_t)B * H * LATENT_W);
  if (S <= 0 || B <= 0) return;
  int n_tiles = n_threads / B;
  if (n_tiles < 1) n_tiles = 1;
  const int tile_tokens = (S + n_tiles - 1) / n_tiles;
  const int tiles_used = (S + tile_tokens - 1) / tile_tokens;
  const int tasks = B * tiles_used;
  float* t_o = (float*)calloc((size_t)tasks * H * LATENT_W, sizeof(float));
  float* t_m = (float*)malloc(sizeof(float) * (size_t)tasks * H);
  float* t_s = (float*)calloc((size_t)tasks * H, sizeof(float));
  for (int64_t i = 0; i < (int64_t)tasks * H; ++i) t_m[i] = -INFINITY;

#pragma omp parallel num_threads(n_threads)
  {
    float* qn = (float*)malloc(sizeof(float) * (size_t)H * LATENT_W);
    float* qp = (float*)malloc(sizeof(float) * (size_t)H * ROPE_W);
    float* cbuf = (float*)malloc(sizeof(float) * 8 * LATENT_W);
    float* pbuf = (float*)malloc(sizeof(float) * 8 * ROPE_W);
#pragma omp for schedule(static)
    for (int task = 0; task < tasks; ++task) {
      const int b = task / tiles_used, ti = task % tiles_used;
      const int s0 = ti * tile_tokens;
      const int s1 = (s0 + tile_tokens < S) ? s0 + tile_tokens : S;
      for (int i = 0; i < H * LATENT_W; ++i) qn[i] = bf(q_proj[(size_t)b * H * LATENT_W + i]);
      for (int i = 0; i < H * ROPE_W; ++i) qp[i] = bf(q_pe[(size_t)b * H * ROPE_W + i]);
      mla_tile(qn, qp, c_kv + (size_t)b * S * LATENT_W, k_pe + (size_t)b * S * ROPE_W,
               H, s0, s1, scale, t_o + (size_t)task * H * LATENT_W,
               t_m + (size_t)task * H, t_s + (size_t)task * H, cbuf, pbuf);
    }
    free(qn);
    free(qp);
    free(cbuf);
    free(pbuf);
  }

  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < H; ++h) {
      float row_max = -INFINITY;
      for (int ti = 0; ti < tiles_used; ++ti) {
        const float tm = t_m[((size_t)b * tiles_used + ti) * H + h];
        if (tm > row_max) row_max = tm;
      }
      float row_sum = 0.f;
      float* og = out + ((size_t)b * H + h) * LATENT_W;
      for (int ti = 0; ti < tiles_used; ++ti) {
        const size_t tk = (size_t)b * tiles_used + ti;
        const float w = expf(t_m[tk * H + h] - row_max);
        row_sum += w * t_s[tk * H + h];
        const float* to = t_o + (tk * H + h) * LATENT_W;
        for (int d = 0; d < LATENT_W; ++d) og[d] += w * to[d];
      }
      mx[(size_t)b * H + h] = row_max;
      sm[(size_t)b * H + h] = row_sum;
    }
  }
  free(t_o);
  free(t_m);
  free(t_s);
}
