/*
 * yr_oracle.c -- CPU restatement of the fused operators on the YiRage hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP backend is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path (yirage_amd) never links or
 * calls it.
 *
 * Conventions
 *   - 16-bit tensors are passed as raw uint16 storage plus a dtype code
 *     (YO_F16 = 0, YO_BF16 = 1).  Activations that the reference keeps in a
 *     16-bit dtype between tasks are passed as float arrays whose values are
 *     already representable in that dtype (yo_round() does the rounding).
 *   - All reductions accumulate in double, which is a stricter reference than
 *     the fp32 accumulation the device kernels use.
 *   - Row-major everywhere.  Linear weights come in two layouts:
 *       YO_W_NK (0): W[N][K]  (torch Linear.weight; MPK linear task)
 *       YO_W_KN (1): W[K][N]  (kernel-graph matmul X @ W)
 *
 * Each function cites the reference file:line whose semantics it restates.
 * Functions without an independent check are marked "parity unpinned" in the
 * header comment; at present every function here is pinned by the tests in
 * tests/test_oracle.py (closed forms, brute force, invariants, known answers).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define YO_F16 0
#define YO_BF16 1
#define YO_W_NK 0
#define YO_W_KN 1

/* ------------------------------------------------------------------------ */
/* 16-bit conversions (IEEE round-to-nearest-even)                          */
/* ------------------------------------------------------------------------ */

static float g_h2f[65536];
static int g_h2f_ready = 0;

static float h2f_slow(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: renormalise */
      int e = -1;
      do { e++; man <<= 1; } while ((man & 0x400) == 0);
      man &= 0x3ff;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static void init_tables(void) {
  if (g_h2f_ready) return;
  for (int i = 0; i < 65536; i++) g_h2f[i] = h2f_slow((uint16_t)i);
  g_h2f_ready = 1;
}

float yo_h2f(uint16_t h) { init_tables(); return g_h2f[h]; }

float yo_bf2f(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t yo_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* NaN */
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

uint16_t yo_f2h(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* overflow -> inf */
  if (a < 0x38800000u) {                                            /* subnormal / zero */
    /* value = a_float; half subnormal unit = 2^-24 */
    float af;
    memcpy(&af, &a, 4);
    float scaled = af * 16777216.0f; /* exact: multiply by 2^24 */
    /* round half to even on an exact float */
    float r = nearbyintf(scaled);
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t exp = ((a >> 23) - 127 + 15);
  uint32_t man = a & 0x7fffffu;
  uint32_t h = (exp << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

static inline float ld16(const uint16_t* p, size_t i, int dt) {
  return dt == YO_F16 ? g_h2f[p[i]] : yo_bf2f(p[i]);
}

static inline float round16(float v, int dt) {
  return dt == YO_F16 ? g_h2f[yo_f2h(v)] : yo_bf2f(yo_f2bf(v));
}

void yo_to_float(const uint16_t* src, size_t n, int dt, float* dst) {
  init_tables();
  for (size_t i = 0; i < n; i++) dst[i] = ld16(src, i, dt);
}

void yo_from_float(const float* src, size_t n, int dt, uint16_t* dst) {
  for (size_t i = 0; i < n; i++) dst[i] = dt == YO_F16 ? yo_f2h(src[i]) : yo_f2bf(src[i]);
}

/* Round float values in place to the value set of a 16-bit dtype. */
void yo_round(float* a, size_t n, int dt) {
  init_tables();
  for (size_t i = 0; i < n; i++) a[i] = round16(a[i], dt);
}

/* ------------------------------------------------------------------------ */
/* Deterministic synthetic data (identical bits on host and device)          */
/* ------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Approximately N(0, std): Irwin-Hall sum of four 16-bit uniforms, centred,
 * scaled by a float constant.  Integer arithmetic up to one float multiply,
 * so the device generator reproduces it bit for bit. */
static inline float synth_normal(uint64_t seed, uint64_t idx, float scale) {
  uint64_t h = mix64(mix64(seed) ^ (idx * 0xD1342543DE82EF95ull));
  int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
              (int32_t)((h >> 32) & 0xffff) + (int32_t)((h >> 48) & 0xffff) - 131070;
  return (float)s * scale;
}

/* scale = std / 37837.2265 (sqrt(4 * (65536^2 - 1) / 12)); the same float
 * constant is computed the same way on the device side. */
float yo_synth_scale(float stddev) { return stddev / 37837.2265f; }

void yo_synth_fill(uint16_t* dst, size_t n, int dt, uint64_t seed, uint64_t offset, float stddev) {
  float sc = yo_synth_scale(stddev);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; i++) {
    float v = synth_normal(seed, offset + (uint64_t)i, sc);
    dst[i] = dt == YO_F16 ? yo_f2h(v) : yo_f2bf(v);
  }
}

void yo_synth_fill_float(float* dst, size_t n, int dt, uint64_t seed, uint64_t offset, float stddev) {
  init_tables();
  float sc = yo_synth_scale(stddev);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; i++) {
    float v = synth_normal(seed, offset + (uint64_t)i, sc);
    dst[i] = dt == YO_F16 ? g_h2f[yo_f2h(v)] : yo_bf2f(yo_f2bf(v));
  }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm                                                                  */
/* ------------------------------------------------------------------------ */

/* y = x * (rsqrt(mean(x^2) + eps) * w)
 * follows tasks/ampere/rmsnorm.cuh:76-128 (fp32 sum of squares, then
 * val *= rms_rcp * w).  w may be NULL (no affine, kernel-graph rms_norm,
 * src/kernel/rms_norm.cc:100-114). */
void yo_rmsnorm(const float* x, int rows, int H, const float* w, float eps, float* out) {
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * H;
    double ss = 0.0;
    for (int k = 0; k < H; k++) ss += (double)xr[k] * xr[k];
    double rr = 1.0 / sqrt(ss / H + (double)eps);
    for (int k = 0; k < H; k++)
      out[(size_t)r * H + k] = (float)((double)xr[k] * (rr * (w ? (double)w[k] : 1.0)));
  }
}

/* ------------------------------------------------------------------------ */
/* Linear / matmul                                                          */
/* ------------------------------------------------------------------------ */

/* out[b][n] = sum_k x[b][k] * W(k, n)  (+ residual[b][n])
 * NK layout follows tasks/ampere/linear.cuh:38-49 / linear_cutlass.cuh:34-475
 * (W row-major [N,K], fp32 accumulate, residual added to the accumulator);
 * KN layout follows the kernel-graph matmul src/kernel/matmul.cc:73-96. */
void yo_linear(const float* x, int B, int K, const uint16_t* W, int wdt, int layout, int N,
               const float* residual, float* out) {
  init_tables();
  if (layout == YO_W_NK) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
      const uint16_t* wr = W + (size_t)n * K;
      for (int b = 0; b < B; b++) {
        const float* xr = x + (size_t)b * K;
        double acc = 0.0;
        for (int k = 0; k < K; k++) acc += (double)xr[k] * ld16(wr, k, wdt);
        if (residual) acc += residual[(size_t)b * N + n];
        out[(size_t)b * N + n] = (float)acc;
      }
    }
  } else {
    int nth = 1;
#ifdef _OPENMP
    nth = omp_get_max_threads();
#endif
    int chunk = (N + nth - 1) / nth;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < nth; t++) {
      int n0 = t * chunk, n1 = n0 + chunk < N ? n0 + chunk : N;
      if (n0 >= n1) continue;
      int w = n1 - n0;
      double* acc = (double*)calloc((size_t)B * w, sizeof(double));
      for (int k = 0; k < K; k++) {
        const uint16_t* wr = W + (size_t)k * N;
        for (int b = 0; b < B; b++) {
          double xv = x[(size_t)b * K + k];
          if (xv == 0.0) continue;
          double* a = acc + (size_t)b * w;
          for (int n = n0; n < n1; n++) a[n - n0] += xv * ld16(wr, n, wdt);
        }
      }
      for (int b = 0; b < B; b++)
        for (int n = n0; n < n1; n++) {
          double v = acc[(size_t)b * w + n - n0];
          if (residual) v += residual[(size_t)b * N + n];
          out[(size_t)b * N + n] = (float)v;
        }
      free(acc);
    }
  }
}

/* Fused RMSNorm+linear of the superoptimize pattern matmul(rms_norm(X)*G, W)
 * (demo/reference_mugraphs/rms_norm.py:16-25, lowering
 * src/transpiler/transpile.cc:681-693), with the BASELINE contract
 * out = (X * rsqrt(mean(X^2) + eps) * gamma) @ W, no intermediate rounding. */
void yo_rmsnorm_linear(const float* x, int B, int K, const float* gamma, float eps,
                       const uint16_t* W, int wdt, int layout, int N, float* out) {
  float* xn = (float*)malloc(sizeof(float) * (size_t)B * K);
  yo_rmsnorm(x, B, K, gamma, eps, xn);
  yo_linear(xn, B, K, W, wdt, layout, N, NULL, out);
  free(xn);
}

/* silu(a) = a / (1 + exp(-a)) in fp32 (tasks/ampere/element_unary.cuh:41-42). */
static inline double silu_d(double a) { return a / (1.0 + exp(-a)); }

/* Gated MLP of the superoptimize pattern mul(silu(X@W1), X@W3)
 * (demo/reference_mugraphs/gated_mlp.py:75-86): both products accumulate in
 * fp32 and the SiLU-product is formed before the single output rounding. */
void yo_gated_mlp(const float* x, int B, int K, const uint16_t* W1, const uint16_t* W3, int wdt,
                  int layout, int N, float* out) {
  float* g = (float*)malloc(sizeof(float) * (size_t)B * N);
  float* u = (float*)malloc(sizeof(float) * (size_t)B * N);
  yo_linear(x, B, K, W1, wdt, layout, N, NULL, g);
  yo_linear(x, B, K, W3, wdt, layout, N, NULL, u);
  for (size_t i = 0; i < (size_t)B * N; i++) out[i] = (float)(silu_d(g[i]) * u[i]);
  free(g);
  free(u);
}

/* MPK silu_mul: out = T(silu(float(gate))) * up, i.e. the SiLU result is
 * rounded to the storage dtype before the product, and the product is rounded
 * again (tasks/ampere/silu_mul.cuh:31-40).  gate/up hold dtype values. */
void yo_silu_mul(const float* gate, const float* up, size_t n, int dt, float* out) {
  init_tables();
  for (size_t i = 0; i < n; i++) {
    float s = round16((float)silu_d(gate[i]), dt);
    out[i] = round16(s * up[i], dt);
  }
}

/* ------------------------------------------------------------------------ */
/* Rotary embedding                                                          */
/* ------------------------------------------------------------------------ */

/* Rotate-half RoPE of one head vector in place, rounded to dt
 * (tasks/ampere/rotary_embedding.cuh:22-81). cos/sin: one row of [pos, D]. */
static void rope_head(float* v, int D, const float* cs, const float* sn, int dt) {
  float tmp[1024];
  int h = D / 2;
  for (int i = 0; i < D; i++) {
    float r;
    if (i < h) r = v[i] * cs[i] - v[i + h] * sn[i];
    else r = v[i] * cs[i] + v[i - h] * sn[i];
    tmp[i] = round16(r, dt);
  }
  memcpy(v, tmp, sizeof(float) * D);
}

void yo_rope(float* x, int n_heads, int D, const float* cos_row, const float* sin_row, int dt) {
  init_tables();
  for (int h = 0; h < n_heads; h++) rope_head(x + (size_t)h * D, D, cos_row, sin_row, dt);
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

/* softmax(q.K^T * scale) . V over n rows gathered by a callback-free index
 * list; q, k, v are float vectors of length D. */
static void attend(const float* q, int D, int n, const float* const* krows, const float* const* vrows,
                   double scale, float* out) {
  double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
  double m = -INFINITY;
  for (int j = 0; j < n; j++) {
    double d = 0.0;
    for (int i = 0; i < D; i++) d += (double)q[i] * krows[j][i];
    s[j] = d * scale;
    if (s[j] > m) m = s[j];
  }
  double l = 0.0;
  for (int j = 0; j < n; j++) { s[j] = exp(s[j] - m); l += s[j]; }
  for (int i = 0; i < D; i++) {
    double o = 0.0;
    for (int j = 0; j < n; j++) o += s[j] * vrows[j][i];
    out[i] = n > 0 ? (float)(o / l) : 0.0f;
  }
  free(s);
}

/* Standalone paged GQA decode (one query token per sequence):
 * out[b][h] = softmax(q[b][h] . K_b^T / sqrt(D)) . V_b with kv head h / (Hq/Hkv).
 * Cache layout [num_pages][page][Hkv][D] (NHD, tasks/ampere/
 * multitoken_paged_attention_4_16.cuh:60-63); sequence b owns pages
 * kv_indices[kv_indptr[b] .. kv_indptr[b+1]) and has kv_len[b] tokens. */
void yo_gqa_decode_paged(const float* q, int B, int Hq, int Hkv, int D, const uint16_t* kc,
                         const uint16_t* vc, int dt, int page, const int* kv_indptr,
                         const int* kv_indices, const int* kv_len, float* out) {
  init_tables();
  int G = Hq / Hkv;
  double scale = 1.0 / sqrt((double)D);
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < B; b++) {
    for (int hk = 0; hk < Hkv; hk++) {
      int n = kv_len[b];
      float* kf = (float*)malloc(sizeof(float) * (size_t)n * D);
      float* vf = (float*)malloc(sizeof(float) * (size_t)n * D);
      const float** kr = (const float**)malloc(sizeof(float*) * (size_t)(n > 0 ? n : 1));
      const float** vr = (const float**)malloc(sizeof(float*) * (size_t)(n > 0 ? n : 1));
      for (int t = 0; t < n; t++) {
        int pg = kv_indices[kv_indptr[b] + t / page];
        size_t base = (((size_t)pg * page + t % page) * Hkv + hk) * D;
        for (int i = 0; i < D; i++) {
          kf[(size_t)t * D + i] = ld16(kc, base + i, dt);
          vf[(size_t)t * D + i] = ld16(vc, base + i, dt);
        }
        kr[t] = kf + (size_t)t * D;
        vr[t] = vf + (size_t)t * D;
      }
      for (int g = 0; g < G; g++) {
        int h = hk * G + g;
        attend(q + ((size_t)b * Hq + h) * D, D, n, kr, vr, scale, out + ((size_t)b * Hq + h) * D);
      }
      free(kf); free(vf); free(kr); free(vr);
    }
  }
}

/* Causal GQA prefill, layout Q[B][S][Hq][D], K/V[B][S][Hkv][D], O like Q.
 * Query token i attends keys 0..i (mask col <= row, multitoken_paged_
 * attention_4_16.cuh:40-656 with seq_len == num_tokens).  Only query rows
 * listed in rows[0..n_rows) are computed (n_rows < 0: all rows), so the
 * full-size case can be checked on a sample. */
void yo_gqa_prefill(const float* q, const float* k, const float* v, int B, int S, int Hq, int Hkv,
                    int D, int causal, const int* rows, int n_rows, float* out) {
  int G = Hq / Hkv;
  double scale = 1.0 / sqrt((double)D);
  int nr = n_rows < 0 ? S : n_rows;
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int b = 0; b < B; b++)
    for (int ri = 0; ri < nr; ri++)
      for (int h = 0; h < Hq; h++) {
        int i = n_rows < 0 ? ri : rows[ri];
        int hk = h / G;
        int n = causal ? i + 1 : S;
        const float** kr = (const float**)malloc(sizeof(float*) * (size_t)n);
        const float** vr = (const float**)malloc(sizeof(float*) * (size_t)n);
        for (int t = 0; t < n; t++) {
          kr[t] = k + (((size_t)b * S + t) * Hkv + hk) * D;
          vr[t] = v + (((size_t)b * S + t) * Hkv + hk) * D;
        }
        attend(q + (((size_t)b * S + i) * Hq + h) * D, D, n, kr, vr, scale,
               out + (((size_t)b * S + i) * Hq + h) * D);
        free(kr); free(vr);
      }
}

/* MPK paged attention task (tasks/ampere/multitoken_paged_attention_4_16.cuh
 * :40-656): for each request r the new tokens qo_indptr[r]..qo_indptr[r+1]
 * carry packed per-kv-group rows [q * G | k | v] (QKV shuffled per group,
 * demo/llama3/demo.py:508-514).  q and k are RoPE-rotated and rounded to dt,
 * the new k/v are appended to the paged cache, and each new token attends
 * causally to every cached position up to its own.
 * seq_len = (pages - 1) * page + last_page_len, with last_page_len == 0 read as
 * a full last page (the page manager writes 0 for an exactly full page,
 * persistent_kernel.cuh:250-251).  cos/sin may be NULL (no RoPE). */
/* Per-head RMSNorm of q / k before RoPE (qk_norm of the reference's paged
 * attention task: multitoken_paged_attention_4_16.cuh:348-375 calling
 * tasks/ampere/norm.cuh:21-126): x_i * rsqrt(mean(x^2) + eps) * w_i, stored
 * back in the activation type before the rotation reads it. */
static void qk_norm_head(float* v, int D, const float* w, double eps, int dt) {
  double ss = 0.0;
  for (int i = 0; i < D; i++) ss += (double)v[i] * v[i];
  const double rcp = 1.0 / sqrt(ss / D + eps);
  for (int i = 0; i < D; i++) v[i] = round16((float)(v[i] * rcp * w[i]), dt);
}

void yo_paged_attention(const float* qkv, int Hq, int Hkv, int D, uint16_t* kc, uint16_t* vc, int dt,
                        int page, int R, const int* qo_indptr, const int* kv_indptr,
                        const int* kv_indices, const int* last_page_len, const float* cos_t,
                        const float* sin_t, const float* q_norm, const float* k_norm, float qk_eps,
                        float* out) {
  init_tables();
  int G = Hq / Hkv;
  int row = (Hq + 2 * Hkv) * D;
  double scale = 1.0 / sqrt((double)D);
  for (int r = 0; r < R; r++) {
    int t0 = qo_indptr[r], t1 = qo_indptr[r + 1];
    int nt = t1 - t0;
    if (nt <= 0) continue;
    int np = kv_indptr[r + 1] - kv_indptr[r];
    int lpl = last_page_len[r] == 0 ? page : last_page_len[r];
    int seq_len = (np - 1) * page + lpl;
    int base = seq_len - nt;
    float qbuf[1024];
    /* append new k/v (RoPE on k) */
    for (int j = 0; j < nt; j++) {
      int pos = base + j;
      const float* src = qkv + (size_t)(t0 + j) * row;
      for (int hk = 0; hk < Hkv; hk++) {
        float kb[1024];
        memcpy(kb, src + (size_t)hk * (G + 2) * D + (size_t)G * D, sizeof(float) * D);
        if (k_norm) qk_norm_head(kb, D, k_norm, qk_eps, dt);
        if (cos_t) rope_head(kb, D, cos_t + (size_t)pos * D, sin_t + (size_t)pos * D, dt);
        const float* vb = src + (size_t)hk * (G + 2) * D + (size_t)(G + 1) * D;
        int pg = kv_indices[kv_indptr[r] + pos / page];
        size_t cbase = (((size_t)pg * page + pos % page) * Hkv + hk) * D;
        for (int i = 0; i < D; i++) {
          kc[cbase + i] = dt == YO_F16 ? yo_f2h(kb[i]) : yo_f2bf(kb[i]);
          vc[cbase + i] = dt == YO_F16 ? yo_f2h(vb[i]) : yo_f2bf(vb[i]);
        }
      }
    }
    /* attend */
    for (int hk = 0; hk < Hkv; hk++) {
      float* kf = (float*)malloc(sizeof(float) * (size_t)seq_len * D);
      float* vf = (float*)malloc(sizeof(float) * (size_t)seq_len * D);
      const float** kr = (const float**)malloc(sizeof(float*) * (size_t)seq_len);
      const float** vr = (const float**)malloc(sizeof(float*) * (size_t)seq_len);
      for (int t = 0; t < seq_len; t++) {
        int pg = kv_indices[kv_indptr[r] + t / page];
        size_t cbase = (((size_t)pg * page + t % page) * Hkv + hk) * D;
        for (int i = 0; i < D; i++) {
          kf[(size_t)t * D + i] = ld16(kc, cbase + i, dt);
          vf[(size_t)t * D + i] = ld16(vc, cbase + i, dt);
        }
        kr[t] = kf + (size_t)t * D;
        vr[t] = vf + (size_t)t * D;
      }
      for (int j = 0; j < nt; j++) {
        int pos = base + j;
        const float* src = qkv + (size_t)(t0 + j) * row + (size_t)hk * (G + 2) * D;
        for (int g = 0; g < G; g++) {
          memcpy(qbuf, src + (size_t)g * D, sizeof(float) * D);
          if (q_norm) qk_norm_head(qbuf, D, q_norm, qk_eps, dt);
          if (cos_t) rope_head(qbuf, D, cos_t + (size_t)pos * D, sin_t + (size_t)pos * D, dt);
          attend(qbuf, D, pos + 1, kr, vr, scale,
                 out + (size_t)(t0 + j) * Hq * D + (size_t)(hk * G + g) * D);
        }
      }
      free(kf); free(vf); free(kr); free(vr);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Argmax / embedding                                                        */
/* ------------------------------------------------------------------------ */

/* Row-wise argmax, lowest index on ties (torch.argmax semantics); the
 * reference's partial+reduce scheme (tasks/ampere/argmax.cuh:71-155) leaves
 * the tie-break unspecified, so the build fixes it here.  Only the first
 * n_valid columns of each row of width V take part (vocab padding is masked). */
void yo_argmax(const float* x, int rows, int V, int n_valid, int64_t* out) {
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * V;
    int64_t best = -1;
    float bv = -INFINITY;
    for (int i = 0; i < n_valid; i++)
      if (best < 0 || xr[i] > bv) { bv = xr[i]; best = i; }
    out[r] = best;
  }
}

/* ------------------------------------------------------------------------ */
/* Offline batch / page manager (persistent_kernel.cuh:107-132, 169-322)     */
/* ------------------------------------------------------------------------ */

typedef struct {
  int max_requests;      /* YPK_MAX_NUM_BATCHED_REQUESTS */
  int max_tokens;        /* YPK_MAX_NUM_BATCHED_TOKENS */
  int max_pages;         /* YPK_MAX_NUM_PAGES */
  int page_size;         /* YPK_PAGE_SIZE */
  int max_seq_length;    /* YPK_MAX_SEQ_LENGTH (row stride of tokens) */
  int total_num_requests;
  int64_t eos_token_id;
  int* step;             /* [total_num_requests] */
  int64_t* tokens;       /* [total_num_requests][max_seq_length] */
  int64_t* input_tokens; /* [max_tokens] */
  int64_t* output_tokens;/* [max_tokens] */
  int* prompt_length;    /* [total_num_requests] */
  int* qo_indptr;        /* [max_requests + 1] */
  int* kv_indptr;        /* [max_requests + 1] */
  int* kv_indices;       /* [max_pages] */
  int* last_page_len;    /* [max_requests] */
  int* request_ids;      /* [max_requests] */
  int* next_request_id;  /* [1] */
  int* page_queue;       /* [max_pages] */
  int* page_queue_head;  /* [1] */
  int* page_queue_tail;  /* [1] */
} yo_batch_state;

void yo_batch_init(yo_batch_state* s) {
  for (int i = 0; i < s->total_num_requests; i++) s->step[i] = 0;
  *s->next_request_id = 0;
  for (int i = 0; i < s->max_requests; i++) s->request_ids[i] = -1;
  for (int i = 0; i < s->max_requests + 1; i++) { s->qo_indptr[i] = 0; s->kv_indptr[i] = 0; }
  *s->page_queue_head = 0;
  *s->page_queue_tail = s->max_pages;
  for (int i = 0; i < s->max_pages; i++) s->page_queue[i] = i;
}

static int imin(int a, int b) { return a < b ? a : b; }

/* Returns 1 when the next batch holds at least one token. */
int yo_batch_prepare_next(yo_batch_state* s) {
  const int MR = s->max_requests, MT = s->max_tokens, MP = s->max_pages, PS = s->page_size;
  const int MSL = s->max_seq_length;
  int head = *s->page_queue_head, tail = *s->page_queue_tail;
  /* finalize the previous batch */
  for (int i = 0; i < MR; i++) {
    int rid = s->request_ids[i];
    if (rid == -1) continue;
    int step = s->step[rid];
    int qo = s->qo_indptr[i];
    int nt = s->qo_indptr[i + 1] - qo;
    int plen = s->prompt_length[rid];
    for (int j = 0; j < nt; j++)
      if (step + j + 1 >= plen && step + j + 1 < MSL)
        s->tokens[(size_t)rid * MSL + step + j + 1] = s->output_tokens[qo + j];
    s->step[rid] = step + nt;
    if ((step + nt + 1 >= MSL) ||
        ((s->tokens[(size_t)rid * MSL + step + nt] == s->eos_token_id) && (step + nt >= plen))) {
      s->request_ids[i] = -1;
      int kp = s->kv_indptr[i];
      int np = s->kv_indptr[i + 1] - kp;
      for (int j = 0; j < np; j++) { s->page_queue[tail % MP] = s->kv_indices[kp + j]; tail++; }
    }
  }
  /* snapshot of the page table */
  int npages_all = s->kv_indptr[MR];
  int* snap = (int*)malloc(sizeof(int) * (size_t)(npages_all > 0 ? npages_all : 1));
  for (int i = 0; i < npages_all; i++) snap[i] = s->kv_indices[i];
  int nreq = 0, ntok = 0, npg = 0;
  for (int i = 0; i < MR; i++) {
    int rid = s->request_ids[i];
    if (rid == -1) continue;
    int kp = s->kv_indptr[i];
    int nold = s->kv_indptr[i + 1] - kp;
    s->request_ids[nreq] = rid;
    s->qo_indptr[nreq] = ntok;
    s->kv_indptr[nreq] = npg;
    int step = s->step[rid];
    int nnew = s->prompt_length[rid] - step;
    if (nnew > 0) nnew = imin(nnew, MT - ntok);
    else nnew = imin(1, MT - ntok);
    for (int j = 0; j < nnew; j++) s->input_tokens[ntok + j] = s->tokens[(size_t)rid * MSL + step + j];
    int nnp = (step + nnew + PS - 1) / PS;
    s->last_page_len[nreq] = (step + nnew) % PS;
    for (int j = 0; j < nold; j++) s->kv_indices[npg + j] = snap[kp + j];
    for (int j = nold; j < nnp; j++) { s->kv_indices[npg + j] = s->page_queue[head % MP]; head++; }
    npg += nnp;
    ntok += nnew;
    nreq++;
  }
  free(snap);
  while (nreq < MR && ntok < MT) {
    int nid = *s->next_request_id;
    if (nid >= s->total_num_requests) break;
    s->request_ids[nreq] = nid;
    s->qo_indptr[nreq] = ntok;
    s->kv_indptr[nreq] = npg;
    int nnew = imin(s->prompt_length[nid], MT - ntok);
    for (int j = 0; j < nnew; j++) s->input_tokens[ntok + j] = s->tokens[(size_t)nid * MSL + j];
    int nnp = (nnew + PS - 1) / PS;
    s->last_page_len[nreq] = nnew % PS;
    for (int j = 0; j < nnp; j++) { s->kv_indices[npg + j] = s->page_queue[head % MP]; head++; }
    ntok += nnew;
    npg += nnp;
    nreq++;
    *s->next_request_id = nid + 1;
  }
  for (int i = nreq; i < MR; i++) s->request_ids[i] = -1;
  for (int i = nreq; i <= MR; i++) { s->qo_indptr[i] = ntok; s->kv_indptr[i] = npg; }
  *s->page_queue_head = head;
  *s->page_queue_tail = tail;
  return ntok != 0;
}

/* Online-mode prepare_next_batch (persistent_kernel.cuh:325-351): one
 * request whose host feeds the number of tokens it accepted this step
 * (new_token_nums[0], the meta tensor num_new_tokens); the step advances by
 * it, and the run continues unless the old step + 2 reaches max_seq_length or
 * the token after the old step is eos.  Returns 1 to continue. */
int yo_batch_prepare_online(yo_batch_state* s, const int* new_token_nums) {
  const int step = s->step[0];
  s->step[0] = step + new_token_nums[0];
  if (step + 2 >= s->max_seq_length || s->tokens[step + 1] == s->eos_token_id) return 0;
  return 1;
}

int yo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void yo_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
