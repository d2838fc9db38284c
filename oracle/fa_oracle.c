/*
 * fa_oracle.c -- CPU fp32 restatement of the reference's flow-matching denoise loops.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the MI355X kernels: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product path (flashact_amd/) never links, imports or calls it.
 *
 * Restated algorithms (reference = /root/reference, read-only):
 *   pi0.5 action expert, one Euler loop ......... src/pi05/mk6.cu:279-518 (stage order),
 *       adaRMS + gated residual ................. src/pi05/mk6.cu:137-164, 302, 429, 499-505
 *       QKV + split-half RoPE ................... src/pi05/mk6.cu:221-244 (pairs j, j+128)
 *       MQA over prefix + own suffix keys ...... src/pi05/mk6.cu:312-421 (scale 1/16)
 *       GeLU(tanh)-gated MLP .................... src/pi05/mk6.cu:79-82, 434-497
 *       final norm + action_out + Euler ......... src/pi05/mk6.cu:502-517 (dt = -1/S)
 *       time embedding / time MLP / mods ........ src/pi05/hybrid_model.py:111-128,
 *                                                 src/pi05/pack_weights.py:23-31
 *       RoPE table .............................. src/pi05/pack_weights.py:54-58
 *       FP8-W8A16 weights (fo_pi05_denoise_fp8) . e4m3 codes + per-row scales (hybrid_model.py:105-110),
 *                                                 row sum times scale (mk6.cu:204-225)
 *   MolmoAct2 action expert ..................... src/molmoact2/mk_ma2.cu:258-575
 *       adaLN norm ............................... src/molmoact2/mk_ma2.cu:130-158
 *       self-attn qk-norm + RoPE (48 pairs) ..... src/molmoact2/mk_ma2.cu:292-381
 *       cross-attn over per-layer context KV .... src/molmoact2/mk_ma2.cu:397-529
 *       SiLU-gated MLP ........................... src/molmoact2/mk_ma2.cu:246-251, 542-552
 *       final layer + masked Euler (dt = +1/S) .. src/molmoact2/mk_ma2.cu:558-571
 *   Gemma-2B backbone prefix prefill ............ openpi PaliGemma forward with use_cache, called at
 *       (config 3)                                benchmarks/pi05/eval_numerics.py:50-57 (openpi is
 *                                                 absent: restated from the Gemma decoder layer and
 *                                                 pinned against transformers' GemmaDecoderLayer);
 *       K/V kept per layer ...................... src/pi05/pack_weights.py:60-70 (compact_kv)
 *
 * Weights use the reference's natural (unpacked) layouts, [out][in] row-major, stored as
 * bf16 bit patterns (uint16). Every value is converted exactly to fp32 and all arithmetic
 * is fp32 (the CPU reference workload), so the oracle and the GPU path see identical inputs and
 * differ only in arithmetic precision. Pins: see tests/test_oracle_*.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE 754 binary16 -> fp32 (exact): sign, 5-bit exponent (bias 15), 10-bit fraction; exponent 0
 * holds the subnormals frac * 2^-24, exponent 31 the infinities and NaNs. */
static inline float h2f(uint16_t h) {
  const int sgn = h >> 15, ex = (h >> 10) & 31, fr = h & 1023;
  float v;
  if (ex == 0) v = ldexpf((float)fr, -24);
  else if (ex == 31) v = fr ? NAN : INFINITY;
  else v = ldexpf((float)(1024 + fr), ex - 25);
  return sgn ? -v : v;
}

void fo_f16_decode(const uint16_t* bits, int n, float* out) {
  for (int i = 0; i < n; i++) out[i] = h2f(bits[i]);
}

static inline float dot_f32(const float* a, const float* b, int n) {
  /* 8 independent partial sums so the compiler can vectorise without -ffast-math */
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; j++) s[j] += a[i + j] * b[i + j];
  float r = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
  for (; i < n; i++) r += a[i] * b[i];
  return r;
}

int fo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* The 2 x 4 dot products of rows x0, x1 with rows w[0..3] (stride K), K a multiple of 8. Each keeps
 * dot_f32's eight partial sums and their reduction order, so every result equals dot_f32's; the
 * blocking only lets one load of x serve four weight rows. */
static inline void dot_2x4(const float* x0, const float* x1, const float* w, int K, float r[2][4]) {
  __m256 s[2][4];
  for (int b = 0; b < 4; b++) s[0][b] = s[1][b] = _mm256_setzero_ps();
  for (int i = 0; i < K; i += 8) {
    const __m256 a0 = _mm256_loadu_ps(x0 + i), a1 = _mm256_loadu_ps(x1 + i);
    for (int b = 0; b < 4; b++) {
      const __m256 wv = _mm256_loadu_ps(w + (size_t)b * K + i);
      s[0][b] = _mm256_fmadd_ps(a0, wv, s[0][b]);
      s[1][b] = _mm256_fmadd_ps(a1, wv, s[1][b]);
    }
  }
  for (int a = 0; a < 2; a++)
    for (int b = 0; b < 4; b++) {
      float t[8];
      _mm256_storeu_ps(t, s[a][b]);
      r[a][b] = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    }
}

/* Y[m][n] = sum_k X[m][k] * W[n][k] (+ bias[n]); W bf16 [N][K]. Weight rows are converted to fp32 in
 * blocks of four and each pair of X rows is multiplied with the block (dot_2x4). */
static void linear_bf16(const float* X, int M, int K, const uint16_t* W, const float* bias, int N, float* Y) {
#pragma omp parallel
  {
    float* wrow = (float*)malloc(sizeof(float) * 4 * (size_t)K);
#pragma omp for schedule(static)
    for (int n0 = 0; n0 < N; n0 += 4) {
      const int nb = N - n0 < 4 ? N - n0 : 4;
      for (int j = 0; j < nb; j++) {
        const uint16_t* w = W + (size_t)(n0 + j) * K;
        for (int k = 0; k < K; k++) wrow[(size_t)j * K + k] = bf(w[k]);
      }
      int m = 0;
      if (nb == 4 && K % 8 == 0) {
        for (; m + 2 <= M; m += 2) {
          float r[2][4];
          dot_2x4(X + (size_t)m * K, X + (size_t)(m + 1) * K, wrow, K, r);
          for (int a = 0; a < 2; a++)
            for (int j = 0; j < 4; j++) Y[(size_t)(m + a) * N + n0 + j] = r[a][j] + (bias ? bias[n0 + j] : 0.f);
        }
      }
      for (; m < M; m++)
        for (int j = 0; j < nb; j++)
          Y[(size_t)m * N + n0 + j] = dot_f32(X + (size_t)m * K, wrow + (size_t)j * K, K) + (bias ? bias[n0 + j] : 0.f);
    }
    free(wrow);
  }
}

/* Y[m][n] = sum_k X[m][k] * W[n][k] + bias[n]; W fp32 [N][K]. */
static void linear_f32(const float* X, int M, int K, const float* W, const float* bias, int N, float* Y) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    float b = bias ? bias[n] : 0.f;
    for (int m = 0; m < M; m++) Y[(size_t)m * N + n] = dot_f32(X + (size_t)m * K, W + (size_t)n * K, K) + b;
  }
}

/* OCP E4M3 (e4m3fn): e == 0 -> m 2^-9, else (1 + m/8) 2^(e-7); codes 0x7f / 0xff are NaN. */
static inline float e4m3(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7)
    v = NAN;
  else if (e == 0)
    v = ldexpf((float)m, -9);
  else
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return (c & 0x80) ? -v : v;
}

void fo_e4m3_decode(const uint8_t* codes, int n, float* out) {
  for (int i = 0; i < n; i++) out[i] = e4m3(codes[i]);
}

/* A stack of weight matrices [..][N][K]: bf16 bits, or e4m3 codes with one fp32 scale per row. */
typedef struct {
  const uint16_t* bf;
  const uint8_t* q;
  const float* s;
} fo_wmat;

/* Y[m][n] = sum_k X[m][k] W[row0 + n][k]; for e4m3 weights the row sum is multiplied by the row's
 * scale afterwards, (sum_k x_k q_nk) s_n, as the reference's W8A16 GEMM does (mk6.cu:204-225). */
static void linear_w(const float* X, int M, int K, fo_wmat W, size_t row0, int N, float* Y) {
  if (!W.q) {
    linear_bf16(X, M, K, W.bf + row0 * (size_t)K, NULL, N, Y);
    return;
  }
#pragma omp parallel
  {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; n++) {
      const uint8_t* w = W.q + (row0 + (size_t)n) * K;
      for (int k = 0; k < K; k++) wrow[k] = e4m3(w[k]);
      const float sc = W.s[row0 + n];
      for (int m = 0; m < M; m++) Y[(size_t)m * N + n] = dot_f32(X + (size_t)m * K, wrow, K) * sc;
    }
    free(wrow);
  }
}

static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
static inline float gelu_tanh_f(float x) {
  /* GeLU, tanh approximation (Hendrycks & Gimpel 2016), as used by mk6.cu:79-82 */
  const float k0 = 0.7978845608028654f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + 0.044715f * x * x * x)));
}

/* adaRMS: h = x * rsqrt(mean(x^2) + eps) * (1 + scale) + shift   (mk6.cu:145-161) */
static void ada_rms(const float* x, int M, int Dm, const float* scale, const float* shift, float* h) {
  for (int m = 0; m < M; m++) {
    const float* xr = x + (size_t)m * Dm;
    float ss = dot_f32(xr, xr, Dm);
    float r = 1.0f / sqrtf(ss / (float)Dm + 1e-6f);
    for (int d = 0; d < Dm; d++) h[(size_t)m * Dm + d] = xr[d] * r * (1.0f + scale[d]) + shift[d];
  }
}

/* ------------------------------------------------------------------ */
/* pi0.5 time conditioning (hybrid_model.py:111-128)                   */
/* ------------------------------------------------------------------ */

/* openpi create_sinusoidal_pos_embedding: fraction = linspace(0,1,dim/2) (fp64),
 * period = min * (max/min)^fraction, freq = 2*pi/period, out = [sin(freq*t), cos(freq*t)]
 * computed in fp64 and rounded to fp32 (pack_weights.py:26-31). */
void fo_sinusoid_embedding(const float* t, int n, int dim, double min_period, double max_period, float* out) {
  int half = dim / 2;
  for (int i = 0; i < n; i++) {
    for (int k = 0; k < half; k++) {
      double frac = (half > 1) ? (double)k / (double)(half - 1) : 0.0;
      double period = min_period * pow(max_period / min_period, frac);
      double arg = (1.0 / period * 2.0 * M_PI) * (double)t[i];
      out[(size_t)i * dim + k] = (float)sin(arg);
      out[(size_t)i * dim + half + k] = (float)cos(arg);
    }
  }
}

/* mods[s][l][0|1][3D] and mod_final[s][3D] for the fixed schedule t_s = 1 - s/S.
 * cond = silu(W_to silu(W_ti temb + b_ti) + b_to); mod = W_dense cond + b_dense.
 * Weights fp32: w_ti/w_to [D][D], w_in/w_post [NL][3D][D], w_fin [3D][D]. */
void fo_pi05_mods(int S, int NL, int D, const float* w_ti, const float* b_ti, const float* w_to, const float* b_to,
                  const float* w_in, const float* b_in, const float* w_post, const float* b_post,
                  const float* w_fin, const float* b_fin, float* mods, float* mod_final) {
  float* tt = (float*)malloc(sizeof(float) * S);
  for (int s = 0; s < S; s++) tt[s] = 1.0f - (float)s / (float)S;
  float* temb = (float*)malloc(sizeof(float) * (size_t)S * D);
  float* a = (float*)malloc(sizeof(float) * (size_t)S * D);
  float* cond = (float*)malloc(sizeof(float) * (size_t)S * D);
  float* m = (float*)malloc(sizeof(float) * (size_t)S * 3 * D);
  fo_sinusoid_embedding(tt, S, D, 4e-3, 4.0, temb);
  linear_f32(temb, S, D, w_ti, b_ti, D, a);
  for (size_t i = 0; i < (size_t)S * D; i++) a[i] = silu_f(a[i]);
  linear_f32(a, S, D, w_to, b_to, D, cond);
  for (size_t i = 0; i < (size_t)S * D; i++) cond[i] = silu_f(cond[i]);
  for (int l = 0; l < NL; l++) {
    for (int k = 0; k < 2; k++) {
      const float* W = (k == 0 ? w_in : w_post) + (size_t)l * 3 * D * D;
      const float* B = (k == 0 ? b_in : b_post) + (size_t)l * 3 * D;
      linear_f32(cond, S, D, W, B, 3 * D, m);
      for (int s = 0; s < S; s++)
        memcpy(mods + (((size_t)s * NL + l) * 2 + k) * 3 * D, m + (size_t)s * 3 * D, sizeof(float) * 3 * D);
    }
  }
  linear_f32(cond, S, D, w_fin, b_fin, 3 * D, mod_final);
  free(tt); free(temb); free(a); free(cond); free(m);
}

/* RoPE table (pack_weights.py:54-58): inv_freq_j = 1 / 10000^(2j/HD) in fp32,
 * angle = pos * inv_freq_j in fp32, pos = start + t. cos/sin [T][HD/2]. */
void fo_rope_table(int start, int T, int HD, double base, float* cosv, float* sinv) {
  int half = HD / 2;
  for (int t = 0; t < T; t++) {
    float pos = (float)(start + t);
    for (int j = 0; j < half; j++) {
      float invf = 1.0f / powf((float)base, (float)(2 * j) / (float)HD);
      float ang = pos * invf;
      cosv[(size_t)t * half + j] = cosf(ang);
      sinv[(size_t)t * half + j] = sinf(ang);
    }
  }
}

/* ------------------------------------------------------------------ */
/* pi0.5 denoise loop (mk6.cu:279-518)                                 */
/* ------------------------------------------------------------------ */
typedef struct {
  int NL, D, H, HD, F, AD;
  int Lp, Tv, S, batch;
  int kv_f16; /* 0: kpre / vpre hold bf16 bits; 1: fp16 bits (the reference's cache dtype) */
} fo_pi05_dims;

/* Weights (bf16 bits, natural layouts):
 *   wq [NL][H*HD][D], wk [NL][HD][D], wv [NL][HD][D], wo [NL][D][H*HD],
 *   wg [NL][F][D], wu [NL][F][D], wd [NL][D][F]
 * mods [S][NL][2][3D] (scale|shift|gate), mod_final [S][3D]
 * rope_cos/sin [Tv][HD/2] for positions Lp + t
 * w_ain [D][AD], b_ain [D], w_aout [AD][D], b_aout [AD] (fp32)
 * kpre, vpre [batch][NL][Lp][HD] bf16, or fp16 with kv_f16 (already-RoPE'd prefix keys, values)
 * x_t [batch][Tv][AD] fp32, updated in place. */
static int pi05_loop(const fo_pi05_dims* dm, fo_wmat wq, fo_wmat wk, fo_wmat wv, fo_wmat wo, fo_wmat wg, fo_wmat wu,
                     fo_wmat wd, const float* mods, const float* mod_final, const float* rope_cos,
                     const float* rope_sin, const float* w_ain, const float* b_ain, const float* w_aout,
                     const float* b_aout, const uint16_t* kpre, const uint16_t* vpre, float* x_t) {
  const int NL = dm->NL, D = dm->D, H = dm->H, HD = dm->HD, F = dm->F, AD = dm->AD;
  const int Lp = dm->Lp, Tv = dm->Tv, S = dm->S, B = dm->batch;
  const int QD = H * HD, half = HD / 2, L = Lp + Tv;
  if (NL < 1 || D < 1 || H < 1 || HD < 2 || (HD & 1) || F < 1 || AD < 1 || Lp < 0 || Tv < 1 || S < 1 || B < 1) return -1;
  const float dt = -1.0f / (float)S;
  const float scale = 1.0f / sqrtf((float)HD);

  float* x = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* h = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* q = (float*)malloc(sizeof(float) * (size_t)Tv * QD);
  float* k = (float*)malloc(sizeof(float) * (size_t)Tv * HD);
  float* v = (float*)malloc(sizeof(float) * (size_t)Tv * HD);
  float* att = (float*)malloc(sizeof(float) * (size_t)Tv * QD);
  float* o = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* g = (float*)malloc(sizeof(float) * (size_t)Tv * F);
  float* u = (float*)malloc(sizeof(float) * (size_t)Tv * F);
  float* Kl = (float*)malloc(sizeof(float) * (size_t)L * HD);
  float* Vl = (float*)malloc(sizeof(float) * (size_t)L * HD);
  float* act = (float*)malloc(sizeof(float) * (size_t)Tv * AD);

  for (int b = 0; b < B; b++) {
    float* xt = x_t + (size_t)b * Tv * AD;
    for (int s = 0; s < S; s++) {
      /* embed (mk6.cu:280-288) */
      linear_f32(xt, Tv, AD, w_ain, b_ain, D, x);
      for (int l = 0; l < NL; l++) {
        const float* mod_in = mods + (((size_t)s * NL + l) * 2 + 0) * 3 * D;
        const float* mod_post = mods + (((size_t)s * NL + l) * 2 + 1) * 3 * D;
        /* attention block */
        ada_rms(x, Tv, D, mod_in, mod_in + D, h);
        linear_w(h, Tv, D, wq, (size_t)l * QD, QD, q);
        linear_w(h, Tv, D, wk, (size_t)l * HD, HD, k);
        linear_w(h, Tv, D, wv, (size_t)l * HD, HD, v);
        for (int t = 0; t < Tv; t++) {
          const float* c = rope_cos + (size_t)t * half;
          const float* sn = rope_sin + (size_t)t * half;
          for (int hh = 0; hh <= H; hh++) {
            float* vec = (hh < H) ? q + (size_t)t * QD + (size_t)hh * HD : k + (size_t)t * HD;
            for (int j = 0; j < half; j++) {
              float a0 = vec[j], a1 = vec[j + half];
              vec[j] = a0 * c[j] - a1 * sn[j];
              vec[j + half] = a1 * c[j] + a0 * sn[j];
            }
          }
        }
        const uint16_t* kp = kpre + (((size_t)b * NL + l) * Lp) * HD;
        const uint16_t* vp = vpre + (((size_t)b * NL + l) * Lp) * HD;
        if (dm->kv_f16)
          for (size_t i = 0; i < (size_t)Lp * HD; i++) { Kl[i] = h2f(kp[i]); Vl[i] = h2f(vp[i]); }
        else
          for (size_t i = 0; i < (size_t)Lp * HD; i++) { Kl[i] = bf(kp[i]); Vl[i] = bf(vp[i]); }
        memcpy(Kl + (size_t)Lp * HD, k, sizeof(float) * (size_t)Tv * HD);
        memcpy(Vl + (size_t)Lp * HD, v, sizeof(float) * (size_t)Tv * HD);
#pragma omp parallel
        {
          float* p = (float*)malloc(sizeof(float) * (size_t)L);
#pragma omp for schedule(static)
          for (int th = 0; th < Tv * H; th++) {
            int t = th / H, hh = th % H;
            const float* qv = q + (size_t)t * QD + (size_t)hh * HD;
            float mx = -INFINITY;
            for (int j = 0; j < L; j++) {
              p[j] = dot_f32(qv, Kl + (size_t)j * HD, HD) * scale;
              if (p[j] > mx) mx = p[j];
            }
            float sum = 0.f;
            for (int j = 0; j < L; j++) { p[j] = expf(p[j] - mx); sum += p[j]; }
            float inv = 1.0f / sum;
            float* out = att + (size_t)t * QD + (size_t)hh * HD;
            for (int d = 0; d < HD; d++) out[d] = 0.f;
            for (int j = 0; j < L; j++) {
              float w = p[j] * inv;
              const float* vr = Vl + (size_t)j * HD;
              for (int d = 0; d < HD; d++) out[d] += w * vr[d];
            }
          }
          free(p);
        }
        linear_w(att, Tv, QD, wo, (size_t)l * D, D, o);
        for (int t = 0; t < Tv; t++)
          for (int d = 0; d < D; d++) x[(size_t)t * D + d] += mod_in[2 * D + d] * o[(size_t)t * D + d];
        /* MLP block */
        ada_rms(x, Tv, D, mod_post, mod_post + D, h);
        linear_w(h, Tv, D, wg, (size_t)l * F, F, g);
        linear_w(h, Tv, D, wu, (size_t)l * F, F, u);
        for (size_t i = 0; i < (size_t)Tv * F; i++) g[i] = gelu_tanh_f(g[i]) * u[i];
        linear_w(g, Tv, F, wd, (size_t)l * D, D, o);
        for (int t = 0; t < Tv; t++)
          for (int d = 0; d < D; d++) x[(size_t)t * D + d] += mod_post[2 * D + d] * o[(size_t)t * D + d];
      }
      /* final norm + action_out + Euler (mk6.cu:502-517) */
      const float* mf = mod_final + (size_t)s * 3 * D;
      ada_rms(x, Tv, D, mf, mf + D, h);
      linear_f32(h, Tv, D, w_aout, b_aout, AD, act);
      for (size_t i = 0; i < (size_t)Tv * AD; i++) xt[i] += dt * act[i];
    }
  }
  free(x); free(h); free(q); free(k); free(v); free(att); free(o); free(g); free(u);
  free(Kl); free(Vl); free(act);
  return 0;
}

int fo_pi05_denoise(const fo_pi05_dims* dm, const uint16_t* wq, const uint16_t* wk, const uint16_t* wv,
                    const uint16_t* wo, const uint16_t* wg, const uint16_t* wu, const uint16_t* wd,
                    const float* mods, const float* mod_final, const float* rope_cos, const float* rope_sin,
                    const float* w_ain, const float* b_ain, const float* w_aout, const float* b_aout,
                    const uint16_t* kpre, const uint16_t* vpre, float* x_t) {
  const fo_wmat W[7] = {{wq, NULL, NULL}, {wk, NULL, NULL}, {wv, NULL, NULL}, {wo, NULL, NULL},
                        {wg, NULL, NULL}, {wu, NULL, NULL}, {wd, NULL, NULL}};
  return pi05_loop(dm, W[0], W[1], W[2], W[3], W[4], W[5], W[6], mods, mod_final, rope_cos, rope_sin, w_ain, b_ain,
                   w_aout, b_aout, kpre, vpre, x_t);
}

/* FP8-W8A16 weights (the reference's pi0.5 numerics, hybrid_model.py:105-110): e4m3 codes in the
 * same natural layouts plus one fp32 scale per row, sq [NL][H*HD], sk / sv [NL][HD], so [NL][D],
 * sg / su [NL][F], sd [NL][D]. */
int fo_pi05_denoise_fp8(const fo_pi05_dims* dm, const uint8_t* qq, const float* sq, const uint8_t* qk,
                        const float* sk, const uint8_t* qv, const float* sv, const uint8_t* qo, const float* so,
                        const uint8_t* qg, const float* sg, const uint8_t* qu, const float* su, const uint8_t* qd,
                        const float* sd, const float* mods, const float* mod_final, const float* rope_cos,
                        const float* rope_sin, const float* w_ain, const float* b_ain, const float* w_aout,
                        const float* b_aout, const uint16_t* kpre, const uint16_t* vpre, float* x_t) {
  const fo_wmat W[7] = {{NULL, qq, sq}, {NULL, qk, sk}, {NULL, qv, sv}, {NULL, qo, so},
                        {NULL, qg, sg}, {NULL, qu, su}, {NULL, qd, sd}};
  return pi05_loop(dm, W[0], W[1], W[2], W[3], W[4], W[5], W[6], mods, mod_final, rope_cos, rope_sin, w_ain, b_ain,
                   w_aout, b_aout, kpre, vpre, x_t);
}

/* ------------------------------------------------------------------ */
/* MolmoAct2 flow loop (mk_ma2.cu:258-575)                             */
/* ------------------------------------------------------------------ */
typedef struct {
  int NL, D, H, HD, F, AD;
  int Lk, Tv, S, adim, batch;
} fo_ma2_dims;

static void rms_heads(float* v, int M, int H, int HD) {
  /* per-head RMS norm without weight, eps 1e-6 (mk_ma2.cu:300-315, 403-421) */
  for (int m = 0; m < M; m++)
    for (int hh = 0; hh < H; hh++) {
      float* p = v + (size_t)m * H * HD + (size_t)hh * HD;
      float r = 1.0f / sqrtf(dot_f32(p, p, HD) / (float)HD + 1e-6f);
      for (int d = 0; d < HD; d++) p[d] *= r;
    }
}

/* softmax(q k^T * scale) v over L keys for each (token, head); K,V [L][H*HD] */
static void mha(const float* q, int M, int H, int HD, const float* K, const float* V, int L, float scale, float* out) {
  const int QD = H * HD;
#pragma omp parallel
  {
    float* p = (float*)malloc(sizeof(float) * (size_t)L);
#pragma omp for schedule(static)
    for (int th = 0; th < M * H; th++) {
      int t = th / H, hh = th % H;
      const float* qv = q + (size_t)t * QD + (size_t)hh * HD;
      float mx = -INFINITY;
      for (int j = 0; j < L; j++) {
        p[j] = dot_f32(qv, K + (size_t)j * QD + (size_t)hh * HD, HD) * scale;
        if (p[j] > mx) mx = p[j];
      }
      float sum = 0.f;
      for (int j = 0; j < L; j++) { p[j] = expf(p[j] - mx); sum += p[j]; }
      float inv = 1.0f / sum;
      float* o = out + (size_t)t * QD + (size_t)hh * HD;
      for (int d = 0; d < HD; d++) o[d] = 0.f;
      for (int j = 0; j < L; j++) {
        float w = p[j] * inv;
        const float* vr = V + (size_t)j * QD + (size_t)hh * HD;
        for (int d = 0; d < HD; d++) o[d] += w * vr[d];
      }
    }
    free(p);
  }
}

/* Weights (bf16 bits, natural layouts, fp32 biases):
 *   w_qkv [NL][3D][D] + b_qkv [NL][3D] (rows q | k | v), w_so [NL][D][D] + b_so,
 *   w_cq + b_cq, w_co + b_co, w_g/w_u [NL][F][D] + b_g/b_u [NL][F], w_dn [NL][D][F] + b_dn
 * mods [S][NL][3][3][D] ({msa,mca,mlp} x {scale,shift,gate}), mod_final [S][2][D] (scale, shift)
 * rope_cos/sin [Tv][HD/2] (positions 0..Tv-1, split-half pairs d, d+HD/2)
 * w_ain [D][AD] fp32 + b_ain, w_aout [AD][D] bf16 + b_aout fp32
 * kctx, vctx [batch][NL][Lk][D] bf16 (projected, normed cross K; cross V)
 * x_t [batch][Tv][AD] fp32 in/out; only dims < adim are updated. */
int fo_ma2_flow(const fo_ma2_dims* dm, const uint16_t* w_qkv, const float* b_qkv, const uint16_t* w_so,
                const float* b_so, const uint16_t* w_cq, const float* b_cq, const uint16_t* w_co, const float* b_co,
                const uint16_t* w_g, const float* b_g, const uint16_t* w_u, const float* b_u, const uint16_t* w_dn,
                const float* b_dn, const float* mods, const float* mod_final, const float* rope_cos,
                const float* rope_sin, const float* w_ain, const float* b_ain, const uint16_t* w_aout,
                const float* b_aout, const uint16_t* kctx, const uint16_t* vctx, float* x_t) {
  const int NL = dm->NL, D = dm->D, H = dm->H, HD = dm->HD, F = dm->F, AD = dm->AD;
  const int Lk = dm->Lk, Tv = dm->Tv, S = dm->S, adim = dm->adim, B = dm->batch;
  const int half = HD / 2;
  if (NL < 1 || D < 1 || H < 1 || HD < 2 || (HD & 1) || H * HD != D || F < 1 || AD < 1 || Lk < 1 || Tv < 1 ||
      S < 1 || adim < 0 || adim > AD || B < 1)
    return -1;
  const float dt = 1.0f / (float)S;
  const float scale = 1.0f / sqrtf((float)HD);

  float* x = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* h = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* qkv = (float*)malloc(sizeof(float) * (size_t)Tv * 3 * D);
  float* q = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* k = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* v = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* att = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* o = (float*)malloc(sizeof(float) * (size_t)Tv * D);
  float* gg = (float*)malloc(sizeof(float) * (size_t)Tv * F);
  float* uu = (float*)malloc(sizeof(float) * (size_t)Tv * F);
  float* Kc = (float*)malloc(sizeof(float) * (size_t)Lk * D);
  float* Vc = (float*)malloc(sizeof(float) * (size_t)Lk * D);
  float* wa = (float*)malloc(sizeof(float) * (size_t)AD * D);
  float* act = (float*)malloc(sizeof(float) * (size_t)Tv * AD);
  for (size_t i = 0; i < (size_t)AD * D; i++) wa[i] = bf(w_aout[i]);

  for (int b = 0; b < B; b++) {
    float* xt = x_t + (size_t)b * Tv * AD;
    for (int s = 0; s < S; s++) {
      linear_f32(xt, Tv, AD, w_ain, b_ain, D, x); /* mk_ma2.cu:259-268 */
      for (int l = 0; l < NL; l++) {
        const float* ml = mods + ((size_t)s * NL + l) * 9 * D;
        const float *sc_msa = ml, *sh_msa = ml + D, *g_msa = ml + 2 * D;
        const float *sc_mca = ml + 3 * D, *sh_mca = ml + 4 * D, *g_mca = ml + 5 * D;
        const float *sc_mlp = ml + 6 * D, *sh_mlp = ml + 7 * D, *g_mlp = ml + 8 * D;
        /* self attention */
        ada_rms(x, Tv, D, sc_msa, sh_msa, h);
        linear_bf16(h, Tv, D, w_qkv + (size_t)l * 3 * D * D, b_qkv + (size_t)l * 3 * D, 3 * D, qkv);
        for (int t = 0; t < Tv; t++) {
          memcpy(q + (size_t)t * D, qkv + (size_t)t * 3 * D, sizeof(float) * D);
          memcpy(k + (size_t)t * D, qkv + (size_t)t * 3 * D + D, sizeof(float) * D);
          memcpy(v + (size_t)t * D, qkv + (size_t)t * 3 * D + 2 * D, sizeof(float) * D);
        }
        rms_heads(q, Tv, H, HD);
        rms_heads(k, Tv, H, HD);
        for (int t = 0; t < Tv; t++) {
          const float* c = rope_cos + (size_t)t * half;
          const float* sn = rope_sin + (size_t)t * half;
          for (int hh = 0; hh < H; hh++)
            for (int which = 0; which < 2; which++) {
              float* vec = (which == 0 ? q : k) + (size_t)t * D + (size_t)hh * HD;
              for (int j = 0; j < half; j++) {
                float a0 = vec[j], a1 = vec[j + half];
                vec[j] = a0 * c[j] - a1 * sn[j];
                vec[j + half] = a0 * sn[j] + a1 * c[j];
              }
            }
        }
        mha(q, Tv, H, HD, k, v, Tv, scale, att);
        linear_bf16(att, Tv, D, w_so + (size_t)l * D * D, b_so + (size_t)l * D, D, o);
        for (size_t i = 0; i < (size_t)Tv * D; i++) x[i] += g_msa[i % D] * o[i];
        /* cross attention */
        ada_rms(x, Tv, D, sc_mca, sh_mca, h);
        linear_bf16(h, Tv, D, w_cq + (size_t)l * D * D, b_cq + (size_t)l * D, D, q);
        rms_heads(q, Tv, H, HD);
        const uint16_t* kc = kctx + (((size_t)b * NL + l) * Lk) * D;
        const uint16_t* vc = vctx + (((size_t)b * NL + l) * Lk) * D;
        for (size_t i = 0; i < (size_t)Lk * D; i++) { Kc[i] = bf(kc[i]); Vc[i] = bf(vc[i]); }
        mha(q, Tv, H, HD, Kc, Vc, Lk, scale, att);
        linear_bf16(att, Tv, D, w_co + (size_t)l * D * D, b_co + (size_t)l * D, D, o);
        for (size_t i = 0; i < (size_t)Tv * D; i++) x[i] += g_mca[i % D] * o[i];
        /* MLP */
        ada_rms(x, Tv, D, sc_mlp, sh_mlp, h);
        linear_bf16(h, Tv, D, w_g + (size_t)l * F * D, b_g + (size_t)l * F, F, gg);
        linear_bf16(h, Tv, D, w_u + (size_t)l * F * D, b_u + (size_t)l * F, F, uu);
        for (size_t i = 0; i < (size_t)Tv * F; i++) gg[i] = silu_f(gg[i]) * uu[i];
        linear_bf16(gg, Tv, F, w_dn + (size_t)l * D * F, b_dn + (size_t)l * D, D, o);
        for (size_t i = 0; i < (size_t)Tv * D; i++) x[i] += g_mlp[i % D] * o[i];
      }
      const float* mf = mod_final + (size_t)s * 2 * D;
      ada_rms(x, Tv, D, mf, mf + D, h);
      linear_f32(h, Tv, D, wa, b_aout, AD, act);
      for (int t = 0; t < Tv; t++)
        for (int a = 0; a < adim; a++) xt[(size_t)t * AD + a] += dt * act[(size_t)t * AD + a];
    }
  }
  free(x); free(h); free(qkv); free(q); free(k); free(v); free(att); free(o); free(gg); free(uu);
  free(Kc); free(Vc); free(wa); free(act);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Gemma backbone prefix prefill (the benchmark's prefill workload)   */
/* ------------------------------------------------------------------ */
typedef struct {
  int NL, D, H, HD, F, Lp, batch;
} fo_prefill_dims;

/* The prefix prefill the reference runs through openpi's PaliGemma forward with use_cache
 * (benchmarks/pi05/eval_numerics.py:50-57), restated from the Gemma decoder layer:
 *   h = x rsqrt(mean(x^2) + 1e-6) (1 + w_in); q = h Wq^T, k = h Wk^T, v = h Wv^T
 *   RoPE on q and k at positions 0..Lp-1 (pairs j, j + HD/2, base 10000)
 *   attn = softmax(q k^T / sqrt(HD)) v, every prefix token against every prefix token (the
 *          prefix attends to itself without a mask), H query heads sharing the K/V head
 *   x += attn Wo^T; h = rms(x) (1 + w_post); x += (gelu_tanh(h Wg^T) (h Wu^T)) Wd^T
 * Output: the RoPE'd K and the V of every layer, kout/vout [batch][NL][Lp][HD] fp32 (the rows
 * compact_kv keeps, src/pi05/pack_weights.py:60-70). The last layer stops after its K/V.
 * Weights: bf16 bits, natural layouts wq [NL][H*HD][D], wk/wv [NL][HD][D], wo [NL][D][H*HD],
 * wg/wu [NL][F][D], wd [NL][D][F]; ln_in/ln_post [NL][D] fp32; rope_cos/sin [Lp][HD/2];
 * x_in [batch][Lp][D] fp32, the hidden states entering layer 0. */
int fo_gemma_prefill(const fo_prefill_dims* dm, const uint16_t* wq, const uint16_t* wk, const uint16_t* wv,
                     const uint16_t* wo, const uint16_t* wg, const uint16_t* wu, const uint16_t* wd,
                     const float* ln_in, const float* ln_post, const float* rope_cos, const float* rope_sin,
                     const float* x_in, float* kout, float* vout) {
  const int NL = dm->NL, D = dm->D, H = dm->H, HD = dm->HD, F = dm->F, Lp = dm->Lp, B = dm->batch;
  if (NL < 1 || D < 1 || H < 1 || HD < 2 || (HD & 1) || F < 1 || Lp < 1 || B < 1) return -1;
  const int QD = H * HD, half = HD / 2;
  const float scale = 1.0f / sqrtf((float)HD);
  float* x = (float*)malloc(sizeof(float) * (size_t)Lp * D);
  float* h = (float*)malloc(sizeof(float) * (size_t)Lp * D);
  float* q = (float*)malloc(sizeof(float) * (size_t)Lp * QD);
  float* k = (float*)malloc(sizeof(float) * (size_t)Lp * HD);
  float* v = (float*)malloc(sizeof(float) * (size_t)Lp * HD);
  float* att = (float*)malloc(sizeof(float) * (size_t)Lp * QD);
  float* o = (float*)malloc(sizeof(float) * (size_t)Lp * D);
  float* g = (float*)malloc(sizeof(float) * (size_t)Lp * F);
  float* u = (float*)malloc(sizeof(float) * (size_t)Lp * F);
  float* zero = (float*)calloc((size_t)D, sizeof(float));
  for (int b = 0; b < B; b++) {
    memcpy(x, x_in + (size_t)b * Lp * D, sizeof(float) * (size_t)Lp * D);
    for (int l = 0; l < NL; l++) {
      ada_rms(x, Lp, D, ln_in + (size_t)l * D, zero, h);
      linear_bf16(h, Lp, D, wq + (size_t)l * QD * D, NULL, QD, q);
      linear_bf16(h, Lp, D, wk + (size_t)l * HD * D, NULL, HD, k);
      linear_bf16(h, Lp, D, wv + (size_t)l * HD * D, NULL, HD, v);
      for (int t = 0; t < Lp; t++) {
        const float* c = rope_cos + (size_t)t * half;
        const float* sn = rope_sin + (size_t)t * half;
        for (int hh = 0; hh <= H; hh++) {
          float* vec = hh < H ? q + (size_t)t * QD + (size_t)hh * HD : k + (size_t)t * HD;
          for (int j = 0; j < half; j++) {
            float a0 = vec[j], a1 = vec[j + half];
            vec[j] = a0 * c[j] - a1 * sn[j];
            vec[j + half] = a1 * c[j] + a0 * sn[j];
          }
        }
      }
      float* ko = kout + ((size_t)b * NL + l) * Lp * HD;
      float* vo = vout + ((size_t)b * NL + l) * Lp * HD;
      memcpy(ko, k, sizeof(float) * (size_t)Lp * HD);
      memcpy(vo, v, sizeof(float) * (size_t)Lp * HD);
      if (l == NL - 1) break;
#pragma omp parallel
      {
        float* p = (float*)malloc(sizeof(float) * (size_t)Lp);
#pragma omp for schedule(static)
        for (int th = 0; th < Lp * H; th++) {
          int t = th / H, hh = th % H;
          const float* qv = q + (size_t)t * QD + (size_t)hh * HD;
          float mx = -INFINITY;
          for (int j = 0; j < Lp; j++) {
            p[j] = dot_f32(qv, k + (size_t)j * HD, HD) * scale;
            if (p[j] > mx) mx = p[j];
          }
          float sum = 0.f;
          for (int j = 0; j < Lp; j++) { p[j] = expf(p[j] - mx); sum += p[j]; }
          float inv = 1.0f / sum;
          float* out = att + (size_t)t * QD + (size_t)hh * HD;
          for (int d = 0; d < HD; d++) out[d] = 0.f;
          for (int j = 0; j < Lp; j++) {
            float w = p[j] * inv;
            const float* vr = v + (size_t)j * HD;
            for (int d = 0; d < HD; d++) out[d] += w * vr[d];
          }
        }
        free(p);
      }
      linear_bf16(att, Lp, QD, wo + (size_t)l * D * QD, NULL, D, o);
      for (size_t i = 0; i < (size_t)Lp * D; i++) x[i] += o[i];
      ada_rms(x, Lp, D, ln_post + (size_t)l * D, zero, h);
      linear_bf16(h, Lp, D, wg + (size_t)l * F * D, NULL, F, g);
      linear_bf16(h, Lp, D, wu + (size_t)l * F * D, NULL, F, u);
      for (size_t i = 0; i < (size_t)Lp * F; i++) g[i] = gelu_tanh_f(g[i]) * u[i];
      linear_bf16(g, Lp, F, wd + (size_t)l * D * F, NULL, D, o);
      for (size_t i = 0; i < (size_t)Lp * D; i++) x[i] += o[i];
    }
  }
  free(x); free(h); free(q); free(k); free(v); free(att); free(o); free(g); free(u); free(zero);
  return 0;
}
