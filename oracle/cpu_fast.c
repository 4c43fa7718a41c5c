/*
 * CPU baseline: a C restatement of the reference's FP32 CPU convolution
 * algorithms, timed by bench.py beside the GPU numbers.  Test
 * infrastructure like the rest of oracle/: nothing in the shipped library
 * links or calls it.  tests/test_cpu_fast.py checks it against the oracle's
 * double-accumulating convolution and forward.
 *
 * Routing per convolution restates TensorOps.Conv for the CPU backend
 * (src/SimdYolo/Compute.cs:185-233):
 *   - 3x3 s1 p1 d1 g1 with ic >= 8, oc >= 8 and oh*ow >= 64: Winograd,
 *     F(4x4,3x3) when (32 <= ic <= 64, 32 <= oc <= 128, oh, ow <= 160) or the
 *     shape is one of CpuWinograd4.AdditionalHotShape's
 *     (src/SimdYolo/CpuWinograd4.cs:28-32, default SIMDYOLO_CPU_F4_EXPAND=2),
 *     otherwise F(2x2,3x3) (src/SimdYolo/CpuWinograd.cs:20-60);
 *   - depthwise (groups == ic == oc): direct per channel
 *     (src/SimdYolo/CpuSpatial.cs:79-128);
 *   - everything else, 1x1 included: the implicit GEMM of
 *     CpuConvolution.Conv (src/SimdYolo/CpuConvolution.cs:29-57), im2col
 *     panels of 16 output pixels multiplied by pre-packed weights.
 * Winograd transforms: the reference's matrices and formulas
 * (CpuWinograd4.cs:36,51-64,186-204 for F(4,3); CpuWinograd.cs:27-46,100-113
 * for F(2,3)); weight transforms are computed once per convolution, as the
 * reference caches them per constant weight tensor (CpuWinograd4.cs:65).
 * Plane products and the implicit GEMM share one packed SGEMM
 * (CpuGemm.MultiplyBatch, src/SimdYolo/CpuGemm.cs:40): weights in panels of 6
 * rows, activations in panels of 16 columns, a 6x16 AVX2/FMA register tile,
 * OpenMP over panels (and planes).  Bias and SiLU are applied while a panel
 * is in cache; SiLU uses the reference's FastExp
 * (src/SimdYolo/CpuActivation.cs:87-119: 6th-order Taylor on [-ln2/2, ln2/2]
 * with a split ln 2, expf beyond |x| > 87).  AVX-512 stays off, as in the
 * reference's default (src/SimdYolo/CpuGemm512.cs:9).
 */
#include "cpu_fast.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

enum { MR = 6, NR = 16 };

static void* amalloc(size_t bytes) {
  void* p = NULL;
  if (posix_memalign(&p, 64, bytes ? bytes : 64)) return NULL;
  return p;
}

/* ------------------------------------------------------------ SiLU */

/* CpuActivation.FastExp (CpuActivation.cs:96-119) on eight lanes. */
static inline __m256 fast_exp8(__m256 x) {
  const __m256 mag = _mm256_and_ps(x, _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff)));
  if (_mm256_movemask_ps(_mm256_cmp_ps(mag, _mm256_set1_ps(87.f), _CMP_LE_OQ)) != 255) {
    float v[8];
    _mm256_storeu_ps(v, x);
    for (int i = 0; i < 8; ++i) v[i] = expf(v[i]);
    return _mm256_loadu_ps(v);
  }
  const __m256 ne = _mm256_sub_ps(_mm256_setzero_ps(),
                                  _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.4426950408889634f)),
                                                  _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
  __m256 r = _mm256_fmadd_ps(ne, _mm256_set1_ps(0.693145751953125f), x);
  r = _mm256_fmadd_ps(ne, _mm256_set1_ps(1.428606765330187e-6f), r);
  __m256 p = _mm256_set1_ps(1.f / 720.f);
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.f / 120.f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.f / 24.f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.f / 6.f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(.5f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.f));
  const __m256i e = _mm256_cvtps_epi32(_mm256_sub_ps(_mm256_setzero_ps(), ne));
  const __m256i pw = _mm256_slli_epi32(_mm256_add_epi32(e, _mm256_set1_epi32(127)), 23);
  return _mm256_mul_ps(p, _mm256_castsi256_ps(pw));
}

/* v / (1 + FastExp(-v)): CpuActivation.FastSilu (CpuActivation.cs:87-90). */
static inline __m256 fast_silu8(__m256 v) {
  return _mm256_div_ps(v, _mm256_add_ps(_mm256_set1_ps(1.f), fast_exp8(_mm256_sub_ps(_mm256_setzero_ps(), v))));
}

/* Scalar tails use the library exponent (Compute.cs:513). */
static inline float silu1(float v) { return v / (1.f + expf(-v)); }

/* y[0..n) = act(y + b) */
static void bias_act(float* y, int n, float b, int silu) {
  int i = 0;
  const __m256 vb = _mm256_set1_ps(b);
  for (; i + 8 <= n; i += 8) {
    __m256 v = _mm256_add_ps(_mm256_loadu_ps(y + i), vb);
    if (silu) v = fast_silu8(v);
    _mm256_storeu_ps(y + i, v);
  }
  for (; i < n; ++i) {
    const float v = y[i] + b;
    y[i] = silu ? silu1(v) : v;
  }
}

/* ------------------------------------------------------------ packed SGEMM */

/* A [M][K] (row stride lda) into panels of MR rows: p[(m / MR)][k][MR], rows
 * past M zero. */
static float* pack_a(const float* a, int M, int K, size_t lda) {
  const int mp = (M + MR - 1) / MR;
  float* p = (float*)amalloc(sizeof(float) * (size_t)mp * K * MR);
  for (int i = 0; i < mp; ++i)
    for (int k = 0; k < K; ++k)
      for (int r = 0; r < MR; ++r) {
        const int m = i * MR + r;
        p[((size_t)i * K + k) * MR + r] = m < M ? a[(size_t)m * lda + k] : 0.f;
      }
  return p;
}

/* c[r][0..nr) (row stride ldc) = sum_k ap[k][r] * bp[k][0..16) for the 6 x 16
 * register tile; rows >= mr are not stored. */
static void kernel_6x16(int K, const float* ap, const float* bp, float* c, size_t ldc, int mr, int nr) {
  __m256 c00 = _mm256_setzero_ps(), c01 = _mm256_setzero_ps(), c10 = _mm256_setzero_ps(), c11 = _mm256_setzero_ps();
  __m256 c20 = _mm256_setzero_ps(), c21 = _mm256_setzero_ps(), c30 = _mm256_setzero_ps(), c31 = _mm256_setzero_ps();
  __m256 c40 = _mm256_setzero_ps(), c41 = _mm256_setzero_ps(), c50 = _mm256_setzero_ps(), c51 = _mm256_setzero_ps();
  for (int k = 0; k < K; ++k) {
    const __m256 b0 = _mm256_load_ps(bp + NR * k), b1 = _mm256_load_ps(bp + NR * k + 8);
    const float* a = ap + MR * k;
    __m256 t = _mm256_broadcast_ss(a + 0);
    c00 = _mm256_fmadd_ps(t, b0, c00); c01 = _mm256_fmadd_ps(t, b1, c01);
    t = _mm256_broadcast_ss(a + 1);
    c10 = _mm256_fmadd_ps(t, b0, c10); c11 = _mm256_fmadd_ps(t, b1, c11);
    t = _mm256_broadcast_ss(a + 2);
    c20 = _mm256_fmadd_ps(t, b0, c20); c21 = _mm256_fmadd_ps(t, b1, c21);
    t = _mm256_broadcast_ss(a + 3);
    c30 = _mm256_fmadd_ps(t, b0, c30); c31 = _mm256_fmadd_ps(t, b1, c31);
    t = _mm256_broadcast_ss(a + 4);
    c40 = _mm256_fmadd_ps(t, b0, c40); c41 = _mm256_fmadd_ps(t, b1, c41);
    t = _mm256_broadcast_ss(a + 5);
    c50 = _mm256_fmadd_ps(t, b0, c50); c51 = _mm256_fmadd_ps(t, b1, c51);
  }
  if (mr == MR && nr == NR) {
    _mm256_storeu_ps(c, c00); _mm256_storeu_ps(c + 8, c01);
    _mm256_storeu_ps(c + ldc, c10); _mm256_storeu_ps(c + ldc + 8, c11);
    _mm256_storeu_ps(c + 2 * ldc, c20); _mm256_storeu_ps(c + 2 * ldc + 8, c21);
    _mm256_storeu_ps(c + 3 * ldc, c30); _mm256_storeu_ps(c + 3 * ldc + 8, c31);
    _mm256_storeu_ps(c + 4 * ldc, c40); _mm256_storeu_ps(c + 4 * ldc + 8, c41);
    _mm256_storeu_ps(c + 5 * ldc, c50); _mm256_storeu_ps(c + 5 * ldc + 8, c51);
    return;
  }
  float tile[MR][NR] __attribute__((aligned(32)));
  _mm256_store_ps(tile[0], c00); _mm256_store_ps(tile[0] + 8, c01);
  _mm256_store_ps(tile[1], c10); _mm256_store_ps(tile[1] + 8, c11);
  _mm256_store_ps(tile[2], c20); _mm256_store_ps(tile[2] + 8, c21);
  _mm256_store_ps(tile[3], c30); _mm256_store_ps(tile[3] + 8, c31);
  _mm256_store_ps(tile[4], c40); _mm256_store_ps(tile[4] + 8, c41);
  _mm256_store_ps(tile[5], c50); _mm256_store_ps(tile[5] + 8, c51);
  for (int r = 0; r < mr; ++r) memcpy(c + r * ldc, tile[r], sizeof(float) * nr);
}

/* C[0..M)[0..nr) (row stride ldc) = packed A x one K x 16 B panel. */
static void gemm_panel(const float* ap, int M, int K, const float* bp, float* c, size_t ldc, int nr) {
  for (int i = 0; i * MR < M; ++i) {
    const int mr = M - i * MR < MR ? M - i * MR : MR;
    kernel_6x16(K, ap + (size_t)i * K * MR, bp, c + (size_t)i * MR * ldc, ldc, mr, nr);
  }
}

/* ------------------------------------------------------------ convolutions */

struct cf_conv {
  int ic, oc, k, s, groups, silu;
  float* bias;        /* oc */
  float* a;           /* implicit GEMM: packed [oc][ic*k*k] */
  float* u4[36];      /* F(4,3): packed U[p] [oc][ic] */
  float* u2[16];      /* F(2,3): packed U[p] [oc][ic] */
  float* dw;          /* depthwise: [oc][k*k] */
  float* scratch;     /* Winograd V and M */
  size_t scratch_len; /* floats */
};

/* Compute.cs:185-188 and CpuWinograd4.AdditionalHotShape (CpuWinograd4.cs:28-32). */
static int f4_shape(int ic, int oc, int oh, int ow) {
  if (ic >= 32 && ic <= 64 && oc >= 32 && oc <= 128 && oh <= 160 && ow <= 160) return 1;
  if (ic == 80 && oc == 80 && oh == 80 && ow == 80) return 1;
  return ic >= 32 && ic <= 256 && oc >= 32 && oc <= 256 && ic + oc <= 512 && (ic >= 80 || oc > 128) && oh >= 20 &&
         oh <= 160 && ow >= 20 && ow <= 160;
}

static int wino_eligible(const cf_conv* c) { return c->groups == 1 && c->k == 3 && c->s == 1 && c->ic >= 8 && c->oc >= 8; }

/* U = G g G^T with the reference's F(4,3) G, float arithmetic in its order
 * (CpuWinograd4.cs:36,51-64). */
static void f4_weights(const float* w, int oc, int ic, float* u /* [36][oc][ic] */) {
  static const float G[18] = {.25f, 0, 0, -1.f / 6, -1.f / 6, -1.f / 6, -1.f / 6, 1.f / 6, -1.f / 6,
                              1.f / 24, 1.f / 12, 1.f / 6, 1.f / 24, -1.f / 12, 1.f / 6, 0, 0, 1};
  for (int co = 0; co < oc; ++co)
    for (int ci = 0; ci < ic; ++ci) {
      const float* d = w + ((size_t)co * ic + ci) * 9;
      float t[18];
      for (int r = 0; r < 6; ++r)
        for (int c = 0; c < 3; ++c) t[r * 3 + c] = G[r * 3] * d[c] + G[r * 3 + 1] * d[3 + c] + G[r * 3 + 2] * d[6 + c];
      for (int r = 0; r < 6; ++r)
        for (int c = 0; c < 6; ++c)
          u[((size_t)(r * 6 + c) * oc + co) * ic + ci] =
              t[r * 3] * G[c * 3] + t[r * 3 + 1] * G[c * 3 + 1] + t[r * 3 + 2] * G[c * 3 + 2];
    }
}

/* F(2,3) weight transform (CpuWinograd.cs:27-46). */
static void f2_weights(const float* w, int oc, int ic, float* u /* [16][oc][ic] */) {
  const size_t plane = (size_t)oc * ic;
  for (int co = 0; co < oc; ++co)
    for (int ci = 0; ci < ic; ++ci) {
      const float* g = w + ((size_t)co * ic + ci) * 9;
      float t[12];
      for (int c = 0; c < 3; ++c) {
        const float a = g[c], b = g[3 + c], d = g[6 + c];
        t[c] = a;
        t[3 + c] = (a + b + d) * .5f;
        t[6 + c] = (a - b + d) * .5f;
        t[9 + c] = d;
      }
      const size_t i = (size_t)co * ic + ci;
      for (int r = 0; r < 4; ++r) {
        const float a = t[r * 3], b = t[r * 3 + 1], c = t[r * 3 + 2];
        u[(r * 4) * plane + i] = a;
        u[(r * 4 + 1) * plane + i] = (a + b + c) * .5f;
        u[(r * 4 + 2) * plane + i] = (a - b + c) * .5f;
        u[(r * 4 + 3) * plane + i] = c;
      }
    }
}

cf_conv* cf_conv_create(const float* w, const float* bias, int oc, int ic, int k, int s, int groups, int silu) {
  cf_conv* c = (cf_conv*)calloc(1, sizeof(cf_conv));
  if (!c) return NULL;
  c->ic = ic; c->oc = oc; c->k = k; c->s = s; c->groups = groups; c->silu = silu;
  c->bias = (float*)amalloc(sizeof(float) * oc);
  for (int o = 0; o < oc; ++o) c->bias[o] = bias ? bias[o] : 0.f;
  if (groups > 1) {
    c->dw = (float*)amalloc(sizeof(float) * (size_t)oc * k * k);
    memcpy(c->dw, w, sizeof(float) * (size_t)oc * k * k);
    return c;
  }
  c->a = pack_a(w, oc, ic * k * k, (size_t)ic * k * k);
  if (wino_eligible(c)) {
    float* u = (float*)amalloc(sizeof(float) * 36 * (size_t)oc * ic);
    f4_weights(w, oc, ic, u);
    for (int p = 0; p < 36; ++p) c->u4[p] = pack_a(u + (size_t)p * oc * ic, oc, ic, ic);
    f2_weights(w, oc, ic, u);
    for (int p = 0; p < 16; ++p) c->u2[p] = pack_a(u + (size_t)p * oc * ic, oc, ic, ic);
    free(u);
  }
  return c;
}

void cf_conv_destroy(cf_conv* c) {
  if (!c) return;
  free(c->bias);
  free(c->a);
  free(c->dw);
  for (int p = 0; p < 36; ++p) free(c->u4[p]);
  for (int p = 0; p < 16; ++p) free(c->u2[p]);
  free(c->scratch);
  free(c);
}

static float* scratch(cf_conv* c, size_t floats) {
  if (floats > c->scratch_len) {
    free(c->scratch);
    c->scratch = (float*)amalloc(sizeof(float) * floats);
    c->scratch_len = c->scratch ? floats : 0;
  }
  return c->scratch;
}

/* F(4,3) input transform rows (CpuWinograd4.Transform, CpuWinograd4.cs:186-194). */
static inline void f4_in(const float* d, int st, float* o, int os) {
  o[0] = 4 * d[0] - 5 * d[2 * st] + d[4 * st];
  o[os] = -4 * (d[st] + d[2 * st]) + d[3 * st] + d[4 * st];
  o[2 * os] = 4 * (d[st] - d[2 * st]) - d[3 * st] + d[4 * st];
  o[3 * os] = -2 * d[st] - d[2 * st] + 2 * d[3 * st] + d[4 * st];
  o[4 * os] = 2 * d[st] - d[2 * st] - 2 * d[3 * st] + d[4 * st];
  o[5 * os] = 4 * d[st] - 5 * d[3 * st] + d[5 * st];
}

/* F(4,3) inverse rows (CpuWinograd4.Inverse, CpuWinograd4.cs:196-203). */
static inline void f4_out(const float* d, int st, float* o, int os) {
  o[0] = d[0] + d[st] + d[2 * st] + d[3 * st] + d[4 * st];
  o[os] = d[st] - d[2 * st] + 2 * (d[3 * st] - d[4 * st]);
  o[2 * os] = d[st] + d[2 * st] + 4 * (d[3 * st] + d[4 * st]);
  o[3 * os] = d[st] - d[2 * st] + 8 * (d[3 * st] - d[4 * st]) + d[5 * st];
}

/* One image of a Winograd conv: V [P][panels][ic][16] -> M [P][oc][panels*16]
 * -> y.  m = 4 (F(4,3), 6x6 patches) or 2 (F(2,3), 4x4 patches). */
static void winograd(cf_conv* c, int m, const float* x, int h, int w, float* y) {
  const int ic = c->ic, oc = c->oc, a = m + 2, P = a * a;
  const int th = (h + m - 1) / m, tw = (w + m - 1) / m, tiles = th * tw;
  const int panels = (tiles + NR - 1) / NR, tp = panels * NR;
  float* V = scratch(c, (size_t)P * tp * ic + (size_t)P * oc * tp);
  float* M = V + (size_t)P * tp * ic;
  float* const* U = m == 4 ? c->u4 : c->u2;
#pragma omp parallel for schedule(static)
  for (int ci = 0; ci < ic; ++ci) {
    const float* src = x + (size_t)ci * h * w;
    for (int t = 0; t < tp; ++t) {
      float v[36];
      if (t < tiles) {
        const int ty = t / tw, tx = t - ty * tw;
        float d[36], tmp[36];
        for (int r = 0; r < a; ++r)
          for (int q = 0; q < a; ++q) {
            const int yy = ty * m - 1 + r, xx = tx * m - 1 + q;
            d[r * a + q] = (unsigned)yy < (unsigned)h && (unsigned)xx < (unsigned)w ? src[(size_t)yy * w + xx] : 0.f;
          }
        if (m == 4) {
          for (int q = 0; q < 6; ++q) f4_in(d + q, 6, tmp + q, 6);  /* columns */
          for (int r = 0; r < 6; ++r) f4_in(tmp + r * 6, 1, v + r * 6, 1);
        } else {
          /* B^T d B with B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1] (CpuWinograd.cs:136-170). */
          for (int q = 0; q < 4; ++q) {
            tmp[q] = d[q] - d[8 + q];
            tmp[4 + q] = d[4 + q] + d[8 + q];
            tmp[8 + q] = d[8 + q] - d[4 + q];
            tmp[12 + q] = d[4 + q] - d[12 + q];
          }
          for (int r = 0; r < 4; ++r) {
            const float* s = tmp + 4 * r;
            v[4 * r] = s[0] - s[2];
            v[4 * r + 1] = s[1] + s[2];
            v[4 * r + 2] = s[2] - s[1];
            v[4 * r + 3] = s[1] - s[3];
          }
        }
      } else {
        memset(v, 0, sizeof v);
      }
      const int pn = t / NR, j = t - pn * NR;
      for (int p = 0; p < P; ++p) V[(((size_t)p * panels + pn) * ic + ci) * NR + j] = v[p];
    }
  }
#pragma omp parallel for collapse(2) schedule(static)
  for (int p = 0; p < P; ++p)
    for (int pn = 0; pn < panels; ++pn)
      gemm_panel(U[p], oc, ic, V + ((size_t)p * panels + pn) * ic * NR, M + (size_t)p * oc * tp + (size_t)pn * NR, tp,
                 NR);
#pragma omp parallel for schedule(static)
  for (int co = 0; co < oc; ++co) {
    float* dst = y + (size_t)co * h * w;
    const float b = c->bias[co];
    for (int t = 0; t < tiles; ++t) {
      const int ty = t / tw, tx = t - ty * tw;
      float mm[36], tmp[24], o[16];
      for (int p = 0; p < P; ++p) mm[p] = M[((size_t)p * oc + co) * tp + t];
      if (m == 4) {
        for (int q = 0; q < 6; ++q) f4_out(mm + q, 6, tmp + q, 6);
        for (int r = 0; r < 4; ++r) f4_out(tmp + r * 6, 1, o + r * 4, 1);
      } else {
        /* A^T = [1 1 1 0; 0 1 -1 -1] (CpuWinograd.cs:100-113). */
        const float t0[4] = {mm[0] + mm[4] + mm[8], mm[1] + mm[5] + mm[9], mm[2] + mm[6] + mm[10],
                             mm[3] + mm[7] + mm[11]};
        const float t1[4] = {mm[4] - mm[8] - mm[12], mm[5] - mm[9] - mm[13], mm[6] - mm[10] - mm[14],
                             mm[7] - mm[11] - mm[15]};
        o[0] = t0[0] + t0[1] + t0[2];
        o[1] = t0[1] - t0[2] - t0[3];
        o[2] = t1[0] + t1[1] + t1[2];
        o[3] = t1[1] - t1[2] - t1[3];
      }
      for (int r = 0; r < m && ty * m + r < h; ++r)
        for (int q = 0; q < m && tx * m + q < w; ++q) dst[(size_t)(ty * m + r) * w + tx * m + q] = o[r * m + q] + b;
    }
    bias_act(dst, h * w, 0.f, c->silu);
  }
}

/* Implicit GEMM (CpuConvolution.Conv): per panel of 16 output pixels, the
 * im2col columns (k ordered (c, ky, kx) as the OIHW weights), then packed
 * weights x panel, then bias and SiLU on the panel. */
static void implicit(cf_conv* c, const float* x, int h, int w, float* y, int oh, int ow) {
  const int ic = c->ic, oc = c->oc, k = c->k, s = c->s, pad = k / 2, K = ic * k * k;
  const int spatial = oh * ow, panels = (spatial + NR - 1) / NR;
#pragma omp parallel
  {
    float* bp = (float*)amalloc(sizeof(float) * (size_t)K * NR);
#pragma omp for schedule(static)
    for (int pn = 0; pn < panels; ++pn) {
      const int j0 = pn * NR, nr = spatial - j0 < NR ? spatial - j0 : NR;
      if (k == 1 && s == 1) {
        for (int ci = 0; ci < ic; ++ci) {
          const float* src = x + (size_t)ci * h * w + j0;
          float* d = bp + (size_t)ci * NR;
          for (int j = 0; j < NR; ++j) d[j] = j < nr ? src[j] : 0.f;
        }
      } else {
        int iy0[NR], ix0[NR];
        for (int j = 0; j < NR; ++j) {
          const int pix = j0 + (j < nr ? j : 0), oy = pix / ow, ox = pix - oy * ow;
          iy0[j] = j < nr ? oy * s - pad : -(1 << 20);  /* columns past the end read zero */
          ix0[j] = ox * s - pad;
        }
        for (int ci = 0; ci < ic; ++ci)
          for (int ky = 0; ky < k; ++ky)
            for (int kx = 0; kx < k; ++kx) {
              float* row = bp + (size_t)((ci * k + ky) * k + kx) * NR;
              const float* src = x + (size_t)ci * h * w;
              for (int j = 0; j < NR; ++j) {
                const int iy = iy0[j] + ky, ix = ix0[j] + kx;
                row[j] = (unsigned)iy < (unsigned)h && (unsigned)ix < (unsigned)w ? src[(size_t)iy * w + ix] : 0.f;
              }
            }
      }
      gemm_panel(c->a, oc, K, bp, y + j0, spatial, nr);
      for (int co = 0; co < oc; ++co) bias_act(y + (size_t)co * spatial + j0, nr, c->bias[co], c->silu);
    }
    free(bp);
  }
}

/* Depthwise direct (CpuSpatial.Depthwise semantics): per channel. */
static void depthwise(cf_conv* c, const float* x, int h, int w, float* y, int oh, int ow) {
  const int k = c->k, s = c->s, pad = k / 2;
#pragma omp parallel for schedule(static)
  for (int ch = 0; ch < c->oc; ++ch) {
    const float* src = x + (size_t)ch * h * w;
    const float* wt = c->dw + (size_t)ch * k * k;
    float* dst = y + (size_t)ch * oh * ow;
    for (int oy = 0; oy < oh; ++oy)
      for (int ox = 0; ox < ow; ++ox) {
        float v = 0.f;
        for (int ky = 0; ky < k; ++ky)
          for (int kx = 0; kx < k; ++kx) {
            const int iy = oy * s - pad + ky, ix = ox * s - pad + kx;
            if ((unsigned)iy < (unsigned)h && (unsigned)ix < (unsigned)w) v += src[(size_t)iy * w + ix] * wt[ky * k + kx];
          }
        dst[(size_t)oy * ow + ox] = v;
      }
    bias_act(dst, oh * ow, c->bias[ch], c->silu);
  }
}

int cf_conv_run(cf_conv* c, const float* x, int n, int h, int w, float* y, int* oh_out, int* ow_out) {
  if (!c || !x || n <= 0) return 1;
  const int pad = c->k / 2;
  const int oh = (h + 2 * pad - c->k) / c->s + 1, ow = (w + 2 * pad - c->k) / c->s + 1;
  if (oh_out) *oh_out = oh;
  if (ow_out) *ow_out = ow;
  if (!y) return 0;
  for (int b = 0; b < n; ++b) {
    const float* xb = x + (size_t)b * c->ic * h * w;
    float* yb = y + (size_t)b * c->oc * oh * ow;
    if (c->dw) depthwise(c, xb, h, w, yb, oh, ow);
    else if (wino_eligible(c) && oh * ow >= 64) winograd(c, f4_shape(c->ic, c->oc, oh, ow) ? 4 : 2, xb, h, w, yb);
    else implicit(c, xb, h, w, yb, oh, ow);
  }
  return 0;
}

int cf_conv_algorithm(const cf_conv* c, int h, int w) {
  const int pad = c->k / 2;
  const int oh = (h + 2 * pad - c->k) / c->s + 1, ow = (w + 2 * pad - c->k) / c->s + 1;
  if (c->dw) return CF_DEPTHWISE;
  if (wino_eligible(c) && oh * ow >= 64) return f4_shape(c->ic, c->oc, oh, ow) ? CF_WINOGRAD4 : CF_WINOGRAD2;
  return CF_IMPLICIT;
}

int cf_threads(void) { return omp_get_max_threads(); }

/* Detect-head decode of one level (CpuHead.DecodeInto, src/SimdYolo/CpuHead.cs:57-124,
 * with CpuDfl.Decode, src/SimdYolo/CpuDfl.cs:19-61): per side and block of 256
 * anchors the max-subtracted softmax expectation over the bins, eight anchors
 * per vector; class sigmoids per channel; then the grid decode.  OpenMP over
 * (image, side, block) and (image, class). */
void cf_detect_decode(const float* boxes, const float* scores, int batch, int nc, int h, int w, int bins, float stride,
                      int xyxy, float* out, int out_anchors, int start) {
  const int spatial = h * w, tile = 256, tiles = (spatial + tile - 1) / tile;
  float* dist = (float*)amalloc(sizeof(float) * (size_t)batch * 4 * spatial);
  const int blocks = batch * 4 * tiles;
#pragma omp parallel for schedule(static)
  for (int blk = 0; blk < blocks; ++blk) {
    const int bs = blk / tiles, a0 = (blk % tiles) * tile, a1 = a0 + tile < spatial ? a0 + tile : spatial;
    const float* src = boxes + (size_t)bs * bins * spatial;
    float* dst = dist + (size_t)bs * spatial;
    int a = a0;
    if (bins == 1) {
      memcpy(dst + a0, src + a0, sizeof(float) * (a1 - a0));
      continue;
    }
    for (; a + 8 <= a1; a += 8) {
      __m256 mx = _mm256_set1_ps(-INFINITY);
      for (int r = 0; r < bins; ++r) mx = _mm256_max_ps(mx, _mm256_loadu_ps(src + (size_t)r * spatial + a));
      __m256 sum = _mm256_setzero_ps(), num = _mm256_setzero_ps();
      for (int r = 0; r < bins; ++r) {
        const __m256 e = fast_exp8(_mm256_sub_ps(_mm256_loadu_ps(src + (size_t)r * spatial + a), mx));
        sum = _mm256_add_ps(sum, e);
        num = _mm256_add_ps(num, _mm256_mul_ps(e, _mm256_set1_ps((float)r)));
      }
      _mm256_storeu_ps(dst + a, _mm256_div_ps(num, sum));
    }
    for (; a < a1; ++a) {
      float mx = -INFINITY, sum = 0.f, num = 0.f;
      for (int r = 0; r < bins; ++r) mx = fmaxf(mx, src[(size_t)r * spatial + a]);
      for (int r = 0; r < bins; ++r) {
        const float e = expf(src[(size_t)r * spatial + a] - mx);
        sum += e;
        num += e * r;
      }
      dst[a] = num / sum;
    }
  }
#pragma omp parallel for schedule(static)
  for (int bc = 0; bc < batch * nc; ++bc) {
    const int b = bc / nc, c = bc - b * nc;
    const float* src = scores + (size_t)bc * spatial;
    float* dst = out + ((size_t)b * (nc + 4) + 4 + c) * out_anchors + start;
    int a = 0;
    for (; a + 8 <= spatial; a += 8) {
      const __m256 v = _mm256_loadu_ps(src + a);
      _mm256_storeu_ps(dst + a, _mm256_div_ps(_mm256_set1_ps(1.f),
                                               _mm256_add_ps(_mm256_set1_ps(1.f),
                                                             fast_exp8(_mm256_sub_ps(_mm256_setzero_ps(), v)))));
    }
    for (; a < spatial; ++a) dst[a] = 1.f / (1.f + expf(-src[a]));
  }
#pragma omp parallel for schedule(static)
  for (int br = 0; br < batch * h; ++br) {
    const int b = br / h, row = br - b * h;
    const float* d = dist + (size_t)b * 4 * spatial + (size_t)row * w;
    float* o = out + (size_t)b * (nc + 4) * out_anchors + start + (size_t)row * w;
    for (int col = 0; col < w; ++col) {
      const float cx = col + .5f, cy = row + .5f;
      const float x1 = (cx - d[col]) * stride, y1 = (cy - d[spatial + col]) * stride;
      const float x2 = (cx + d[2 * spatial + col]) * stride, y2 = (cy + d[3 * spatial + col]) * stride;
      o[col] = xyxy ? x1 : (x1 + x2) * .5f;
      o[out_anchors + col] = xyxy ? y1 : (y1 + y2) * .5f;
      o[2 * (size_t)out_anchors + col] = xyxy ? x2 : x2 - x1;
      o[3 * (size_t)out_anchors + col] = xyxy ? y2 : y2 - y1;
    }
  }
  free(dist);
}
