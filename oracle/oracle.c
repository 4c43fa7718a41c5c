/*
 * CPU restatement of SimdYolo's FP32 forward path.  TEST INFRASTRUCTURE ONLY:
 * the parity checker for the HIP backend and the CPU-baseline timing leg.
 * The shipped library never links or calls this file.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off).  Contraction
 * is off because the reference (C#/RyuJIT) never fuses a*b+c into an FMA, and
 * several restated formulas (BN fold, head coordinates, letterbox) are
 * compared bit-exactly.
 */
#include "oracle.h"
#include "cpu_fast.h"

/* Set while or_fast_yolov8_forward runs (the CPU baseline; see conv_t). */
static int g_fast_mode = 0;

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- helpers */

/* .NET MathF.Max(val1, val2) (IEEE 754:2019 maximum: NaN propagates, +0 > -0),
 * the semantics the reference relies on in CpuEndToEnd.cs:54-55 and the
 * separable max pool (CpuSpatial.cs:370-400). */
static float dn_max(float a, float b) {
  if (a != b) {
    if (!isnan(a)) return b < a ? a : b;
    return a;
  }
  return signbit(b) ? a : b;
}

/* .NET Single.CompareTo: NaN sorts below every number, +0 == -0. */
static int dn_compare(float a, float b) {
  if (a < b) return -1;
  if (a > b) return 1;
  if (a == b) return 0;
  if (isnan(a)) return isnan(b) ? 0 : -1;
  return 1;
}

static float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ---------------------------------------------------------------- BN fold */

/* src/SimdYolo/PtModel.cs:135-143: scale = gamma/sqrt(var+eps) (float),
 * w' = w*scale, b' = beta + (b0 - mean)*scale. */
void or_fold_bn(const float* w, int oc, int per_oc, const float* conv_bias,
                const float* gamma, const float* beta, const float* mean,
                const float* var, float eps, float* w_out, float* b_out) {
  for (int c = 0; c < oc; ++c) {
    float scale = gamma[c] / sqrtf(var[c] + eps);
    for (int j = 0; j < per_oc; ++j) w_out[(size_t)c * per_oc + j] = w[(size_t)c * per_oc + j] * scale;
    float b0 = conv_bias ? conv_bias[c] : 0.0f;
    b_out[c] = beta[c] + (b0 - mean[c]) * scale;
  }
}

/* -------------------------------------------------------------- conv2d */

/* Geometry of src/SimdYolo/Compute.cs:171-182; bias + SiLU epilogue of
 * Compute.cs:270-280.  Accumulation in double (Program.cs:210-221). */
int or_conv2d(const float* x, int n, int c, int h, int w, const float* wt,
              const float* bias, int oc, int kh, int kw, int sh, int sw,
              int pt, int pl, int pb, int pr, int dh, int dw, int groups,
              int silu, float* y, int* oh_out, int* ow_out) {
  if (groups <= 0 || c % groups || oc % groups || sh <= 0 || sw <= 0 || dh <= 0 || dw <= 0) return 1;
  long hn = (long)h + pt + pb - (long)dh * (kh - 1) - 1;
  long wn = (long)w + pl + pr - (long)dw * (kw - 1) - 1;
  if (hn < 0 || wn < 0) return 1;
  int oh = (int)(hn / sh + 1), ow = (int)(wn / sw + 1);
  if (oh_out) *oh_out = oh;
  if (ow_out) *ow_out = ow;
  if (!y) return 0;
  const int cig = c / groups, cog = oc / groups;
  const long planes = (long)n * oc;
#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)oh * ow);
#pragma omp for schedule(dynamic, 1)
    for (long p = 0; p < planes; ++p) {
      int b = (int)(p / oc), co = (int)(p % oc), g = co / cog;
      double b0 = bias ? (double)bias[co] : 0.0;
      for (long i = 0; i < (long)oh * ow; ++i) acc[i] = b0;
      for (int ci = 0; ci < cig; ++ci) {
        const float* xp = x + ((size_t)b * c + (size_t)g * cig + ci) * h * w;
        for (int ky = 0; ky < kh; ++ky)
          for (int kx = 0; kx < kw; ++kx) {
            double wv = wt[(((size_t)co * cig + ci) * kh + ky) * kw + kx];
            int ox0 = 0, ox1 = ow; /* ox range with ix in [0, w) */
            int base = kx * dw - pl;
            while (ox0 < ow && ox0 * sw + base < 0) ++ox0;
            while (ox1 > ox0 && (ox1 - 1) * sw + base >= w) --ox1;
            for (int oy = 0; oy < oh; ++oy) {
              int iy = oy * sh - pt + ky * dh;
              if (iy < 0 || iy >= h) continue;
              const float* row = xp + (size_t)iy * w;
              double* ar = acc + (size_t)oy * ow;
              if (sw == 1)
                for (int ox = ox0; ox < ox1; ++ox) ar[ox] += wv * (double)row[ox + base];
              else
                for (int ox = ox0; ox < ox1; ++ox) ar[ox] += wv * (double)row[ox * sw + base];
            }
          }
      }
      float* yp = y + (size_t)p * oh * ow;
      for (long i = 0; i < (long)oh * ow; ++i) {
        float v = (float)acc[i];
        if (silu) v = (float)((double)v / (1.0 + exp(-(double)v)));
        yp[i] = v;
      }
    }
    free(acc);
  }
  return 0;
}

/* Compute.cs:506 / :513 (x * sigmoid(x)), evaluated in double. */
void or_silu(float* x, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    double v = x[i];
    x[i] = (float)(v / (1.0 + exp(-v)));
  }
}

/* ------------------------------------------------------------- pooling */

/* Output size: Compute.cs:697-707 (PoolOutputSize). */
static long pool_out(int len, int k, int s, int before, int after, int ceil_mode) {
  long num = (long)len + before + after - k;
  if (ceil_mode) num += s - 1;
  if (num < 0) return -1;
  long size = num / s + 1;
  if (ceil_mode) {
    long lim = ((long)len + before + s - 1) / s;
    if (lim < size) size = lim;
  }
  return size;
}

/* Max pool with padding excluded (windows clipped to the image):
 * CpuSpatial.cs:345-410 and the scalar check of Program.cs:135-148. */
int or_maxpool(const float* x, int n, int c, int h, int w, int kh, int kw,
               int sh, int sw, int pt, int pl, int pb, int pr, int ceil_mode,
               float* y, int* oh_out, int* ow_out) {
  long oh = pool_out(h, kh, sh, pt, pb, ceil_mode), ow = pool_out(w, kw, sw, pl, pr, ceil_mode);
  if (oh <= 0 || ow <= 0) return 1;
  if (oh_out) *oh_out = (int)oh;
  if (ow_out) *ow_out = (int)ow;
  if (!y) return 0;
#pragma omp parallel for schedule(static)
  for (long p = 0; p < (long)n * c; ++p) {
    const float* xp = x + (size_t)p * h * w;
    float* yp = y + (size_t)p * oh * ow;
    for (long oy = 0; oy < oh; ++oy)
      for (long ox = 0; ox < ow; ++ox) {
        float m = -INFINITY;
        for (int ky = 0; ky < kh; ++ky) {
          long iy = oy * sh - pt + ky;
          if (iy < 0 || iy >= h) continue;
          for (int kx = 0; kx < kw; ++kx) {
            long ix = ox * sw - pl + kx;
            if (ix < 0 || ix >= w) continue;
            m = dn_max(m, xp[iy * w + ix]);
          }
        }
        yp[oy * ow + ox] = m;
      }
  }
  return 0;
}

/* CpuSpatial.cs:21-47: out[y][x] = in[y*ih/h][x*iw/w] (integer division). */
void or_resize_nearest(const float* x, int n, int c, int ih, int iw, int oh, int ow, float* y) {
#pragma omp parallel for schedule(static) if (g_fast_mode)
  for (long p = 0; p < (long)n * c; ++p)
    for (int yy = 0; yy < oh; ++yy)
      for (int xx = 0; xx < ow; ++xx)
        y[((size_t)p * oh + yy) * ow + xx] = x[((size_t)p * ih + (long)yy * ih / oh) * iw + (long)xx * iw / ow];
}

/* ----------------------------------------------------------- head decode */

/* CpuHead.cs:57-124 + CpuDfl.cs:19-61.  Distances: max-subtracted softmax
 * expectation over `bins` (evaluated in double, then rounded); bins == 1 uses
 * the raw regression value.  Coordinates follow CpuHead.cs:114-121 in float:
 * x1 = (col + .5 - d0) * s, y1 = (row + .5 - d1) * s, x2 = (col + .5 + d2) * s,
 * y2 = (row + .5 + d3) * s, then xywh ((x1+x2)*.5, (y1+y2)*.5, x2-x1, y2-y1)
 * unless xyxy.  Scores: 1/(1+exp(-logit)). */
void or_detect_decode(const float* boxes, const float* scores, int batch,
                      int nc, int h, int w, int bins, float stride, int xyxy,
                      float* out, int out_anchors, int start) {
  const int spatial = h * w;
  for (int b = 0; b < batch; ++b) {
    float* ob = out + (size_t)b * (nc + 4) * out_anchors;
    for (int a = 0; a < spatial; ++a) {
      float d[4];
      for (int side = 0; side < 4; ++side) {
        const float* src = boxes + ((size_t)b * 4 * bins + (size_t)side * bins) * spatial + a;
        if (bins == 1) {
          d[side] = src[0];
          continue;
        }
        float mx = -INFINITY;
        for (int r = 0; r < bins; ++r) mx = dn_max(mx, src[(size_t)r * spatial]);
        double sum = 0, num = 0;
        for (int r = 0; r < bins; ++r) {
          double e = exp((double)src[(size_t)r * spatial] - (double)mx);
          sum += e;
          num += e * r;
        }
        d[side] = (float)(num / sum);
      }
      const int col = a % w, row = a / w;
      const float cx = (float)col + .5f, cy = (float)row + .5f;
      const float x1 = (cx - d[0]) * stride, y1 = (cy - d[1]) * stride;
      const float x2 = (cx + d[2]) * stride, y2 = (cy + d[3]) * stride;
      const size_t o = (size_t)start + a;
      ob[o] = xyxy ? x1 : (x1 + x2) * .5f;
      ob[(size_t)out_anchors + o] = xyxy ? y1 : (y1 + y2) * .5f;
      ob[(size_t)2 * out_anchors + o] = xyxy ? x2 : x2 - x1;
      ob[(size_t)3 * out_anchors + o] = xyxy ? y2 : y2 - y1;
      for (int c = 0; c < nc; ++c)
        ob[(size_t)(4 + c) * out_anchors + o] = sigmoidf_ref(scores[((size_t)b * nc + c) * spatial + a]);
    }
  }
}

/* ------------------------------------------------------- end-to-end top-k */

typedef struct {
  float score;
  int index;
} entry_t;

/* ComparePt, CpuEndToEnd.cs:101-107: score descending by Single.CompareTo
 * (NaN last), ties by index ascending. */
static int cmp_pt(const void* pa, const void* pb) {
  const entry_t *a = (const entry_t*)pa, *b = (const entry_t*)pb;
  int order = -dn_compare(a->score, b->score);
  if (order) return order;
  return (a->index > b->index) - (a->index < b->index);
}

/* Compare, CpuEndToEnd.cs:203-208: NaN first, then descending, ties by index. */
static int cmp_onnx(const void* pa, const void* pb) {
  const entry_t *a = (const entry_t*)pa, *b = (const entry_t*)pb;
  int an = isnan(a->score), bn = isnan(b->score);
  int order = an ? (bn ? 0 : -1) : (bn ? 1 : -dn_compare(a->score, b->score));
  if (order) return order;
  return (a->index > b->index) - (a->index < b->index);
}

/* Per-anchor class maximum with .NET Max semantics (CpuEndToEnd.cs:47-56,
 * 161-173): NaN propagates; only the ordering of the result is used. */
static void class_maxima(const float* src, int anchors, int classes, float* maxima) {
  for (int a = 0; a < anchors; ++a) maxima[a] = -INFINITY;
  for (int c = 0; c < classes; ++c) {
    const float* row = src + (size_t)(4 + c) * anchors;
    for (int a = 0; a < anchors; ++a) maxima[a] = dn_max(maxima[a], row[a]);
  }
}

/* Full-sort restatement of SelectPt (CpuEndToEnd.cs:26-94; the same result the
 * reference test builds by full sorting, CpuPtEndToEndTests.cs:93-121).
 * Output [batch][k][6 + extra], k = min(maximum, anchors). */
int or_e2e_select_pt(const float* x, int batch, int channels, int anchors,
                     int classes, int maximum, float* out) {
  if (classes <= 0 || channels < classes + 4 || maximum < 0 || anchors < 0) return 1;
  const int k = maximum < anchors ? maximum : anchors;
  const int extra = channels - classes - 4, fields = 6 + extra;
  if (k == 0 || batch == 0) return 0;
  float* maxima = (float*)malloc(sizeof(float) * anchors);
  entry_t* cand = (entry_t*)malloc(sizeof(entry_t) * (size_t)(anchors > k * classes ? anchors : k * classes));
  for (int b = 0; b < batch; ++b) {
    const float* src = x + (size_t)b * channels * anchors;
    class_maxima(src, anchors, classes, maxima);
    for (int a = 0; a < anchors; ++a) cand[a] = (entry_t){maxima[a], a};
    qsort(cand, anchors, sizeof(entry_t), cmp_pt);
    int* sel = (int*)malloc(sizeof(int) * k);
    for (int i = 0; i < k; ++i) sel[i] = cand[i].index;
    int m = 0;
    for (int i = 0; i < k; ++i)
      for (int c = 0; c < classes; ++c)
        cand[m++] = (entry_t){src[(size_t)(4 + c) * anchors + sel[i]], sel[i] * classes + c};
    qsort(cand, m, sizeof(entry_t), cmp_pt);
    for (int i = 0; i < k; ++i) {
      int index = cand[i].index, anchor = index / classes;
      float* dst = out + ((size_t)b * k + i) * fields;
      for (int j = 0; j < 4; ++j) dst[j] = src[(size_t)j * anchors + anchor];
      dst[4] = cand[i].score;
      dst[5] = (float)(index % classes);
      for (int j = 0; j < extra; ++j) dst[6 + j] = src[(size_t)(classes + 4 + j) * anchors + anchor];
    }
    free(sel);
  }
  free(cand);
  free(maxima);
  return 0;
}

/* Full-sort restatement of SelectOnnx (CpuEndToEnd.cs:147-196).  The
 * reference does not clamp `maximum` to the anchor count; this restatement
 * requires maximum <= anchors. */
int or_e2e_select_onnx(const float* x, int batch, int channels, int anchors,
                       int classes, int maximum, float* out) {
  if (classes <= 0 || channels < classes + 4 || maximum < 0 || maximum > anchors) return 1;
  const int k = maximum, extra = channels - classes - 4, fields = 6 + extra;
  if (k == 0 || batch == 0) return 0;
  float* maxima = (float*)malloc(sizeof(float) * anchors);
  entry_t* cand = (entry_t*)malloc(sizeof(entry_t) * (size_t)(anchors > k * classes ? anchors : k * classes));
  int* rank_anchor = (int*)malloc(sizeof(int) * k);
  for (int b = 0; b < batch; ++b) {
    const float* src = x + (size_t)b * channels * anchors;
    class_maxima(src, anchors, classes, maxima);
    for (int a = 0; a < anchors; ++a) cand[a] = (entry_t){maxima[a], a};
    qsort(cand, anchors, sizeof(entry_t), cmp_onnx);
    for (int i = 0; i < k; ++i) rank_anchor[i] = cand[i].index;
    int m = 0;
    for (int c = 0; c < classes; ++c)
      for (int r = 0; r < k; ++r)
        cand[m++] = (entry_t){src[(size_t)(4 + c) * anchors + rank_anchor[r]], r * classes + c};
    qsort(cand, m, sizeof(entry_t), cmp_onnx);
    for (int i = 0; i < k; ++i) {
      int index = cand[i].index, anchor = rank_anchor[index / classes];
      float* dst = out + ((size_t)b * k + i) * fields;
      for (int j = 0; j < 4; ++j) dst[j] = src[(size_t)j * anchors + anchor];
      dst[4] = cand[i].score;
      dst[5] = (float)(index % classes);
      for (int j = 0; j < extra; ++j) dst[6 + j] = src[(size_t)(classes + 4 + j) * anchors + anchor];
    }
  }
  free(rank_anchor);
  free(cand);
  free(maxima);
  return 0;
}

/* ------------------------------------------------------------------ NMS */

/* YoloDetector.cs:648-652. */
float or_iou(const or_detection* a, const or_detection* b) {
  float w = fmaxf(0, fminf(a->x + a->width, b->x + b->width) - fmaxf(a->x, b->x));
  float h = fmaxf(0, fminf(a->y + a->height, b->y + b->height) - fmaxf(a->y, b->y));
  float inter = w * h;
  float den = a->width * a->height + b->width * b->height - inter;
  return inter / fmaxf(FLT_TRUE_MIN, den);
}

typedef struct {
  or_detection d;
  int order;
} cand_t;

/* Stable descending order by confidence (Enumerable.OrderByDescending). */
static int cmp_cand(const void* pa, const void* pb) {
  const cand_t *a = (const cand_t*)pa, *b = (const cand_t*)pb;
  int o = -dn_compare(a->d.confidence, b->d.confidence);
  if (o) return o;
  return (a->order > b->order) - (a->order < b->order);
}

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* DetectionDecoder.DecodeIndexed, YoloDetector.cs:539-643. */
int or_nms_decode(const float* data, int dim1, int dim2, int layout,
                  int class_count, float confidence, float iou,
                  int max_detections, int max_candidates, int agnostic,
                  const or_letterbox_t* t, or_detection* out, int* count) {
  *count = 0;
  if (max_detections <= 0 || max_candidates <= 0 || class_count < 0) return 1;
  if (layout == 0) {
    int expected = class_count > 0 ? 4 + class_count : 0;
    if (expected > 0 && dim1 == expected && dim2 != expected) layout = 1;
    else if (expected > 0 && dim2 == expected && dim1 != expected) layout = 2;
    else if (dim2 == 6 && dim1 != 6) layout = 3;
    else if (dim1 >= 5 && dim1 < dim2) layout = 1;
    else if (dim2 >= 5 && dim2 < dim1) layout = 2;
    else return 2;
  }
  const int end2end = layout == 3, cf = layout == 1;
  const int n = cf ? dim2 : dim1, fields = cf ? dim1 : dim2;
  if (fields < 5 || (end2end && fields != 6)) return 1;
  const int class_fields = class_count > 0 ? 4 + class_count : fields;
  if (!end2end && (class_fields < 5 || class_fields > fields)) return 1;
#define AT(a, c) data[cf ? (size_t)(c) * n + (a) : (size_t)(a) * fields + (c)]
  cand_t* cands = (cand_t*)malloc(sizeof(cand_t) * (size_t)(n > 0 ? n : 1));
  int nc = 0;
  for (int a = 0; a < n; ++a) {
    int cls = 0;
    float conf;
    if (end2end) {
      conf = AT(a, 4);
      float cv = AT(a, 5);
      if (!isfinite(cv) || cv < 0 || cv != truncf(cv)) continue;
      cls = (int)cv;
    } else {
      conf = -INFINITY;
      for (int c = 4; c < class_fields; ++c) {
        float s = AT(a, c);
        if (s > conf) {
          conf = s;
          cls = c - 4;
        }
      }
    }
    if (!isfinite(conf) || conf < confidence) continue;
    float x = AT(a, 0), y = AT(a, 1), w = AT(a, 2), h = AT(a, 3);
    if (!isfinite(x) || !isfinite(y) || !isfinite(w) || !isfinite(h)) continue;
    if (end2end) {
      w -= x;
      h -= y;
    } else {
      x -= w * .5f;
      y -= h * .5f;
    }
    if (w <= 0 || h <= 0) continue;
    cands[nc].d = (or_detection){cls, conf, x, y, w, h, a};
    cands[nc].order = nc;
    ++nc;
  }
#undef AT
  qsort(cands, nc, sizeof(cand_t), cmp_cand);
  if (nc > max_candidates) nc = max_candidates;
  or_detection* kept = (or_detection*)malloc(sizeof(or_detection) * (size_t)max_detections);
  int nk = 0;
  for (int i = 0; i < nc && nk < max_detections; ++i) {
    const or_detection* d = &cands[i].d;
    if (!end2end) {
      int suppressed = 0;
      for (int j = 0; j < nk; ++j) {
        if (!(agnostic || kept[j].class_id == d->class_id)) continue;
        if (!(or_iou(&kept[j], d) > iou)) continue;
        suppressed = 1;
        break;
      }
      if (suppressed) continue;
    }
    kept[nk++] = *d;
  }
  int m = 0;
  for (int i = 0; i < nk; ++i) {
    or_detection d = kept[i];
    float x1 = clampf((d.x - t->pad_x) / t->scale_x, 0, (float)t->source_width);
    float y1 = clampf((d.y - t->pad_y) / t->scale_y, 0, (float)t->source_height);
    float x2 = clampf((d.x + d.width - t->pad_x) / t->scale_x, 0, (float)t->source_width);
    float y2 = clampf((d.y + d.height - t->pad_y) / t->scale_y, 0, (float)t->source_height);
    d.x = x1;
    d.y = y1;
    d.width = x2 - x1;
    d.height = y2 - y1;
    if (d.width > 0 && d.height > 0) out[m++] = d;
  }
  *count = m;
  free(kept);
  free(cands);
  return 0;
}

/* ------------------------------------------------------------- masks */

/* Source-axis -> prototype-axis bilinear tables (CpuMaskDecoder.cs:33-38). */
static void mask_map(int length, int start, int end, int* first, int* second, float* frac) {
  for (int i = 0; i < length; ++i) {
    float c = start + (i + .5f) * (end - start) / length - .5f;
    if (c < start) c = (float)start;
    if (c > end - 1) c = (float)(end - 1);
    first[i] = (int)c;
    second[i] = first[i] + 1 < end - 1 ? first[i] + 1 : end - 1;
    frac[i] = c - first[i];
  }
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* CpuMaskDecoder.cs:18-81: low = sum_c coeff_c * proto_c (double here), ROI of
 * the letterboxed image inside the prototype grid, half-pixel bilinear map of
 * each source pixel, sigmoid, crop to the box (pixels left of ceil(x) or above
 * ceil(y) stay 0). */
int or_mask_decode(const float* proto, int nm, int mh, int mw, const float* coeffs, const or_detection* box,
                   const or_letterbox_t* t, float* out, int* info) {
  const int plane = mh * mw;
  int left_roi = clampi((int)rintf((float)t->pad_x * mw / t->target_width), 0, mw - 1);
  int top_roi = clampi((int)rintf((float)t->pad_y * mh / t->target_height), 0, mh - 1);
  int right_roi = clampi((int)rintf((t->pad_x + t->source_width * t->scale_x) * mw / t->target_width), left_roi + 1, mw);
  int bottom_roi =
      clampi((int)rintf((t->pad_y + t->source_height * t->scale_y) * mh / t->target_height), top_roi + 1, mh);
  int left = (int)floorf(box->x), top = (int)floorf(box->y);
  int right = (int)ceilf(box->x + box->width), bottom = (int)ceilf(box->y + box->height);
  int width = right - left, height = bottom - top;
  info[0] = left; info[1] = top; info[2] = width; info[3] = height;
  if (!out) return 0;
  if (width <= 0 || height <= 0 || right > t->source_width || bottom > t->source_height || left < 0 || top < 0)
    return 1;
  double* low = (double*)calloc((size_t)plane, sizeof(double));
  for (int c = 0; c < nm; ++c)
    for (int i = 0; i < plane; ++i) low[i] += (double)coeffs[c] * proto[(size_t)c * plane + i];
  int *x0 = (int*)malloc(sizeof(int) * t->source_width), *x1 = (int*)malloc(sizeof(int) * t->source_width);
  int *y0 = (int*)malloc(sizeof(int) * t->source_height), *y1 = (int*)malloc(sizeof(int) * t->source_height);
  float *fx = (float*)malloc(sizeof(float) * t->source_width), *fy = (float*)malloc(sizeof(float) * t->source_height);
  mask_map(t->source_width, left_roi, right_roi, x0, x1, fx);
  mask_map(t->source_height, top_roi, bottom_roi, y0, y1, fy);
  int begin_x = (int)ceilf(box->x), begin_y = (int)ceilf(box->y);
  if (begin_x < left) begin_x = left;
  if (begin_y < top) begin_y = top;
  for (int y = top; y < bottom; ++y)
    for (int x = left; x < right; ++x) {
      float v = 0.0f;
      if (y >= begin_y && x >= begin_x) {
        double u = low[(size_t)y0[y] * mw + x0[x]] * (1.0 - fx[x]) + low[(size_t)y0[y] * mw + x1[x]] * fx[x];
        double d = low[(size_t)y1[y] * mw + x0[x]] * (1.0 - fx[x]) + low[(size_t)y1[y] * mw + x1[x]] * fx[x];
        double z = u * (1.0 - fy[y]) + d * fy[y];
        v = (float)(1.0 / (1.0 + exp(-z)));
      }
      out[(size_t)(y - top) * width + (x - left)] = v;
    }
  free(low); free(x0); free(x1); free(y0); free(y1); free(fx); free(fy);
  return 0;
}

/* ------------------------------------------------------------- letterbox */

/* ImagePreprocessor.Letterbox, YoloDetector.cs:448-507.  MathF.Round is
 * round-half-to-even, which is rintf under the default rounding mode. */
int or_letterbox(const uint8_t* pixels, int width, int height, int tw, int th,
                 int bgr, int row_stride, float* out, or_letterbox_t* t) {
  if (width <= 0 || height <= 0 || tw <= 0 || th <= 0) return 1;
  if (row_stride == 0) row_stride = width * 3;
  float gain = fminf((float)tw / width, (float)th / height);
  int rw = (int)rintf(width * gain), rh = (int)rintf(height * gain);
  rw = rw < 1 ? 1 : (rw > tw ? tw : rw);
  rh = rh < 1 ? 1 : (rh > th ? th : rh);
  int px = (tw - rw) / 2, py = (th - rh) / 2;
  size_t plane = (size_t)tw * th;
  const float pad = 114.0f / 255.0f;
  for (size_t i = 0; i < 3 * plane; ++i) out[i] = pad;
  int red = bgr ? 2 : 0, blue = 2 - red;
  for (int y = 0; y < rh; ++y) {
    float sy = (y + .5f) * height / rh - .5f;
    sy = sy < 0 ? 0 : (sy > height - 1 ? (float)(height - 1) : sy);
    int y0 = (int)sy, y1 = y0 + 1 < height - 1 ? y0 + 1 : height - 1;
    float fy = sy - y0, wy = 1 - fy;
    const uint8_t *top = pixels + (size_t)y0 * row_stride, *bot = pixels + (size_t)y1 * row_stride;
    float* r = out + (size_t)(y + py) * tw + px;
    for (int x = 0; x < rw; ++x) {
      float sx = (x + .5f) * width / rw - .5f;
      sx = sx < 0 ? 0 : (sx > width - 1 ? (float)(width - 1) : sx);
      int left = (int)sx, right = left + 1 < width - 1 ? left + 1 : width - 1;
      float fx = sx - left, wx = 1 - fx;
      int ch[3] = {red, 1, blue};
      for (int p = 0; p < 3; ++p) {
        int o = ch[p];
        float upper = top[left * 3 + o] * wx + top[right * 3 + o] * fx;
        float lower = bot[left * 3 + o] * wx + bot[right * 3 + o] * fx;
        r[(size_t)p * plane + x] = (upper * wy + lower * fy) / 255.0f;
      }
    }
  }
  t->source_width = width;
  t->source_height = height;
  t->target_width = tw;
  t->target_height = th;
  t->scale_x = (float)rw / width;
  t->scale_y = (float)rh / height;
  t->pad_x = px;
  t->pad_y = py;
  return 0;
}

/* ------------------------------------------------- YOLOv8 detect network */

/* Topology: ultralytics yolov8.yaml (the module tree the reference's
 * PtModel interprets); module semantics from PtModel.cs:277-317 (Conv, C2f,
 * Bottleneck add, SPPF, Upsample, Concat) and PtModel.cs:444-504 (Detect). */

typedef struct {
  int n, c, h, w;
  float* d;
} t4;

/* In fast mode freed activations go to a small pool reused by size, as the
 * reference's CPU path rents its tensors from pooled arrays
 * (Tensor.TemporaryUninitialized, ArrayPool): no page faults after the first
 * pass.  Outside fast mode plain malloc/free. */
enum { POOL_SLOTS = 64 };
static struct { float* d; size_t len; } g_pool[POOL_SLOTS];

static t4 t_new(int n, int c, int h, int w) {
  const size_t len = (size_t)n * c * h * w;
  if (g_fast_mode)
    for (int i = 0; i < POOL_SLOTS; ++i)
      if (g_pool[i].d && g_pool[i].len == len) {
        t4 t = {n, c, h, w, g_pool[i].d};
        g_pool[i].d = NULL;
        return t;
      }
  t4 t = {n, c, h, w, (float*)malloc(sizeof(float) * len)};
  return t;
}
static void t_free(t4* t) {
  if (g_fast_mode && t->d) {
    for (int i = 0; i < POOL_SLOTS; ++i)
      if (!g_pool[i].d) {
        g_pool[i].d = t->d;
        g_pool[i].len = (size_t)t->n * t->c * t->h * t->w;
        t->d = NULL;
        return;
      }
  }
  free(t->d);
  t->d = NULL;
}

static void pool_release(void) {
  for (int i = 0; i < POOL_SLOTS; ++i) {
    free(g_pool[i].d);
    g_pool[i].d = NULL;
  }
}

typedef struct {
  /* enumeration */
  int* layout;
  int max_tensors, count;
  /* parameter stream */
  const float* params;
  size_t n_params, pos;
  int fail;
  float eps;
} cursor_t;

/* Registers one tensor (kind + dims) and returns a pointer to its data in the
 * parameter stream (NULL in enumeration mode). */
static const float* take(cursor_t* cur, int kind, int d0, int d1, int d2, int d3, int fan_in) {
  if (cur->layout && cur->count < cur->max_tensors) {
    int* e = cur->layout + 6 * cur->count;
    e[0] = kind; e[1] = d0; e[2] = d1; e[3] = d2; e[4] = d3; e[5] = fan_in;
  }
  cur->count++;
  size_t len = (size_t)d0 * d1 * d2 * d3;
  const float* p = NULL;
  if (cur->params) {
    if (cur->pos + len > cur->n_params) cur->fail = 1;
    else p = cur->params + cur->pos;
  }
  cur->pos += len;
  return p;
}

enum { K_CONV_W = 0, K_BN_GAMMA, K_BN_BETA, K_BN_MEAN, K_BN_VAR, K_BIAS_BOX, K_BIAS_CLS, K_BIAS };

/* A Conv module (conv + BN folded + optional SiLU) or a plain Conv2d with bias. */
typedef struct {
  int ic, oc, k, s;
  int silu;
  float *w, *b; /* folded, owned */
  int g;        /* groups */
  cf_conv* fast; /* CPU-baseline plan, built on first use in fast mode */
} conv_t;

/* In fast mode (or_fast_yolov8_forward) convolutions and the detect decode
 * take the CPU-baseline restatement of the reference's FP32 CPU algorithms
 * (cpu_fast.c) instead of the double-accumulating loops, and the copies and
 * adds run on all threads; their arithmetic is unchanged. */

/* Conv(c1, c2, k, s, g, act): conv (no bias) + BN folded + SiLU when act. */
static conv_t load_conv_ga(cursor_t* cur, int ic, int oc, int k, int s, int g, int act) {
  conv_t cv = {ic, oc, k, s, act, NULL, NULL, g, NULL};
  const int icg = ic / g;
  const float* w = take(cur, K_CONV_W, oc, icg, k, k, icg * k * k);
  const float* ga = take(cur, K_BN_GAMMA, oc, 1, 1, 1, 0);
  const float* be = take(cur, K_BN_BETA, oc, 1, 1, 1, 0);
  const float* mu = take(cur, K_BN_MEAN, oc, 1, 1, 1, 0);
  const float* va = take(cur, K_BN_VAR, oc, 1, 1, 1, 0);
  if (w && ga && be && mu && va) {
    cv.w = (float*)malloc(sizeof(float) * (size_t)oc * icg * k * k);
    cv.b = (float*)malloc(sizeof(float) * oc);
    or_fold_bn(w, oc, icg * k * k, NULL, ga, be, mu, va, cur->eps, cv.w, cv.b);
  }
  return cv;
}

static conv_t load_conv(cursor_t* cur, int ic, int oc, int k, int s) { return load_conv_ga(cur, ic, oc, k, s, 1, 1); }

static conv_t load_conv2d(cursor_t* cur, int ic, int oc, int bias_kind) {
  conv_t cv = {ic, oc, 1, 1, 0, NULL, NULL, 1, NULL};
  const float* w = take(cur, K_CONV_W, oc, ic, 1, 1, ic);
  const float* b = take(cur, bias_kind, oc, 1, 1, 1, 0);
  if (w && b) {
    cv.w = (float*)malloc(sizeof(float) * (size_t)oc * ic);
    cv.b = (float*)malloc(sizeof(float) * oc);
    memcpy(cv.w, w, sizeof(float) * (size_t)oc * ic);
    memcpy(cv.b, b, sizeof(float) * oc);
  }
  return cv;
}

static void free_conv(conv_t* c) {
  free(c->w);
  free(c->b);
  cf_conv_destroy(c->fast);
  c->fast = NULL;
}

static t4 run_conv(const conv_t* cv, t4 x) {
  int p = cv->k / 2, oh, ow;
  if (g_fast_mode) {
    conv_t* m = (conv_t*)cv;
    if (!m->fast) m->fast = cf_conv_create(cv->w, cv->b, cv->oc, cv->ic, cv->k, cv->s, cv->g, cv->silu);
    cf_conv_run(m->fast, x.d, x.n, x.h, x.w, NULL, &oh, &ow);
    t4 y = t_new(x.n, cv->oc, oh, ow);
    cf_conv_run(m->fast, x.d, x.n, x.h, x.w, y.d, NULL, NULL);
    return y;
  }
  or_conv2d(x.d, x.n, x.c, x.h, x.w, cv->w, cv->b, cv->oc, cv->k, cv->k, cv->s, cv->s, p, p, p, p, 1, 1, cv->g,
            0, NULL, &oh, &ow);
  t4 y = t_new(x.n, cv->oc, oh, ow);
  or_conv2d(x.d, x.n, x.c, x.h, x.w, cv->w, cv->b, cv->oc, cv->k, cv->k, cv->s, cv->s, p, p, p, p, 1, 1, cv->g,
            cv->silu, y.d, NULL, NULL);
  return y;
}

static void add_into(t4* dst, t4 src) {
  size_t len = (size_t)dst->n * dst->c * dst->h * dst->w;
#pragma omp parallel for schedule(static) if (g_fast_mode)
  for (size_t j = 0; j < len; ++j) dst->d[j] = src.d[j] + dst->d[j];
}

/* Channel concat (Compute.cs:520-540 on axis 1). */
static t4 cat(const t4* xs, int count) {
  int c = 0;
  for (int i = 0; i < count; ++i) c += xs[i].c;
  t4 y = t_new(xs[0].n, c, xs[0].h, xs[0].w);
  size_t plane = (size_t)xs[0].h * xs[0].w;
  for (int b = 0; b < y.n; ++b) {
    int off = 0;
    for (int i = 0; i < count; ++i) {
#pragma omp parallel for schedule(static) if (g_fast_mode)
      for (int ch = 0; ch < xs[i].c; ++ch)
        memcpy(y.d + ((size_t)b * c + off + ch) * plane, xs[i].d + ((size_t)b * xs[i].c + ch) * plane,
               sizeof(float) * plane);
      off += xs[i].c;
    }
  }
  return y;
}

static t4 channel_slice(t4 x, int start, int count) {
  t4 y = t_new(x.n, count, x.h, x.w);
  size_t plane = (size_t)x.h * x.w;
  for (int b = 0; b < x.n; ++b)
#pragma omp parallel for schedule(static) if (g_fast_mode)
    for (int ch = 0; ch < count; ++ch)
      memcpy(y.d + ((size_t)b * count + ch) * plane, x.d + ((size_t)b * x.c + start + ch) * plane,
             sizeof(float) * plane);
  return y;
}

/* C2f (PtModel.cs:307): ys = chunk(cv1(x)); ys += m_i(ys[-1]); cv2(cat(ys)).
 * Bottleneck (PtModel.cs:302-303): cv2(cv1(x)), plus x when `add`. */
typedef struct {
  conv_t cv1, cv2;
  conv_t m[16][2];
  int n, c, add;
} c2f_t;

static c2f_t load_c2f(cursor_t* cur, int c1, int c2, int n, int shortcut) {
  c2f_t m;
  memset(&m, 0, sizeof m);
  m.n = n;
  m.c = c2 / 2;
  m.add = shortcut;
  m.cv1 = load_conv(cur, c1, 2 * m.c, 1, 1);
  m.cv2 = load_conv(cur, (2 + n) * m.c, c2, 1, 1);
  for (int i = 0; i < n; ++i) {
    m.m[i][0] = load_conv(cur, m.c, m.c, 3, 1);
    m.m[i][1] = load_conv(cur, m.c, m.c, 3, 1);
  }
  return m;
}

static t4 run_c2f(const c2f_t* m, t4 x) {
  t4 y = run_conv(&m->cv1, x);
  t4 ys[18];
  ys[0] = channel_slice(y, 0, m->c);
  ys[1] = channel_slice(y, m->c, m->c);
  t_free(&y);
  for (int i = 0; i < m->n; ++i) {
    t4 a = run_conv(&m->m[i][0], ys[i + 1]);
    t4 b = run_conv(&m->m[i][1], a);
    t_free(&a);
    if (m->add) {
      size_t len = (size_t)b.n * b.c * b.h * b.w;
      /* Add(X(), bneck): x + f(x) (PtModel.cs:303; Compute.cs:429-476). */
      for (size_t j = 0; j < len; ++j) b.d[j] = ys[i + 1].d[j] + b.d[j];
    }
    ys[i + 2] = b;
  }
  t4 joined = cat(ys, m->n + 2);
  for (int i = 0; i < m->n + 2; ++i) t_free(&ys[i]);
  t4 out = run_conv(&m->cv2, joined);
  t_free(&joined);
  return out;
}

static void free_c2f(c2f_t* m) {
  free_conv(&m->cv1);
  free_conv(&m->cv2);
  for (int i = 0; i < m->n; ++i) {
    free_conv(&m->m[i][0]);
    free_conv(&m->m[i][1]);
  }
}

/* SPPF (PtModel.cs:310-311): cv1, then n=3 chained MaxPool2d(5, 1, 2), cv2 of the concat. */
typedef struct {
  conv_t cv1, cv2;
} sppf_t;

static t4 run_sppf(const sppf_t* m, t4 x) {
  t4 ys[4];
  ys[0] = run_conv(&m->cv1, x);
  for (int i = 1; i < 4; ++i) {
    t4 p = t_new(ys[i - 1].n, ys[i - 1].c, ys[i - 1].h, ys[i - 1].w);
    or_maxpool(ys[i - 1].d, p.n, p.c, p.h, p.w, 5, 5, 1, 1, 2, 2, 2, 2, 0, p.d, NULL, NULL);
    ys[i] = p;
  }
  t4 joined = cat(ys, 4);
  for (int i = 0; i < 4; ++i) t_free(&ys[i]);
  t4 out = run_conv(&m->cv2, joined);
  t_free(&joined);
  return out;
}

static t4 upsample2(t4 x) {
  t4 y = t_new(x.n, x.c, x.h * 2, x.w * 2);
  or_resize_nearest(x.d, x.n, x.c, x.h, x.w, y.h, y.w, y.d);
  return y;
}

/* ultralytics make_divisible(min(c, max_channels) * width, 8) and the repeat
 * rule max(round(n * depth), 1). */
static int scale_ch(const or_yolo_cfg* cfg, int c) {
  double v = (double)(c < cfg->max_channels ? c : cfg->max_channels) * cfg->width;
  return (int)(ceil(v / 8.0) * 8.0);
}
static int scale_n(const or_yolo_cfg* cfg, int n) {
  if (n <= 1) return n;
  int r = (int)lround((double)n * cfg->depth);
  /* Python's round() is half-to-even; n*depth never lands on .5 for the
   * published scales. */
  return r < 1 ? 1 : r;
}

/* ------------------------------------------------- Segment head */

void or_conv_transpose2x2(const float* x, int n, int ic, int h, int w, const float* wt, const float* bias, int oc,
                          float* y) {
  const size_t plane = (size_t)h * w;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < n; ++b)
    for (int o = 0; o < oc; ++o)
      for (int i = 0; i < h; ++i)
        for (int j = 0; j < w; ++j)
          for (int dy = 0; dy < 2; ++dy)
            for (int dx = 0; dx < 2; ++dx) {
              double acc = bias ? bias[o] : 0.0;
              for (int c = 0; c < ic; ++c)
                acc += (double)x[((size_t)b * ic + c) * plane + (size_t)i * w + j] *
                       wt[(((size_t)c * oc + o) * 2 + dy) * 2 + dx];
              y[(((size_t)b * oc + o) * 2 * h + 2 * i + dy) * 2 * w + 2 * j + dx] = (float)acc;
            }
}

typedef struct {
  int ic, oc;
  float *w, *b;
} deconv_t;

static deconv_t load_deconv2(cursor_t* cur, int ic, int oc) {
  deconv_t d = {ic, oc, NULL, NULL};
  const float* w = take(cur, K_CONV_W, ic, oc, 2, 2, oc * 4);
  const float* b = take(cur, K_BIAS, oc, 1, 1, 1, oc * 4);
  if (w && b) {
    d.w = (float*)malloc(sizeof(float) * (size_t)ic * oc * 4);
    d.b = (float*)malloc(sizeof(float) * oc);
    memcpy(d.w, w, sizeof(float) * (size_t)ic * oc * 4);
    memcpy(d.b, b, sizeof(float) * oc);
  }
  return d;
}

/* Proto(c1, c_, nm) (PtModel.cs:344): cv3(cv2(upsample(cv1(x)))), cv1 and
 * cv2 3x3 Conv, upsample ConvTranspose2d(c_, c_, 2, 2), cv3 1x1 Conv. */
typedef struct {
  conv_t cv1, cv2, cv3;
  deconv_t up;
} proto_t;

/* Segment (PtModel.cs:353-360): the Detect branches, then Proto on the P3
 * feature, then per level cv4 = Conv(x, c4, 3), Conv(c4, c4, 3),
 * Conv2d(c4, nm, 1) with c4 = max(ch0 / 4, nm); state_dict order cv2, cv3,
 * (dfl), proto, cv4. */
typedef struct {
  proto_t proto;
  conv_t cv4[3][3];
  int nm;
} seg_t;

static void load_seg(cursor_t* cur, const or_yolo_cfg* cfg, const int ch[3], int npr_scaled, seg_t* s) {
  memset(s, 0, sizeof *s);
  s->nm = cfg->nm;
  const int c_ = npr_scaled;
  s->proto.cv1 = load_conv(cur, ch[0], c_, 3, 1);
  s->proto.up = load_deconv2(cur, c_, c_);
  s->proto.cv2 = load_conv(cur, c_, c_, 3, 1);
  s->proto.cv3 = load_conv(cur, c_, cfg->nm, 1, 1);
  const int c4 = ch[0] / 4 > cfg->nm ? ch[0] / 4 : cfg->nm;
  for (int i = 0; i < 3; ++i) {
    s->cv4[i][0] = load_conv(cur, ch[i], c4, 3, 1);
    s->cv4[i][1] = load_conv(cur, c4, c4, 3, 1);
    s->cv4[i][2] = load_conv2d(cur, c4, cfg->nm, K_BIAS);
  }
}

static void free_seg(seg_t* s) {
  free_conv(&s->proto.cv1);
  free_conv(&s->proto.cv2);
  free_conv(&s->proto.cv3);
  free(s->proto.up.w);
  free(s->proto.up.b);
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) free_conv(&s->cv4[i][j]);
}

/* Proto on feats[0] into proto_out ([n, nm, 2h, 2w]); the mask coefficients
 * of every level appended to the head as channels nc+4.. (CompleteInstanceHead
 * concat, PtModel.cs:523).  `head` is [n, nc+4+nm, anchors]. */
static void run_seg(const seg_t* s, const t4 feats[3], int nc, float* head, int anchors, float* proto_out) {
  t4 a = run_conv(&s->proto.cv1, feats[0]);
  t4 u = t_new(a.n, s->proto.up.oc, 2 * a.h, 2 * a.w);
  or_conv_transpose2x2(a.d, a.n, a.c, a.h, a.w, s->proto.up.w, s->proto.up.b, s->proto.up.oc, u.d);
  t_free(&a);
  t4 b = run_conv(&s->proto.cv2, u); t_free(&u);
  t4 p = run_conv(&s->proto.cv3, b); t_free(&b);
  if (proto_out) memcpy(proto_out, p.d, sizeof(float) * (size_t)p.n * p.c * p.h * p.w);
  t_free(&p);
  const int C = nc + 4 + s->nm;
  int start = 0;
  for (int i = 0; i < 3; ++i) {
    t4 x0 = run_conv(&s->cv4[i][0], feats[i]);
    t4 x1 = run_conv(&s->cv4[i][1], x0); t_free(&x0);
    t4 mc = run_conv(&s->cv4[i][2], x1); t_free(&x1);
    const int hw = mc.h * mc.w;
    for (int bb = 0; bb < mc.n; ++bb)
      for (int j = 0; j < s->nm; ++j)
        memcpy(head + ((size_t)bb * C + nc + 4 + j) * anchors + start, mc.d + ((size_t)bb * s->nm + j) * hw,
               sizeof(float) * hw);
    start += hw;
    t_free(&mc);
  }
}

/* The detect decode writes [n, nc+4, anchors]; a Segment head's output has
 * nm more channels, so decode into a scratch head and copy its channels. */
static void widen_head(const float* det, float* head, int n, int nc, int nm, int anchors) {
  for (int b = 0; b < n; ++b)
    memcpy(head + (size_t)b * (nc + 4 + nm) * anchors, det + (size_t)b * (nc + 4) * anchors,
           sizeof(float) * (size_t)(nc + 4) * anchors);
}

typedef struct {
  conv_t c0, c1, c3, c5, c7, c16, c19;
  c2f_t f2, f4, f6, f8, f12, f15, f18, f21;
  sppf_t s9;
  conv_t box[3][3], cls[3][3];
  int ch[3], c2, c3h, nc, reg_max;
  seg_t seg;
} yolov8_t;

static void load_yolov8(cursor_t* cur, const or_yolo_cfg* cfg, yolov8_t* m) {
  memset(m, 0, sizeof *m);
  int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
      c1024 = scale_ch(cfg, 1024);
  int n3 = scale_n(cfg, 3), n6 = scale_n(cfg, 6);
  m->c0 = load_conv(cur, 3, c64, 3, 2);
  m->c1 = load_conv(cur, c64, c128, 3, 2);
  m->f2 = load_c2f(cur, c128, c128, n3, 1);
  m->c3 = load_conv(cur, c128, c256, 3, 2);
  m->f4 = load_c2f(cur, c256, c256, n6, 1);
  m->c5 = load_conv(cur, c256, c512, 3, 2);
  m->f6 = load_c2f(cur, c512, c512, n6, 1);
  m->c7 = load_conv(cur, c512, c1024, 3, 2);
  m->f8 = load_c2f(cur, c1024, c1024, n3, 1);
  m->s9.cv1 = load_conv(cur, c1024, c1024 / 2, 1, 1);
  m->s9.cv2 = load_conv(cur, c1024 / 2 * 4, c1024, 1, 1);
  m->f12 = load_c2f(cur, c1024 + c512, c512, n3, 0);
  m->f15 = load_c2f(cur, c512 + c256, c256, n3, 0);
  m->c16 = load_conv(cur, c256, c256, 3, 2);
  m->f18 = load_c2f(cur, c256 + c512, c512, n3, 0);
  m->c19 = load_conv(cur, c512, c512, 3, 2);
  m->f21 = load_c2f(cur, c512 + c1024, c1024, n3, 0);
  m->ch[0] = c256;
  m->ch[1] = c512;
  m->ch[2] = c1024;
  m->nc = cfg->nc;
  m->reg_max = cfg->reg_max;
  /* Detect: c2 = max(16, ch0 // 4, 4*reg_max), c3 = max(ch0, min(nc, 100)). */
  int c2 = 16;
  if (c256 / 4 > c2) c2 = c256 / 4;
  if (4 * cfg->reg_max > c2) c2 = 4 * cfg->reg_max;
  int c3 = cfg->nc < 100 ? cfg->nc : 100;
  if (c256 > c3) c3 = c256;
  m->c2 = c2;
  m->c3h = c3;
  for (int i = 0; i < 3; ++i) {
    m->box[i][0] = load_conv(cur, m->ch[i], c2, 3, 1);
    m->box[i][1] = load_conv(cur, c2, c2, 3, 1);
    m->box[i][2] = load_conv2d(cur, c2, 4 * cfg->reg_max, K_BIAS_BOX);
  }
  for (int i = 0; i < 3; ++i) {
    m->cls[i][0] = load_conv(cur, m->ch[i], c3, 3, 1);
    m->cls[i][1] = load_conv(cur, c3, c3, 3, 1);
    m->cls[i][2] = load_conv2d(cur, c3, cfg->nc, K_BIAS_CLS);
  }
  if (cfg->nm > 0) load_seg(cur, cfg, m->ch, scale_ch(cfg, cfg->npr), &m->seg);
}

static void free_yolov8(yolov8_t* m) {
  conv_t* cs[] = {&m->c0, &m->c1, &m->c3, &m->c5, &m->c7, &m->c16, &m->c19, &m->s9.cv1, &m->s9.cv2};
  for (size_t i = 0; i < sizeof cs / sizeof cs[0]; ++i) free_conv(cs[i]);
  c2f_t* fs[] = {&m->f2, &m->f4, &m->f6, &m->f8, &m->f12, &m->f15, &m->f18, &m->f21};
  for (size_t i = 0; i < sizeof fs / sizeof fs[0]; ++i) free_c2f(fs[i]);
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      free_conv(&m->box[i][j]);
      free_conv(&m->cls[i][j]);
    }
  free_seg(&m->seg);
}

int or_yolov8_layout(const or_yolo_cfg* cfg, int* out, int max_tensors) {
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.layout = out;
  cur.max_tensors = max_tensors;
  cur.eps = cfg->bn_eps;
  yolov8_t m;
  load_yolov8(&cur, cfg, &m);
  free_yolov8(&m);
  return cur.count;
}

static int run_yolov8(yolov8_t* mp, const or_yolo_cfg* cfg, const float* input, int batch, int h, int w,
                      float* out, size_t out_capacity, float* proto_out);

int or_yolov8_forward(const or_yolo_cfg* cfg, const float* params, size_t n_params, const float* input, int batch,
                      int h, int w, float* out, size_t out_capacity, float* proto_out) {
  if (h % 32 || w % 32 || batch <= 0) return 1;
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.params = params;
  cur.n_params = n_params;
  cur.eps = cfg->bn_eps;
  yolov8_t m;
  load_yolov8(&cur, cfg, &m);
  if (cur.fail || cur.pos != n_params) {
    free_yolov8(&m);
    return 2;
  }
  const int rc = run_yolov8(&m, cfg, input, batch, h, w, out, out_capacity, proto_out);
  free_yolov8(&m);
  return rc;
}

/* CPU baseline: the same YOLOv8 walk with the weights loaded (BN folded,
 * convolutions planned) once and the convolutions on cpu_fast.c. */
struct or_fast_model {
  or_yolo_cfg cfg;
  yolov8_t m;
};

or_fast_model* or_fast_yolov8_create(const or_yolo_cfg* cfg, const float* params, size_t n_params) {
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.params = params;
  cur.n_params = n_params;
  cur.eps = cfg->bn_eps;
  or_fast_model* f = (or_fast_model*)calloc(1, sizeof(or_fast_model));
  if (!f) return NULL;
  f->cfg = *cfg;
  load_yolov8(&cur, cfg, &f->m);
  if (cur.fail || cur.pos != n_params) {
    free_yolov8(&f->m);
    free(f);
    return NULL;
  }
  return f;
}

int or_fast_yolov8_forward(or_fast_model* f, const float* input, int batch, int h, int w, float* out,
                           size_t out_capacity) {
  if (!f || h % 32 || w % 32 || batch <= 0 || f->cfg.nm > 0) return 1;
  g_fast_mode = 1;
  const int rc = run_yolov8(&f->m, &f->cfg, input, batch, h, w, out, out_capacity, NULL);
  g_fast_mode = 0;
  return rc;
}

void or_fast_yolov8_destroy(or_fast_model* f) {
  if (!f) return;
  free_yolov8(&f->m);
  free(f);
  pool_release();
}

int or_fast_threads(void) { return cf_threads(); }

static int run_yolov8(yolov8_t* mp, const or_yolo_cfg* cfg, const float* input, int batch, int h, int w,
                      float* out, size_t out_capacity, float* proto_out) {
  const int anchors = (h / 8) * (w / 8) + (h / 16) * (w / 16) + (h / 32) * (w / 32);
  const int nm = cfg->nm > 0 ? cfg->nm : 0;
  if ((size_t)batch * (mp->nc + 4 + nm) * anchors > out_capacity) return 3;
  float* det = nm ? (float*)malloc(sizeof(float) * (size_t)batch * (mp->nc + 4) * anchors) : out;
  t4 x = {batch, 3, h, w, (float*)input};
  t4 l0 = run_conv(&mp->c0, x);
  t4 l1 = run_conv(&mp->c1, l0); t_free(&l0);
  t4 l2 = run_c2f(&mp->f2, l1); t_free(&l1);
  t4 l3 = run_conv(&mp->c3, l2); t_free(&l2);
  t4 l4 = run_c2f(&mp->f4, l3); t_free(&l3);
  t4 l5 = run_conv(&mp->c5, l4);
  t4 l6 = run_c2f(&mp->f6, l5); t_free(&l5);
  t4 l7 = run_conv(&mp->c7, l6);
  t4 l8 = run_c2f(&mp->f8, l7); t_free(&l7);
  t4 l9 = run_sppf(&mp->s9, l8); t_free(&l8);
  t4 l10 = upsample2(l9);
  t4 pair[2] = {l10, l6};
  t4 l11 = cat(pair, 2); t_free(&l10); t_free(&l6);
  t4 l12 = run_c2f(&mp->f12, l11); t_free(&l11);
  t4 l13 = upsample2(l12);
  pair[0] = l13; pair[1] = l4;
  t4 l14 = cat(pair, 2); t_free(&l13); t_free(&l4);
  t4 l15 = run_c2f(&mp->f15, l14); t_free(&l14);
  t4 l16 = run_conv(&mp->c16, l15);
  pair[0] = l16; pair[1] = l12;
  t4 l17 = cat(pair, 2); t_free(&l16); t_free(&l12);
  t4 l18 = run_c2f(&mp->f18, l17); t_free(&l17);
  t4 l19 = run_conv(&mp->c19, l18);
  pair[0] = l19; pair[1] = l9;
  t4 l20 = cat(pair, 2); t_free(&l19); t_free(&l9);
  t4 l21 = run_c2f(&mp->f21, l20); t_free(&l20);
  t4 feats[3] = {l15, l18, l21};
  const float strides[3] = {8.f, 16.f, 32.f};
  int start = 0;
  for (int i = 0; i < 3; ++i) {
    t4 a = run_conv(&mp->box[i][0], feats[i]);
    t4 b = run_conv(&mp->box[i][1], a); t_free(&a);
    t4 box = run_conv(&mp->box[i][2], b); t_free(&b);
    a = run_conv(&mp->cls[i][0], feats[i]);
    b = run_conv(&mp->cls[i][1], a); t_free(&a);
    t4 cls = run_conv(&mp->cls[i][2], b); t_free(&b);
    if (g_fast_mode)
      cf_detect_decode(box.d, cls.d, batch, mp->nc, box.h, box.w, mp->reg_max, strides[i], 0, det, anchors, start);
    else
      or_detect_decode(box.d, cls.d, batch, mp->nc, box.h, box.w, mp->reg_max, strides[i], 0, det, anchors, start);
    start += box.h * box.w;
    t_free(&box);
    t_free(&cls);
  }
  if (nm) {
    widen_head(det, out, batch, mp->nc, nm, anchors);
    free(det);
    run_seg(&mp->seg, feats, mp->nc, out, anchors, proto_out);
  }
  for (int i = 0; i < 3; ++i) t_free(&feats[i]);
  return 0;
}

/* ------------------------------------------------- YOLO11 detect network */

/* Bottleneck(c1, c2, shortcut, k=(3,3), e): cv1 3x3 -> c2*e, cv2 3x3 -> c2,
 * plus x when shortcut and c1 == c2 (PtModel.cs:302-303). */
typedef struct {
  conv_t cv1, cv2;
  int add;
} bneck_t;

static bneck_t load_bneck(cursor_t* cur, int c1, int c2, int shortcut, double e) {
  bneck_t b;
  int c_ = (int)(c2 * e);
  b.cv1 = load_conv(cur, c1, c_, 3, 1);
  b.cv2 = load_conv(cur, c_, c2, 3, 1);
  b.add = shortcut && c1 == c2;
  return b;
}

static t4 run_bneck(const bneck_t* b, t4 x) {
  t4 a = run_conv(&b->cv1, x);
  t4 y = run_conv(&b->cv2, a);
  t_free(&a);
  if (b->add) add_into(&y, x);
  return y;
}

static void free_bneck(bneck_t* b) {
  free_conv(&b->cv1);
  free_conv(&b->cv2);
}

/* C3k (a C3): cv3(cat(m(cv1(x)), cv2(x))), m = n Bottlenecks(c_, c_, e=1)
 * (PtModel.cs:312). */
typedef struct {
  conv_t cv1, cv2, cv3;
  bneck_t m[4];
  int n;
} c3k_t;

static c3k_t load_c3k(cursor_t* cur, int c1, int c2, int n, int shortcut) {
  c3k_t m;
  memset(&m, 0, sizeof m);
  int c_ = (int)(c2 * 0.5);
  m.n = n;
  m.cv1 = load_conv(cur, c1, c_, 1, 1);
  m.cv2 = load_conv(cur, c1, c_, 1, 1);
  m.cv3 = load_conv(cur, 2 * c_, c2, 1, 1);
  for (int i = 0; i < n; ++i) m.m[i] = load_bneck(cur, c_, c_, shortcut, 1.0);
  return m;
}

static t4 run_c3k(const c3k_t* m, t4 x) {
  t4 a = run_conv(&m->cv1, x);
  for (int i = 0; i < m->n; ++i) {
    t4 t = run_bneck(&m->m[i], a);
    t_free(&a);
    a = t;
  }
  t4 b = run_conv(&m->cv2, x);
  t4 pair[2] = {a, b};
  t4 j = cat(pair, 2);
  t_free(&a);
  t_free(&b);
  t4 y = run_conv(&m->cv3, j);
  t_free(&j);
  return y;
}

static void free_c3k(c3k_t* m) {
  free_conv(&m->cv1);
  free_conv(&m->cv2);
  free_conv(&m->cv3);
  for (int i = 0; i < m->n; ++i) free_bneck(&m->m[i]);
}

/* C3k2 (C2f semantics, PtModel.cs:307): inner blocks are C3k(c, c, 2) when
 * c3k, else Bottleneck(c, c, e=0.5); shortcut is on. */
typedef struct {
  conv_t cv1, cv2;
  int n, c, c3k;
  bneck_t b[4];
  c3k_t k[4];
} c3k2_t;

static c3k2_t load_c3k2(cursor_t* cur, int c1, int c2, int n, int c3k, double e) {
  c3k2_t m;
  memset(&m, 0, sizeof m);
  m.n = n;
  m.c = (int)(c2 * e);
  m.c3k = c3k;
  m.cv1 = load_conv(cur, c1, 2 * m.c, 1, 1);
  m.cv2 = load_conv(cur, (2 + n) * m.c, c2, 1, 1);
  for (int i = 0; i < n; ++i) {
    if (c3k) m.k[i] = load_c3k(cur, m.c, m.c, 2, 1);
    else m.b[i] = load_bneck(cur, m.c, m.c, 1, 0.5);
  }
  return m;
}

static t4 run_c3k2(const c3k2_t* m, t4 x) {
  t4 y = run_conv(&m->cv1, x);
  t4 ys[8];
  ys[0] = channel_slice(y, 0, m->c);
  ys[1] = channel_slice(y, m->c, m->c);
  t_free(&y);
  for (int i = 0; i < m->n; ++i) ys[i + 2] = m->c3k ? run_c3k(&m->k[i], ys[i + 1]) : run_bneck(&m->b[i], ys[i + 1]);
  t4 j = cat(ys, m->n + 2);
  for (int i = 0; i < m->n + 2; ++i) t_free(&ys[i]);
  t4 out = run_conv(&m->cv2, j);
  t_free(&j);
  return out;
}

static void free_c3k2(c3k2_t* m) {
  free_conv(&m->cv1);
  free_conv(&m->cv2);
  for (int i = 0; i < m->n; ++i) {
    if (m->c3k) free_c3k(&m->k[i]);
    else free_bneck(&m->b[i]);
  }
}

/* Attention (PtModel.cs:429-437): qkv 1x1 (no act) viewed as
 * [B, heads, 2*kd + hd, N]; S = q^T k * scale, softmax over the last axis,
 * o = v S^T reshaped to [B, C, H, W], then proj(o + pe(v)) with pe a
 * depthwise 3x3 (no act).  Products and softmax in double. */
typedef struct {
  conv_t qkv, proj, pe;
  int heads, kd, hd;
  float scale;
} attn_t;

static attn_t load_attn(cursor_t* cur, int dim, int heads, double attn_ratio) {
  attn_t a;
  a.heads = heads;
  a.hd = dim / heads;
  a.kd = (int)(a.hd * attn_ratio);
  a.scale = 1.0f / sqrtf((float)a.kd);
  int h = dim + 2 * a.kd * heads;
  a.qkv = load_conv_ga(cur, dim, h, 1, 1, 1, 0);
  a.proj = load_conv_ga(cur, dim, dim, 1, 1, 1, 0);
  a.pe = load_conv_ga(cur, dim, dim, 3, 1, dim, 0);
  return a;
}

static t4 run_attn(const attn_t* a, t4 x) {
  const int N = x.h * x.w, per = 2 * a->kd + a->hd, C = a->heads * a->hd;
  t4 qkv = run_conv(&a->qkv, x);
  t4 o = t_new(x.n, C, x.h, x.w), vt = t_new(x.n, C, x.h, x.w);
  double* S = (double*)malloc(sizeof(double) * (size_t)N * N);
  for (int b = 0; b < x.n; ++b)
    for (int hh = 0; hh < a->heads; ++hh) {
      const float* base = qkv.d + ((size_t)b * qkv.c + (size_t)hh * per) * N;
      const float *q = base, *k = base + (size_t)a->kd * N, *v = base + (size_t)2 * a->kd * N;
#pragma omp parallel for schedule(static)
      for (int i = 0; i < N; ++i) {
        double mx = -INFINITY;
        for (int j = 0; j < N; ++j) {
          double s = 0;
          for (int d = 0; d < a->kd; ++d) s += (double)q[(size_t)d * N + i] * k[(size_t)d * N + j];
          s *= (double)a->scale;
          S[(size_t)i * N + j] = s;
          if (s > mx) mx = s;
        }
        double sum = 0;
        for (int j = 0; j < N; ++j) {
          double e = exp(S[(size_t)i * N + j] - mx);
          S[(size_t)i * N + j] = e;
          sum += e;
        }
        for (int j = 0; j < N; ++j) S[(size_t)i * N + j] /= sum;
      }
      float* od = o.d + ((size_t)b * C + (size_t)hh * a->hd) * N;
      float* vd = vt.d + ((size_t)b * C + (size_t)hh * a->hd) * N;
#pragma omp parallel for schedule(static)
      for (int d = 0; d < a->hd; ++d)
        for (int i = 0; i < N; ++i) {
          double s = 0;
          for (int j = 0; j < N; ++j) s += (double)v[(size_t)d * N + j] * S[(size_t)i * N + j];
          od[(size_t)d * N + i] = (float)s;
        }
      memcpy(vd, v, sizeof(float) * (size_t)a->hd * N);
    }
  free(S);
  t_free(&qkv);
  t4 pe = run_conv(&a->pe, vt);
  t_free(&vt);
  add_into(&pe, o); /* Add(attended, pe(v)) */
  t_free(&o);
  t4 y = run_conv(&a->proj, pe);
  t_free(&pe);
  return y;
}

static void free_attn(attn_t* a) {
  free_conv(&a->qkv);
  free_conv(&a->proj);
  free_conv(&a->pe);
}

/* PSABlock (PtModel.cs:341): x = x + attn(x); x = x + ffn(x),
 * ffn = Conv(c, 2c, 1) then Conv(2c, c, 1, act=False). */
typedef struct {
  attn_t attn;
  conv_t f0, f1;
} psa_t;

static psa_t load_psa(cursor_t* cur, int c, int heads) {
  psa_t p;
  p.attn = load_attn(cur, c, heads, 0.5);
  p.f0 = load_conv(cur, c, 2 * c, 1, 1);
  p.f1 = load_conv_ga(cur, 2 * c, c, 1, 1, 1, 0);
  return p;
}

static t4 run_psa(const psa_t* p, t4 x) {
  t4 a = run_attn(&p->attn, x);
  add_into(&a, x); /* x + attn(x) */
  t4 f = run_conv(&p->f0, a);
  t4 g = run_conv(&p->f1, f);
  t_free(&f);
  add_into(&g, a); /* x + ffn(x) */
  t_free(&a);
  return g;
}

/* C2PSA (PtModel.cs:339): a, b = chunk(cv1(x)); b = m(b); cv2(cat(a, b)). */
typedef struct {
  conv_t cv1, cv2;
  psa_t m[4];
  int n, c;
} c2psa_t;

static c2psa_t load_c2psa(cursor_t* cur, int c1, int n) {
  c2psa_t m;
  memset(&m, 0, sizeof m);
  m.n = n;
  m.c = (int)(c1 * 0.5);
  m.cv1 = load_conv(cur, c1, 2 * m.c, 1, 1);
  m.cv2 = load_conv(cur, 2 * m.c, c1, 1, 1);
  for (int i = 0; i < n; ++i) m.m[i] = load_psa(cur, m.c, m.c / 64);
  return m;
}

static t4 run_c2psa(const c2psa_t* m, t4 x) {
  t4 y = run_conv(&m->cv1, x);
  t4 a = channel_slice(y, 0, m->c), b = channel_slice(y, m->c, m->c);
  t_free(&y);
  for (int i = 0; i < m->n; ++i) {
    t4 t = run_psa(&m->m[i], b);
    t_free(&b);
    b = t;
  }
  t4 pair[2] = {a, b};
  t4 j = cat(pair, 2);
  t_free(&a);
  t_free(&b);
  t4 out = run_conv(&m->cv2, j);
  t_free(&j);
  return out;
}

static void free_c2psa(c2psa_t* m) {
  free_conv(&m->cv1);
  free_conv(&m->cv2);
  for (int i = 0; i < m->n; ++i) {
    free_attn(&m->m[i].attn);
    free_conv(&m->m[i].f0);
    free_conv(&m->m[i].f1);
  }
}

typedef struct {
  conv_t c0, c1, c3, c5, c7, c17, c20;
  c3k2_t f2, f4, f6, f8, f13, f16, f19, f22;
  sppf_t s9;
  c2psa_t p10;
  conv_t box[3][3];
  conv_t cls[3][5]; /* DWConv, Conv 1x1, DWConv, Conv 1x1, Conv2d */
  int ch[3], nc, reg_max;
  seg_t seg;
} yolo11_t;

static void load_yolo11(cursor_t* cur, const or_yolo_cfg* cfg, yolo11_t* m) {
  memset(m, 0, sizeof *m);
  int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
      c1024 = scale_ch(cfg, 1024);
  int n2 = scale_n(cfg, 2);
  /* ultralytics parse_model: the m/l/x scales (width >= 1) set c3k on every C3k2. */
  int k = cfg->width >= 1.0 ? 1 : 0;
  m->c0 = load_conv(cur, 3, c64, 3, 2);
  m->c1 = load_conv(cur, c64, c128, 3, 2);
  m->f2 = load_c3k2(cur, c128, c256, n2, k, 0.25);
  m->c3 = load_conv(cur, c256, c256, 3, 2);
  m->f4 = load_c3k2(cur, c256, c512, n2, k, 0.25);
  m->c5 = load_conv(cur, c512, c512, 3, 2);
  m->f6 = load_c3k2(cur, c512, c512, n2, 1, 0.5);
  m->c7 = load_conv(cur, c512, c1024, 3, 2);
  m->f8 = load_c3k2(cur, c1024, c1024, n2, 1, 0.5);
  m->s9.cv1 = load_conv(cur, c1024, c1024 / 2, 1, 1);
  m->s9.cv2 = load_conv(cur, c1024 / 2 * 4, c1024, 1, 1);
  m->p10 = load_c2psa(cur, c1024, n2);
  m->f13 = load_c3k2(cur, c1024 + c512, c512, n2, k, 0.5);
  m->f16 = load_c3k2(cur, c512 + c512, c256, n2, k, 0.5);
  m->c17 = load_conv(cur, c256, c256, 3, 2);
  m->f19 = load_c3k2(cur, c256 + c512, c512, n2, k, 0.5);
  m->c20 = load_conv(cur, c512, c512, 3, 2);
  m->f22 = load_c3k2(cur, c512 + c1024, c1024, n2, 1, 0.5);
  m->ch[0] = c256; m->ch[1] = c512; m->ch[2] = c1024;
  m->nc = cfg->nc;
  m->reg_max = cfg->reg_max;
  int c2 = 16;
  if (c256 / 4 > c2) c2 = c256 / 4;
  if (4 * cfg->reg_max > c2) c2 = 4 * cfg->reg_max;
  int c3 = cfg->nc < 100 ? cfg->nc : 100;
  if (c256 > c3) c3 = c256;
  for (int i = 0; i < 3; ++i) {
    m->box[i][0] = load_conv(cur, m->ch[i], c2, 3, 1);
    m->box[i][1] = load_conv(cur, c2, c2, 3, 1);
    m->box[i][2] = load_conv2d(cur, c2, 4 * cfg->reg_max, K_BIAS_BOX);
  }
  for (int i = 0; i < 3; ++i) {
    m->cls[i][0] = load_conv_ga(cur, m->ch[i], m->ch[i], 3, 1, m->ch[i], 1);
    m->cls[i][1] = load_conv(cur, m->ch[i], c3, 1, 1);
    m->cls[i][2] = load_conv_ga(cur, c3, c3, 3, 1, c3, 1);
    m->cls[i][3] = load_conv(cur, c3, c3, 1, 1);
    m->cls[i][4] = load_conv2d(cur, c3, cfg->nc, K_BIAS_CLS);
  }
  if (cfg->nm > 0) load_seg(cur, cfg, m->ch, scale_ch(cfg, cfg->npr), &m->seg);
}

static void free_yolo11(yolo11_t* m) {
  conv_t* cs[] = {&m->c0, &m->c1, &m->c3, &m->c5, &m->c7, &m->c17, &m->c20, &m->s9.cv1, &m->s9.cv2};
  for (size_t i = 0; i < sizeof cs / sizeof cs[0]; ++i) free_conv(cs[i]);
  c3k2_t* fs[] = {&m->f2, &m->f4, &m->f6, &m->f8, &m->f13, &m->f16, &m->f19, &m->f22};
  for (size_t i = 0; i < sizeof fs / sizeof fs[0]; ++i) free_c3k2(fs[i]);
  free_c2psa(&m->p10);
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 3; ++j) free_conv(&m->box[i][j]);
    for (int j = 0; j < 5; ++j) free_conv(&m->cls[i][j]);
  }
  free_seg(&m->seg);
}

int or_yolo11_layout(const or_yolo_cfg* cfg, int* out, int max_tensors) {
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.layout = out;
  cur.max_tensors = max_tensors;
  cur.eps = cfg->bn_eps;
  yolo11_t* m = (yolo11_t*)malloc(sizeof(yolo11_t));
  load_yolo11(&cur, cfg, m);
  free_yolo11(m);
  free(m);
  return cur.count;
}

int or_yolo11_forward(const or_yolo_cfg* cfg, const float* params, size_t n_params, const float* input, int batch,
                      int h, int w, float* out, size_t out_capacity, float* proto_out) {
  if (h % 32 || w % 32 || batch <= 0) return 1;
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.params = params;
  cur.n_params = n_params;
  cur.eps = cfg->bn_eps;
  yolo11_t* m = (yolo11_t*)malloc(sizeof(yolo11_t));
  load_yolo11(&cur, cfg, m);
  if (cur.fail || cur.pos != n_params) {
    free_yolo11(m);
    free(m);
    return 2;
  }
  const int anchors = (h / 8) * (w / 8) + (h / 16) * (w / 16) + (h / 32) * (w / 32);
  const int nm = cfg->nm > 0 ? cfg->nm : 0;
  if ((size_t)batch * (m->nc + 4 + nm) * anchors > out_capacity) {
    free_yolo11(m);
    free(m);
    return 3;
  }
  float* det = nm ? (float*)malloc(sizeof(float) * (size_t)batch * (m->nc + 4) * anchors) : out;
  t4 x = {batch, 3, h, w, (float*)input};
  t4 l0 = run_conv(&m->c0, x);
  t4 l1 = run_conv(&m->c1, l0); t_free(&l0);
  t4 l2 = run_c3k2(&m->f2, l1); t_free(&l1);
  t4 l3 = run_conv(&m->c3, l2); t_free(&l2);
  t4 l4 = run_c3k2(&m->f4, l3); t_free(&l3);
  t4 l5 = run_conv(&m->c5, l4);
  t4 l6 = run_c3k2(&m->f6, l5); t_free(&l5);
  t4 l7 = run_conv(&m->c7, l6);
  t4 l8 = run_c3k2(&m->f8, l7); t_free(&l7);
  t4 l9 = run_sppf(&m->s9, l8); t_free(&l8);
  t4 l10 = run_c2psa(&m->p10, l9); t_free(&l9);
  t4 l11 = upsample2(l10);
  t4 pair[2] = {l11, l6};
  t4 l12 = cat(pair, 2); t_free(&l11); t_free(&l6);
  t4 l13 = run_c3k2(&m->f13, l12); t_free(&l12);
  t4 l14 = upsample2(l13);
  pair[0] = l14; pair[1] = l4;
  t4 l15 = cat(pair, 2); t_free(&l14); t_free(&l4);
  t4 l16 = run_c3k2(&m->f16, l15); t_free(&l15);
  t4 l17 = run_conv(&m->c17, l16);
  pair[0] = l17; pair[1] = l13;
  t4 l18 = cat(pair, 2); t_free(&l17); t_free(&l13);
  t4 l19 = run_c3k2(&m->f19, l18); t_free(&l18);
  t4 l20 = run_conv(&m->c20, l19);
  pair[0] = l20; pair[1] = l10;
  t4 l21 = cat(pair, 2); t_free(&l20); t_free(&l10);
  t4 l22 = run_c3k2(&m->f22, l21); t_free(&l21);
  t4 feats[3] = {l16, l19, l22};
  const float strides[3] = {8.f, 16.f, 32.f};
  int start = 0;
  for (int i = 0; i < 3; ++i) {
    t4 a = run_conv(&m->box[i][0], feats[i]);
    t4 b = run_conv(&m->box[i][1], a); t_free(&a);
    t4 box = run_conv(&m->box[i][2], b); t_free(&b);
    t4 c = feats[i];
    t4 cls = {0, 0, 0, 0, NULL};
    for (int j = 0; j < 5; ++j) {
      t4 nx = run_conv(&m->cls[i][j], c);
      if (j > 0) t_free(&c);
      c = nx;
    }
    cls = c;
    or_detect_decode(box.d, cls.d, batch, m->nc, box.h, box.w, m->reg_max, strides[i], 0, det, anchors, start);
    start += box.h * box.w;
    t_free(&box);
    t_free(&cls);
  }
  if (nm) {
    widen_head(det, out, batch, m->nc, nm, anchors);
    free(det);
    run_seg(&m->seg, feats, m->nc, out, anchors, proto_out);
  }
  for (int i = 0; i < 3; ++i) t_free(&feats[i]);
  free_yolo11(m);
  free(m);
  return 0;
}

/* ------------------------------------------------- YOLO26 (end-to-end) */

/* C3k2 with attn (the last head block of yolo26.yaml,
 * `C3k2, [1024, True, 0.5, True]`): the C2f walk of PtModel.cs:307 whose
 * inner blocks are Sequential(Bottleneck(c, c, e=0.5), PSABlock(c,
 * attn_ratio 0.5, heads max(c / 64, 1))) (PtModel.cs:302-303, 341). */
typedef struct {
  conv_t cv1, cv2;
  int n, c;
  bneck_t b[4];
  psa_t p[4];
} c3k2a_t;

static c3k2a_t load_c3k2a(cursor_t* cur, int c1, int c2, int n, double e) {
  c3k2a_t m;
  memset(&m, 0, sizeof m);
  m.n = n;
  m.c = (int)(c2 * e);
  m.cv1 = load_conv(cur, c1, 2 * m.c, 1, 1);
  m.cv2 = load_conv(cur, (2 + n) * m.c, c2, 1, 1);
  for (int i = 0; i < n; ++i) {
    m.b[i] = load_bneck(cur, m.c, m.c, 1, 0.5);
    m.p[i] = load_psa(cur, m.c, m.c / 64 > 1 ? m.c / 64 : 1);
  }
  return m;
}

static t4 run_c3k2a(const c3k2a_t* m, t4 x) {
  t4 y = run_conv(&m->cv1, x);
  t4 ys[8];
  ys[0] = channel_slice(y, 0, m->c);
  ys[1] = channel_slice(y, m->c, m->c);
  t_free(&y);
  for (int i = 0; i < m->n; ++i) {
    t4 t = run_bneck(&m->b[i], ys[i + 1]);
    ys[i + 2] = run_psa(&m->p[i], t);
    t_free(&t);
  }
  t4 j = cat(ys, m->n + 2);
  for (int i = 0; i < m->n + 2; ++i) t_free(&ys[i]);
  t4 out = run_conv(&m->cv2, j);
  t_free(&j);
  return out;
}

static void free_c3k2a(c3k2a_t* m) {
  free_conv(&m->cv1);
  free_conv(&m->cv2);
  for (int i = 0; i < m->n; ++i) {
    free_bneck(&m->b[i]);
    free_attn(&m->p[i].attn);
    free_conv(&m->p[i].f0);
    free_conv(&m->p[i].f1);
  }
}

/* Segment26 (PtModel.cs:353-359) with Proto26 (:345-352): the prototypes
 * come from the P3 feature refined by the coarser levels,
 *   r = f0 + up2(feat_refine0(f1)) + up4(feat_refine1(f2))   (nearest),
 * then feat_fuse (3x3), Proto's cv1 (3x3), ConvTranspose2d 2x2 s2, cv2
 * (3x3), cv3 (1x1 to nm).  feat_refine[i] = Conv(ch[i+1], ch0, 1),
 * feat_fuse = Conv(ch0, c_, 3).  Mask coefficients per level from
 * one2one_cv4 = Conv(x, c4, 3), Conv(c4, c4, 3), Conv2d(c4, nm) with
 * c4 = max(ch0 / 4, nm).  Parameter order: Proto's cv1, upsample, cv2, cv3,
 * then feat_refine, feat_fuse, then one2one_cv4 (the training-only semseg
 * branch and the one-to-many cv2/cv3/cv4 copies are not consumed). */
typedef struct {
  proto_t proto;
  conv_t refine[2], fuse;
  conv_t cv4[3][3];
  int nm;
} seg26_t;

static void load_seg26(cursor_t* cur, const or_yolo_cfg* cfg, const int ch[3], int c_, seg26_t* s) {
  memset(s, 0, sizeof *s);
  s->nm = cfg->nm;
  s->proto.cv1 = load_conv(cur, c_, c_, 3, 1);
  s->proto.up = load_deconv2(cur, c_, c_);
  s->proto.cv2 = load_conv(cur, c_, c_, 3, 1);
  s->proto.cv3 = load_conv(cur, c_, cfg->nm, 1, 1);
  s->refine[0] = load_conv(cur, ch[1], ch[0], 1, 1);
  s->refine[1] = load_conv(cur, ch[2], ch[0], 1, 1);
  s->fuse = load_conv(cur, ch[0], c_, 3, 1);
  const int c4 = ch[0] / 4 > cfg->nm ? ch[0] / 4 : cfg->nm;
  for (int i = 0; i < 3; ++i) {
    s->cv4[i][0] = load_conv(cur, ch[i], c4, 3, 1);
    s->cv4[i][1] = load_conv(cur, c4, c4, 3, 1);
    s->cv4[i][2] = load_conv2d(cur, c4, cfg->nm, K_BIAS);
  }
}

static void free_seg26(seg26_t* s) {
  free_conv(&s->proto.cv1);
  free_conv(&s->proto.cv2);
  free_conv(&s->proto.cv3);
  free(s->proto.up.w);
  free(s->proto.up.b);
  free_conv(&s->refine[0]);
  free_conv(&s->refine[1]);
  free_conv(&s->fuse);
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) free_conv(&s->cv4[i][j]);
}

static void run_seg26(const seg26_t* s, const t4 feats[3], int nc, float* head, int anchors, float* proto_out) {
  t4 r = t_new(feats[0].n, feats[0].c, feats[0].h, feats[0].w);
  memcpy(r.d, feats[0].d, sizeof(float) * (size_t)r.n * r.c * r.h * r.w);
  for (int i = 0; i < 2; ++i) {
    t4 hi = run_conv(&s->refine[i], feats[i + 1]);
    t4 up = t_new(hi.n, hi.c, r.h, r.w);
    or_resize_nearest(hi.d, hi.n, hi.c, hi.h, hi.w, r.h, r.w, up.d);
    t_free(&hi);
    add_into(&r, up); /* Add(refined, ResizeNearest(higher)) */
    t_free(&up);
  }
  t4 f = run_conv(&s->fuse, r); t_free(&r);
  t4 a = run_conv(&s->proto.cv1, f); t_free(&f);
  t4 u = t_new(a.n, s->proto.up.oc, 2 * a.h, 2 * a.w);
  or_conv_transpose2x2(a.d, a.n, a.c, a.h, a.w, s->proto.up.w, s->proto.up.b, s->proto.up.oc, u.d);
  t_free(&a);
  t4 b = run_conv(&s->proto.cv2, u); t_free(&u);
  t4 p = run_conv(&s->proto.cv3, b); t_free(&b);
  if (proto_out) memcpy(proto_out, p.d, sizeof(float) * (size_t)p.n * p.c * p.h * p.w);
  t_free(&p);
  const int C = nc + 4 + s->nm;
  int start = 0;
  for (int i = 0; i < 3; ++i) {
    t4 x0 = run_conv(&s->cv4[i][0], feats[i]);
    t4 x1 = run_conv(&s->cv4[i][1], x0); t_free(&x0);
    t4 mc = run_conv(&s->cv4[i][2], x1); t_free(&x1);
    const int hw = mc.h * mc.w;
    for (int bb = 0; bb < mc.n; ++bb)
      for (int j = 0; j < s->nm; ++j)
        memcpy(head + ((size_t)bb * C + nc + 4 + j) * anchors + start, mc.d + ((size_t)bb * s->nm + j) * hw,
               sizeof(float) * hw);
    start += hw;
    t_free(&mc);
  }
}

/* ultralytics yolo26.yaml / yolo26-seg.yaml, restated: the YOLO11 backbone
 * (Conv, C3k2, C2PSA) with SPPF(c, c, 5, n=3, shortcut) whose cv1 has no
 * activation and whose output adds its input; head C3k2 blocks with C3k
 * inner blocks and the last one (layer 22) with attention blocks; the
 * end-to-end Detect (one2one_cv2 / one2one_cv3, PtModel.cs:449-450) with
 * reg_max 1, so boxes are direct distances decoded to x1 y1 x2 y2
 * (CpuHead.cs:57-124 with bins 1, xyxy); Segment26 when nm > 0.  The output
 * is the head before the end-to-end selection, [B, nc+4(+nm), A]. */
typedef struct {
  conv_t c0, c1, c3, c5, c7, c17, c20;
  c3k2_t f2, f4, f6, f8, f13, f16, f19;
  c3k2a_t f22;
  sppf_t s9;
  c2psa_t p10;
  conv_t box[3][3];
  conv_t cls[3][5];
  int ch[3], nc, reg_max;
  seg26_t seg;
} yolo26_t;

static void load_yolo26(cursor_t* cur, const or_yolo_cfg* cfg, yolo26_t* m) {
  memset(m, 0, sizeof *m);
  int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
      c1024 = scale_ch(cfg, 1024);
  int n2 = scale_n(cfg, 2);
  int k = cfg->width >= 1.0 ? 1 : 0;
  m->c0 = load_conv(cur, 3, c64, 3, 2);
  m->c1 = load_conv(cur, c64, c128, 3, 2);
  m->f2 = load_c3k2(cur, c128, c256, n2, k, 0.25);
  m->c3 = load_conv(cur, c256, c256, 3, 2);
  m->f4 = load_c3k2(cur, c256, c512, n2, k, 0.25);
  m->c5 = load_conv(cur, c512, c512, 3, 2);
  m->f6 = load_c3k2(cur, c512, c512, n2, 1, 0.5);
  m->c7 = load_conv(cur, c512, c1024, 3, 2);
  m->f8 = load_c3k2(cur, c1024, c1024, n2, 1, 0.5);
  m->s9.cv1 = load_conv_ga(cur, c1024, c1024 / 2, 1, 1, 1, 0);
  m->s9.cv2 = load_conv(cur, c1024 / 2 * 4, c1024, 1, 1);
  m->p10 = load_c2psa(cur, c1024, n2);
  m->f13 = load_c3k2(cur, c1024 + c512, c512, n2, 1, 0.5);
  m->f16 = load_c3k2(cur, c512 + c512, c256, n2, 1, 0.5);
  m->c17 = load_conv(cur, c256, c256, 3, 2);
  m->f19 = load_c3k2(cur, c256 + c512, c512, n2, 1, 0.5);
  m->c20 = load_conv(cur, c512, c512, 3, 2);
  m->f22 = load_c3k2a(cur, c512 + c1024, c1024, scale_n(cfg, 1), 0.5);
  m->ch[0] = c256; m->ch[1] = c512; m->ch[2] = c1024;
  m->nc = cfg->nc;
  m->reg_max = cfg->reg_max;
  int c2 = 16;
  if (c256 / 4 > c2) c2 = c256 / 4;
  if (4 * cfg->reg_max > c2) c2 = 4 * cfg->reg_max;
  int c3 = cfg->nc < 100 ? cfg->nc : 100;
  if (c256 > c3) c3 = c256;
  for (int i = 0; i < 3; ++i) {
    m->box[i][0] = load_conv(cur, m->ch[i], c2, 3, 1);
    m->box[i][1] = load_conv(cur, c2, c2, 3, 1);
    m->box[i][2] = load_conv2d(cur, c2, 4 * cfg->reg_max, K_BIAS_BOX);
  }
  for (int i = 0; i < 3; ++i) {
    m->cls[i][0] = load_conv_ga(cur, m->ch[i], m->ch[i], 3, 1, m->ch[i], 1);
    m->cls[i][1] = load_conv(cur, m->ch[i], c3, 1, 1);
    m->cls[i][2] = load_conv_ga(cur, c3, c3, 3, 1, c3, 1);
    m->cls[i][3] = load_conv(cur, c3, c3, 1, 1);
    m->cls[i][4] = load_conv2d(cur, c3, cfg->nc, K_BIAS_CLS);
  }
  if (cfg->nm > 0) load_seg26(cur, cfg, m->ch, scale_ch(cfg, cfg->npr), &m->seg);
}

static void free_yolo26(yolo26_t* m) {
  conv_t* cs[] = {&m->c0, &m->c1, &m->c3, &m->c5, &m->c7, &m->c17, &m->c20, &m->s9.cv1, &m->s9.cv2};
  for (size_t i = 0; i < sizeof cs / sizeof cs[0]; ++i) free_conv(cs[i]);
  c3k2_t* fs[] = {&m->f2, &m->f4, &m->f6, &m->f8, &m->f13, &m->f16, &m->f19};
  for (size_t i = 0; i < sizeof fs / sizeof fs[0]; ++i) free_c3k2(fs[i]);
  free_c3k2a(&m->f22);
  free_c2psa(&m->p10);
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 3; ++j) free_conv(&m->box[i][j]);
    for (int j = 0; j < 5; ++j) free_conv(&m->cls[i][j]);
  }
  free_seg26(&m->seg);
}

int or_yolo26_layout(const or_yolo_cfg* cfg, int* out, int max_tensors) {
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.layout = out;
  cur.max_tensors = max_tensors;
  cur.eps = cfg->bn_eps;
  yolo26_t* m = (yolo26_t*)malloc(sizeof(yolo26_t));
  load_yolo26(&cur, cfg, m);
  free_yolo26(m);
  free(m);
  return cur.count;
}

int or_yolo26_forward(const or_yolo_cfg* cfg, const float* params, size_t n_params, const float* input, int batch,
                      int h, int w, float* out, size_t out_capacity, float* proto_out) {
  if (h % 32 || w % 32 || batch <= 0) return 1;
  cursor_t cur;
  memset(&cur, 0, sizeof cur);
  cur.params = params;
  cur.n_params = n_params;
  cur.eps = cfg->bn_eps;
  yolo26_t* m = (yolo26_t*)malloc(sizeof(yolo26_t));
  load_yolo26(&cur, cfg, m);
  if (cur.fail || cur.pos != n_params) {
    free_yolo26(m);
    free(m);
    return 2;
  }
  const int anchors = (h / 8) * (w / 8) + (h / 16) * (w / 16) + (h / 32) * (w / 32);
  const int nm = cfg->nm > 0 ? cfg->nm : 0;
  if ((size_t)batch * (m->nc + 4 + nm) * anchors > out_capacity) {
    free_yolo26(m);
    free(m);
    return 3;
  }
  float* det = nm ? (float*)malloc(sizeof(float) * (size_t)batch * (m->nc + 4) * anchors) : out;
  t4 x = {batch, 3, h, w, (float*)input};
  t4 l0 = run_conv(&m->c0, x);
  t4 l1 = run_conv(&m->c1, l0); t_free(&l0);
  t4 l2 = run_c3k2(&m->f2, l1); t_free(&l1);
  t4 l3 = run_conv(&m->c3, l2); t_free(&l2);
  t4 l4 = run_c3k2(&m->f4, l3); t_free(&l3);
  t4 l5 = run_conv(&m->c5, l4);
  t4 l6 = run_c3k2(&m->f6, l5); t_free(&l5);
  t4 l7 = run_conv(&m->c7, l6);
  t4 l8 = run_c3k2(&m->f8, l7); t_free(&l7);
  t4 l9 = run_sppf(&m->s9, l8);
  add_into(&l9, l8); /* SPPF shortcut: Add(pooled, x) */
  t_free(&l8);
  t4 l10 = run_c2psa(&m->p10, l9); t_free(&l9);
  t4 l11 = upsample2(l10);
  t4 pair[2] = {l11, l6};
  t4 l12 = cat(pair, 2); t_free(&l11); t_free(&l6);
  t4 l13 = run_c3k2(&m->f13, l12); t_free(&l12);
  t4 l14 = upsample2(l13);
  pair[0] = l14; pair[1] = l4;
  t4 l15 = cat(pair, 2); t_free(&l14); t_free(&l4);
  t4 l16 = run_c3k2(&m->f16, l15); t_free(&l15);
  t4 l17 = run_conv(&m->c17, l16);
  pair[0] = l17; pair[1] = l13;
  t4 l18 = cat(pair, 2); t_free(&l17); t_free(&l13);
  t4 l19 = run_c3k2(&m->f19, l18); t_free(&l18);
  t4 l20 = run_conv(&m->c20, l19);
  pair[0] = l20; pair[1] = l10;
  t4 l21 = cat(pair, 2); t_free(&l20); t_free(&l10);
  t4 l22 = run_c3k2a(&m->f22, l21); t_free(&l21);
  t4 feats[3] = {l16, l19, l22};
  const float strides[3] = {8.f, 16.f, 32.f};
  int start = 0;
  for (int i = 0; i < 3; ++i) {
    t4 a = run_conv(&m->box[i][0], feats[i]);
    t4 b = run_conv(&m->box[i][1], a); t_free(&a);
    t4 box = run_conv(&m->box[i][2], b); t_free(&b);
    t4 c = feats[i];
    for (int j = 0; j < 5; ++j) {
      t4 nx = run_conv(&m->cls[i][j], c);
      if (j > 0) t_free(&c);
      c = nx;
    }
    or_detect_decode(box.d, c.d, batch, m->nc, box.h, box.w, m->reg_max, strides[i], 1, det, anchors, start);
    start += box.h * box.w;
    t_free(&box);
    t_free(&c);
  }
  if (nm) {
    widen_head(det, out, batch, m->nc, nm, anchors);
    free(det);
    run_seg26(&m->seg, feats, m->nc, out, anchors, proto_out);
  }
  for (int i = 0; i < 3; ++i) t_free(&feats[i]);
  free_yolo26(m);
  free(m);
  return 0;
}
