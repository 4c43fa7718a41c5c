// Host-side (CPU) pieces of the boundary: BN fold, letterbox and the
// detection decoder with greedy NMS.  They are the C++ counterparts of the
// reference's C# host code the HIP backend sits under.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <vector>

#include "sy_internal.h"

#pragma clang fp contract(off)

extern "C" {

// PtModel.Prepare BN fold (src/SimdYolo/PtModel.cs:135-143), in float exactly
// as the reference computes it (the fold result feeds every conv).
void sy_fold_bn(const float* w, int oc, int per_oc, const float* conv_bias, const float* gamma, const float* beta,
                const float* mean, const float* var, float eps, float* w_out, float* b_out) {
  for (int c = 0; c < oc; ++c) {
    const float scale = gamma[c] / std::sqrt(var[c] + eps);
    const float* src = w + (size_t)c * per_oc;
    float* dst = w_out + (size_t)c * per_oc;
    for (int j = 0; j < per_oc; ++j) dst[j] = src[j] * scale;
    b_out[c] = beta[c] + ((conv_bias ? conv_bias[c] : 0.0f) - mean[c]) * scale;
  }
}

// ImagePreprocessor.Letterbox (src/SimdYolo/YoloDetector.cs:448-507):
// bilinear resize with half-pixel centres, 114/255 padding, RGB planes, /255.
int sy_letterbox_rgb(const uint8_t* pixels, int width, int height, int tw, int th, int bgr, int row_stride,
                     float* out, sy_letterbox* t) {
  SY_CHECK(pixels && out && t, SY_EINVAL, "null argument");
  SY_CHECK(width > 0 && height > 0 && tw > 0 && th > 0, SY_EINVAL, "Image dimensions must be positive.");
  if (row_stride == 0) row_stride = width * 3;
  SY_CHECK(row_stride >= width * 3, SY_EINVAL, "Image buffer too short.");
  const float gain = std::min((float)tw / width, (float)th / height);
  // MathF.Round: half to even (std::nearbyint under the default mode).
  const int rw = std::clamp((int)std::nearbyint(width * gain), 1, tw);
  const int rh = std::clamp((int)std::nearbyint(height * gain), 1, th);
  const int px = (tw - rw) / 2, py = (th - rh) / 2;
  const size_t plane = (size_t)tw * th;
  std::fill(out, out + 3 * plane, 114.0f / 255.0f);
  std::vector<int> x0(rw), x1(rw);
  std::vector<float> fr(rw);
  for (int x = 0; x < rw; ++x) {
    const float sx = std::clamp((x + .5f) * width / rw - .5f, 0.0f, (float)(width - 1));
    const int left = (int)sx;
    x0[x] = left * 3;
    x1[x] = std::min(left + 1, width - 1) * 3;
    fr[x] = sx - left;
  }
  const int red = bgr ? 2 : 0, blue = 2 - red;
  for (int y = 0; y < rh; ++y) {
    const float sy = std::clamp((y + .5f) * height / rh - .5f, 0.0f, (float)(height - 1));
    const int y0 = (int)sy, y1 = std::min(y0 + 1, height - 1);
    const float fy = sy - y0, wy = 1 - fy;
    const uint8_t* top = pixels + (size_t)y0 * row_stride;
    const uint8_t* bottom = pixels + (size_t)y1 * row_stride;
    float* r = out + (size_t)(y + py) * tw + px;
    float* g = r + plane;
    float* b = g + plane;
    for (int x = 0; x < rw; ++x) {
      const float fx = fr[x], wx = 1 - fx;
      auto sample = [&](int o) {
        const float upper = top[x0[x] + o] * wx + top[x1[x] + o] * fx;
        const float lower = bottom[x0[x] + o] * wx + bottom[x1[x] + o] * fx;
        return (upper * wy + lower * fy) / 255.0f;
      };
      r[x] = sample(red);
      g[x] = sample(1);
      b[x] = sample(blue);
    }
  }
  *t = sy_letterbox{width, height, tw, th, (float)rw / width, (float)rh / height, px, py};
  return SY_OK;
}

static float iou(const sy_detection& a, const sy_detection& b) {
  const float w = std::max(0.0f, std::min(a.x + a.width, b.x + b.width) - std::max(a.x, b.x));
  const float h = std::max(0.0f, std::min(a.y + a.height, b.y + b.height) - std::max(a.y, b.y));
  const float inter = w * h;
  return inter / std::max(FLT_TRUE_MIN, a.width * a.height + b.width * b.height - inter);
}

// DetectionDecoder.DecodeIndexed (src/SimdYolo/YoloDetector.cs:539-643):
// layout inference, first-best class (strict >), finite + confidence filter,
// stable descending sort, class-aware greedy NMS with IoU > threshold,
// letterbox mapping and clamping.
int sy_decode_detections(const float* data, int dim1, int dim2, const sy_decode_options* o, const sy_letterbox* t,
                         sy_detection* out, int max_out, int* count) {
  SY_CHECK(data && o && t && count && (out || max_out == 0), SY_EINVAL, "null argument");
  *count = 0;
  SY_CHECK(t->source_width > 0 && t->source_height > 0 && t->target_width > 0 && t->target_height > 0 &&
               std::isfinite(t->scale_x) && std::isfinite(t->scale_y) && t->scale_x > 0 && t->scale_y > 0 &&
               o->max_detections > 0 && o->max_candidates > 0 && o->class_count >= 0,
           SY_EINVAL, "Invalid decode transform/options.");
  int layout = o->layout;
  if (layout == SY_OUTPUT_AUTO) {
    const int expected = o->class_count > 0 ? 4 + o->class_count : 0;
    if (expected > 0 && dim1 == expected && dim2 != expected) layout = SY_OUTPUT_CHANNELS_FIRST;
    else if (expected > 0 && dim2 == expected && dim1 != expected) layout = SY_OUTPUT_CHANNELS_LAST;
    else if (dim2 == 6 && dim1 != 6) layout = SY_OUTPUT_END_TO_END;
    else if (dim1 >= 5 && dim1 < dim2) layout = SY_OUTPUT_CHANNELS_FIRST;
    else if (dim2 >= 5 && dim2 < dim1) layout = SY_OUTPUT_CHANNELS_LAST;
    else {
      sy::set_error("Ambiguous YOLO output layout. Set OutputLayout explicitly.");
      return SY_EINVAL;
    }
  }
  const bool e2e = layout == SY_OUTPUT_END_TO_END, first = layout == SY_OUTPUT_CHANNELS_FIRST;
  const int n = first ? dim2 : dim1, fields = first ? dim1 : dim2;
  SY_CHECK(fields >= 5 && !(e2e && fields != 6), SY_EINVAL, "Invalid detection output.");
  const int class_fields = o->class_count > 0 ? 4 + o->class_count : fields;
  SY_CHECK(e2e || (class_fields >= 5 && class_fields <= fields), SY_EINVAL, "ClassCount does not match output.");
  auto at = [&](int a, int c) { return data[first ? (size_t)c * n + a : (size_t)a * fields + c]; };

  std::vector<sy_detection> cand;
  for (int a = 0; a < n; ++a) {
    int cls = 0;
    float conf;
    if (e2e) {
      conf = at(a, 4);
      const float cv = at(a, 5);
      if (!std::isfinite(cv) || cv < 0 || cv != std::trunc(cv)) continue;
      cls = (int)cv;
    } else {
      conf = -INFINITY;
      for (int c = 4; c < class_fields; ++c) {
        const float s = at(a, c);
        if (s > conf) {
          conf = s;
          cls = c - 4;
        }
      }
    }
    if (!std::isfinite(conf) || conf < o->confidence) continue;
    float x = at(a, 0), y = at(a, 1), w = at(a, 2), h = at(a, 3);
    if (!std::isfinite(x) || !std::isfinite(y) || !std::isfinite(w) || !std::isfinite(h)) continue;
    if (e2e) {
      w -= x;
      h -= y;
    } else {
      x -= w * .5f;
      y -= h * .5f;
    }
    if (w <= 0 || h <= 0) continue;
    cand.push_back(sy_detection{cls, conf, x, y, w, h, a});
  }
  std::stable_sort(cand.begin(), cand.end(),
                   [](const sy_detection& l, const sy_detection& r) { return l.confidence > r.confidence; });
  return sy::finish_detections(cand, e2e, o, t, out, max_out, count);
}

}  // extern "C"

// The part of DecodeIndexed after the candidates are sorted (by confidence,
// descending, ties in anchor order): truncation to max_candidates, greedy NMS
// and the letterbox mapping (src/SimdYolo/YoloDetector.cs:621-642).  Shared by
// the host decoder and the GPU candidate path.
int sy::finish_detections(std::vector<sy_detection>& cand, bool e2e, const sy_decode_options* o,
                          const sy_letterbox* t, sy_detection* out, int max_out, int* count) {
  *count = 0;
  if ((int)cand.size() > o->max_candidates) cand.resize(o->max_candidates);
  std::vector<sy_detection> kept;
  for (const auto& d : cand) {
    if (!e2e) {
      bool suppressed = false;
      for (const auto& k : kept)
        if ((o->agnostic || k.class_id == d.class_id) && iou(k, d) > o->iou) {
          suppressed = true;
          break;
        }
      if (suppressed) continue;
    }
    kept.push_back(d);
    if ((int)kept.size() >= o->max_detections) break;
  }
  int m = 0;
  for (auto d : kept) {
    const float x1 = std::clamp((d.x - t->pad_x) / t->scale_x, 0.0f, (float)t->source_width);
    const float y1 = std::clamp((d.y - t->pad_y) / t->scale_y, 0.0f, (float)t->source_height);
    const float x2 = std::clamp((d.x + d.width - t->pad_x) / t->scale_x, 0.0f, (float)t->source_width);
    const float y2 = std::clamp((d.y + d.height - t->pad_y) / t->scale_y, 0.0f, (float)t->source_height);
    d.x = x1;
    d.y = y1;
    d.width = x2 - x1;
    d.height = y2 - y1;
    if (!(d.width > 0 && d.height > 0)) continue;
    if (m < max_out) out[m] = d;
    ++m;
  }
  *count = m;
  SY_CHECK(m <= max_out, SY_EINVAL, "output buffer holds %d detections, %d decoded", max_out, m);
  return SY_OK;
}
