// Pre- and post-processing on the device, on either side of PredictRaw:
//   * the letterbox of a u8 RGB24/BGR24 image straight into the network's
//     NCHW float input (ImagePreprocessor.Letterbox,
//     src/SimdYolo/YoloDetector.cs:448-507), bit-identical to the host
//     restatement sy_letterbox_rgb (same float operations, no contraction);
//   * the candidate stage of DetectionDecoder.DecodeIndexed
//     (src/SimdYolo/YoloDetector.cs:557-621) for channels-first heads: per
//     anchor the first-best class, the finite/confidence/size filters, and
//     the stable descending sort: a per-anchor pass over the whole GPU, then
//     one sorting workgroup per image.  Greedy NMS and
//     the letterbox mapping stay on the host, as in the reference, and are
//     the same code as the host decoder's.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <vector>

#include "sy_internal.h"

namespace sy {

#pragma clang fp contract(off)

struct LetterboxArgs {
  const uint8_t* px;
  int width, height, row_stride, bgr;
  int tw, th, rw, rh, pad_x, pad_y;
  float* out;
};

// One thread per output pixel; the three planes are written together.
__global__ __launch_bounds__(256) void letterbox_kernel(const LetterboxArgs a) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long plane = (long long)a.tw * a.th;
  if (i >= plane) return;
  const int ox = (int)(i % a.tw), oy = (int)(i / a.tw);
  const int x = ox - a.pad_x, y = oy - a.pad_y;
  float r = 114.0f / 255.0f, g = r, b = r;
  if (x >= 0 && x < a.rw && y >= 0 && y < a.rh) {
    const float sxr = (x + .5f) * a.width / a.rw - .5f;
    const float sx = sxr < 0.0f ? 0.0f : (sxr > (float)(a.width - 1) ? (float)(a.width - 1) : sxr);
    const int left = (int)sx;
    const int x0 = left * 3, x1 = min(left + 1, a.width - 1) * 3;
    const float fx = sx - left, wx = 1 - fx;
    const float syr = (y + .5f) * a.height / a.rh - .5f;
    const float sy = syr < 0.0f ? 0.0f : (syr > (float)(a.height - 1) ? (float)(a.height - 1) : syr);
    const int y0 = (int)sy, y1 = min(y0 + 1, a.height - 1);
    const float fy = sy - y0, wy = 1 - fy;
    const uint8_t* top = a.px + (long long)y0 * a.row_stride;
    const uint8_t* bottom = a.px + (long long)y1 * a.row_stride;
    auto sample = [&](int o) {
      const float upper = top[x0 + o] * wx + top[x1 + o] * fx;
      const float lower = bottom[x0 + o] * wx + bottom[x1 + o] * fx;
      return (upper * wy + lower * fy) / 255.0f;
    };
    const int red = a.bgr ? 2 : 0, blue = 2 - red;
    r = sample(red);
    g = sample(1);
    b = sample(blue);
  }
  a.out[i] = r;
  a.out[plane + i] = g;
  a.out[2 * plane + i] = b;
}

// ---------------------------------------------------------------- NMS candidates

constexpr int kCandThreads = 1024;
constexpr int kCandCap = 16384;  // keys one LDS block sorts (8-byte keys)
constexpr int kCandMaxAnchors = 1 << 22;  // larger images sort through a global work buffer

struct CandArgs {
  const float* head;  // [B][channels][anchors]
  int channels, anchors, class_fields;
  float conf;
  int max_candidates;
  sy_detection* cand;  // [B][max_candidates]
  int* counts;         // [B]
};

// The candidate test of DecodeIndexed for anchor a (channels-first layout):
// first-best class with strict '>', finite confidence >= threshold, finite
// box, centre -> corner, positive size.
__device__ __forceinline__ bool candidate(const float* h, int anchors, int class_fields, float thr, int a,
                                          sy_detection* d) {
  float conf = -INFINITY;
  int cls = 0;
  for (int c = 4; c < class_fields; ++c) {
    const float s = h[(long long)c * anchors + a];
    if (s > conf) {
      conf = s;
      cls = c - 4;
    }
  }
  if (!isfinite(conf) || conf < thr) return false;
  float x = h[a], y = h[(long long)anchors + a], w = h[2LL * anchors + a], hh = h[3LL * anchors + a];
  if (!isfinite(x) || !isfinite(y) || !isfinite(w) || !isfinite(hh)) return false;
  x -= w * .5f;
  y -= hh * .5f;
  if (w <= 0 || hh <= 0) return false;
  *d = sy_detection{cls, conf, x, y, w, hh, a};
  return true;
}

// Sort key: confidence descending (order-preserving bits, -0 as +0), then
// anchor ascending, which is the stable sort of anchors in index order.
__device__ __forceinline__ unsigned long long cand_key(float conf, int a) {
  unsigned u = __float_as_uint(conf == 0.0f ? 0.0f : conf);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)(~u) << 32) | (unsigned)a;
}

static int resolve_layout(int channels, int anchors, const sy_decode_options* o, int* class_fields) {
  int layout = o->layout;
  if (layout == SY_OUTPUT_AUTO) {
    const int expected = o->class_count > 0 ? 4 + o->class_count : 0;
    if (expected > 0 && channels == expected && anchors != expected) layout = SY_OUTPUT_CHANNELS_FIRST;
    else if (expected > 0 && anchors == expected && channels != expected) layout = SY_OUTPUT_CHANNELS_LAST;
    else if (anchors == 6 && channels != 6) layout = SY_OUTPUT_END_TO_END;
    else if (channels >= 5 && channels < anchors) layout = SY_OUTPUT_CHANNELS_FIRST;
    else if (anchors >= 5 && anchors < channels) layout = SY_OUTPUT_CHANNELS_LAST;
    else SY_CHECK(false, SY_EINVAL, "Ambiguous YOLO output layout. Set OutputLayout explicitly.");
  }
  SY_CHECK(layout == SY_OUTPUT_CHANNELS_FIRST, SY_EUNSUPPORTED,
           "the device candidate stage takes channels-first [B, 4+nc, anchors] heads");
  *class_fields = o->class_count > 0 ? 4 + o->class_count : channels;
  SY_CHECK(channels >= 5 && *class_fields >= 5 && *class_fields <= channels, SY_EINVAL,
           "ClassCount does not match output.");
  return SY_OK;
}

// Per-anchor pass over the whole GPU: a workgroup owns 64 anchors of one image
// and its four waves scan a quarter of the classes each (coalesced rows); the
// partial first-best classes are merged in class order, so ties still go to
// the lowest class.  Writes the anchor's sort key, or ~0 for a non-candidate.
constexpr int kScanRows = 24;

__global__ __launch_bounds__(256) void cand_scan_kernel(const CandArgs a, unsigned long long* __restrict__ keys) {
  __shared__ float pc[4][64];
  __shared__ int pk[4][64];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int an = blockIdx.x * 64 + lane;
  const float* h = a.head + (long long)b * a.channels * a.anchors;
  const int nclass = a.class_fields - 4, per = (nclass + 3) / 4;
  const int c0 = 4 + wave * per, c1 = min(a.class_fields, c0 + per);
  float conf = -INFINITY;
  int cls = 0;
  if (an < a.anchors && c0 < c1) {
    // The wave's class rows are loaded in batches of kScanRows before any is
    // compared (rows past the end re-read the last one).
    for (int cb = c0; cb < c1; cb += kScanRows) {
      float v[kScanRows];
#pragma unroll
      for (int i = 0; i < kScanRows; ++i) v[i] = h[(long long)min(cb + i, c1 - 1) * a.anchors + an];
#pragma unroll
      for (int i = 0; i < kScanRows; ++i)
        if (cb + i < c1 && v[i] > conf) {
          conf = v[i];
          cls = cb + i - 4;
        }
    }
  }
  pc[wave][lane] = conf;
  pk[wave][lane] = cls;
  __syncthreads();
  if (wave != 0 || an >= a.anchors) return;
  conf = pc[0][lane];
  cls = pk[0][lane];
#pragma unroll
  for (int w = 1; w < 4; ++w)
    if (pc[w][lane] > conf) {
      conf = pc[w][lane];
      cls = pk[w][lane];
    }
  bool ok = isfinite(conf) && conf >= a.conf;
  if (ok) {
    const float x = h[an], y = h[(long long)a.anchors + an], w = h[2LL * a.anchors + an], hh = h[3LL * a.anchors + an];
    ok = isfinite(x) && isfinite(y) && isfinite(w) && isfinite(hh) && w > 0 && hh > 0;
  }
  keys[(long long)b * a.anchors + an] = ok ? cand_key(conf, an) : ~0ULL;
}

// One workgroup per image: compact the candidate keys into LDS, bitonic sort
// (confidence descending, anchor ascending), write the first max_candidates.
__global__ __launch_bounds__(kCandThreads) void cand_sort_kernel(const CandArgs a,
                                                                 const unsigned long long* __restrict__ keys_in) {
  extern __shared__ unsigned long long keys[];
  __shared__ int s_count;
  const int tid = threadIdx.x, b = blockIdx.x;
  const float* h = a.head + (long long)b * a.channels * a.anchors;
  if (tid == 0) s_count = 0;
  __syncthreads();
  for (int base = 0; base < a.anchors; base += kCandThreads) {
    const int an = base + tid;
    const unsigned long long k = an < a.anchors ? keys_in[(long long)b * a.anchors + an] : ~0ULL;
    const bool take = k != ~0ULL;
    // One LDS atomic per wave; lanes numbered in lane order.
    const unsigned long long m = __ballot(take);
    if (m != 0) {
      const int lane = tid & 63, leader = __ffsll((long long)m) - 1;
      int slot = 0;
      if (lane == leader) slot = atomicAdd(&s_count, __popcll(m));
      slot = __shfl(slot, leader);
      if (take) keys[slot + __popcll(m & ((1ull << lane) - 1))] = k;
    }
  }
  __syncthreads();
  const int n = s_count;
  int p = 1;
  while (p < n) p <<= 1;
  for (int i = n + tid; i < p; i += kCandThreads) keys[i] = ~0ULL;
  __syncthreads();
  // Bitonic sort, ascending, of p keys.
  for (int k = 2; k <= p; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < p; i += kCandThreads) {
        const int l = i ^ j;
        if (l > i) {
          const unsigned long long ki = keys[i], kl = keys[l];
          const bool up = (i & k) == 0;
          if ((ki > kl) == up) {
            keys[i] = kl;
            keys[l] = ki;
          }
        }
      }
      __syncthreads();
    }
  }
  const int m = min(n, a.max_candidates);
  sy_detection* out = a.cand + (long long)b * a.max_candidates;
  for (int i = tid; i < m; i += kCandThreads) {
    const int an = (int)(keys[i] & 0xffffffffu);
    sy_detection d;
    candidate(h, a.anchors, a.class_fields, a.conf, an, &d);
    out[i] = d;
  }
  if (tid == 0) a.counts[b] = m;
}

// Images with more anchors than one LDS block sorts: the candidate keys
// are compacted into a global work buffer of p (a power of two) keys per
// image and bitonic-sorted there with LDS doing most of the work: each
// block of kCandCap keys first runs every stage up to that size in LDS;
// then for each larger merge size the strides >= kCandCap pass over global
// memory and the smaller strides finish block by block in LDS.  One
// workgroup per image; __syncthreads orders its global accesses.
__device__ __forceinline__ void cand_cmpswap(unsigned long long* v, int i, int l, bool up) {
  const unsigned long long ki = v[i], kl = v[l];
  if ((ki > kl) == up) {
    v[i] = kl;
    v[l] = ki;
  }
}

__global__ __launch_bounds__(kCandThreads) void cand_sort_large_kernel(const CandArgs a,
                                                                       const unsigned long long* __restrict__ keys_in,
                                                                       unsigned long long* __restrict__ work, int p) {
  extern __shared__ unsigned long long lk[];
  __shared__ int s_count;
  const int tid = threadIdx.x, b = blockIdx.x;
  const float* h = a.head + (long long)b * a.channels * a.anchors;
  unsigned long long* wk = work + (long long)b * p;
  if (tid == 0) s_count = 0;
  __syncthreads();
  for (int base = 0; base < a.anchors; base += kCandThreads) {
    const int an = base + tid;
    const unsigned long long k = an < a.anchors ? keys_in[(long long)b * a.anchors + an] : ~0ULL;
    const bool take = k != ~0ULL;
    const unsigned long long m = __ballot(take);
    if (m != 0) {
      const int lane = tid & 63, leader = __ffsll((long long)m) - 1;
      int slot = 0;
      if (lane == leader) slot = atomicAdd(&s_count, __popcll(m));
      slot = __shfl(slot, leader);
      if (take) wk[slot + __popcll(m & ((1ull << lane) - 1))] = k;
    }
  }
  __syncthreads();
  const int n = s_count;
  for (int i = n + tid; i < p; i += kCandThreads) wk[i] = ~0ULL;
  __syncthreads();
  constexpr int L = kCandCap;
  // Phase A: every stage with k <= L inside each block.
  for (int blk = 0; blk < p; blk += L) {
    for (int i = tid; i < L; i += kCandThreads) lk[i] = wk[blk + i];
    __syncthreads();
    for (int k = 2; k <= L; k <<= 1)
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < L; i += kCandThreads) {
          const int l = i ^ j;
          if (l > i) cand_cmpswap(lk, i, l, ((blk + i) & k) == 0);
        }
        __syncthreads();
      }
    for (int i = tid; i < L; i += kCandThreads) wk[blk + i] = lk[i];
    __syncthreads();
  }
  // Phase B: larger merges.
  for (int k = 2 * L; k <= p; k <<= 1) {
    for (int j = k >> 1; j >= L; j >>= 1) {
      for (int i = tid; i < p; i += kCandThreads) {
        const int l = i ^ j;
        if (l > i) cand_cmpswap(wk, i, l, (i & k) == 0);
      }
      __syncthreads();
    }
    for (int blk = 0; blk < p; blk += L) {
      for (int i = tid; i < L; i += kCandThreads) lk[i] = wk[blk + i];
      __syncthreads();
      for (int j = L >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < L; i += kCandThreads) {
          const int l = i ^ j;
          if (l > i) cand_cmpswap(lk, i, l, ((blk + i) & k) == 0);
        }
        __syncthreads();
      }
      for (int i = tid; i < L; i += kCandThreads) wk[blk + i] = lk[i];
      __syncthreads();
    }
  }
  const int m = min(n, a.max_candidates);
  sy_detection* out = a.cand + (long long)b * a.max_candidates;
  for (int i = tid; i < m; i += kCandThreads) {
    const int an = (int)(wk[i] & 0xffffffffu);
    sy_detection d;
    candidate(h, a.anchors, a.class_fields, a.conf, an, &d);
    out[i] = d;
  }
  if (tid == 0) a.counts[b] = m;
}

// Scratch of the candidate stage: the per-anchor keys [batch][anchors] and,
// for images larger than one LDS block, the sort's work buffer [batch][p].
static size_t cand_pow2(int anchors) {
  size_t p = 1;
  while (p < (size_t)anchors) p <<= 1;
  return p;
}
size_t nms_scratch_bytes(int batch, int anchors) {
  const size_t keys = ((size_t)batch * anchors * sizeof(unsigned long long) + 255) & ~size_t(255);
  return keys + (anchors > kCandCap ? (size_t)batch * cand_pow2(anchors) * sizeof(unsigned long long) : 0);
}

// Both passes; scratch holds nms_scratch_bytes(batch, anchors) bytes (device).
static int nms_candidates(sy_ctx* ctx, const float* head, int batch, int channels, int anchors,
                          const sy_decode_options* o, sy_detection* cand, int* counts, char* scratch) {
  int class_fields = 0;
  SY_TRY(resolve_layout(channels, anchors, o, &class_fields));
  SY_CHECK(anchors <= kCandMaxAnchors, SY_EUNSUPPORTED, "%d anchors exceed the %d the device sort handles", anchors,
           kCandMaxAnchors);
  SY_CHECK(batch <= 65535, SY_EUNSUPPORTED, "candidate batch too large");
  unsigned long long* keys_tmp = (unsigned long long*)scratch;
  const bool large = anchors > kCandCap;
  const int p = (int)cand_pow2(anchors);
  const size_t lds = (size_t)(large ? kCandCap : p) * sizeof(unsigned long long);
  // Set once per process (a function-local static: safe across threads).
  static const hipError_t attr = [] {
    const int bytes = (int)(kCandCap * sizeof(unsigned long long));
    hipError_t e = hipFuncSetAttribute((const void*)cand_sort_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)cand_sort_large_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    return e;
  }();
  SY_HIP(attr);
  CandArgs a{head, channels, anchors, class_fields, o->confidence, o->max_candidates, cand, counts};
  {
    ProfScope prof(ctx, "nms_cand_scan", 0, 4.0 * (double)batch * anchors * class_fields + 8.0 * batch * anchors);
    hipLaunchKernelGGL(cand_scan_kernel, dim3((unsigned)((anchors + 63) / 64), (unsigned)batch), dim3(256), 0,
                       ctx->stream, a, keys_tmp);
    SY_TRY(check_launch("nms_cand_scan"));
  }
  ProfScope prof(ctx, "nms_cand_sort", 0, 8.0 * (double)batch * anchors);
  if (large) {
    unsigned long long* work =
        (unsigned long long*)(scratch + ((((size_t)batch * anchors * sizeof(unsigned long long)) + 255) & ~size_t(255)));
    hipLaunchKernelGGL(cand_sort_large_kernel, dim3(batch), dim3(kCandThreads), lds, ctx->stream, a, keys_tmp, work,
                       p);
  } else {
    hipLaunchKernelGGL(cand_sort_kernel, dim3(batch), dim3(kCandThreads), lds, ctx->stream, a, keys_tmp);
  }
  return check_launch("nms_cand_sort");
}

}  // namespace sy

using namespace sy;

extern "C" {

int sy_letterbox_device(sy_ctx* ctx, const uint8_t* pixels, int width, int height, int tw, int th, int bgr,
                        int row_stride, float* out, sy_letterbox* t) {
  SY_CHECK(ctx && pixels && out && t, SY_EINVAL, "null argument");
  SY_CHECK(width > 0 && height > 0 && tw > 0 && th > 0, SY_EINVAL, "Image dimensions must be positive.");
  if (row_stride == 0) row_stride = width * 3;
  SY_CHECK(row_stride >= width * 3, SY_EINVAL, "Image buffer too short.");
  // Geometry exactly as the host letterbox computes it.
  const float gain = std::min((float)tw / width, (float)th / height);
  const int rw = std::clamp((int)std::nearbyint(width * gain), 1, tw);
  const int rh = std::clamp((int)std::nearbyint(height * gain), 1, th);
  LetterboxArgs a{pixels, width, height, row_stride, bgr ? 1 : 0, tw, th, rw, rh, (tw - rw) / 2, (th - rh) / 2, out};
  const long long plane = (long long)tw * th;
  {
    ProfScope prof(ctx, "letterbox", 0, (double)height * row_stride + 12.0 * plane);
    hipLaunchKernelGGL(letterbox_kernel, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, ctx->stream, a);
    SY_TRY(check_launch("letterbox"));
  }
  *t = sy_letterbox{width, height, tw, th, (float)rw / width, (float)rh / height, a.pad_x, a.pad_y};
  return SY_OK;
}

int sy_nms_candidates(sy_ctx* ctx, const float* head, int batch, int channels, int anchors,
                      const sy_decode_options* o, sy_detection* cand, int* counts) {
  SY_CHECK(ctx && head && o && cand && counts, SY_EINVAL, "null argument");
  SY_CHECK(batch > 0 && anchors > 0 && o->max_candidates > 0, SY_EINVAL, "invalid candidate request");
  SY_CHECK(anchors <= kCandMaxAnchors, SY_EUNSUPPORTED, "%d anchors exceed the %d the device sort handles", anchors,
           kCandMaxAnchors);
  SY_TRY(ensure_scratch(ctx, nms_scratch_bytes(batch, anchors)));
  return nms_candidates(ctx, head, batch, channels, anchors, o, cand, counts, ctx->scratch);
}

int sy_decode_detections_device(sy_ctx* ctx, const float* head, int batch, int channels, int anchors,
                                const sy_decode_options* o, const sy_letterbox* t, sy_detection* out, int max_out,
                                int* counts) {
  SY_CHECK(ctx && head && o && t && counts && (out || max_out == 0), SY_EINVAL, "null argument");
  SY_CHECK(batch > 0, SY_EINVAL, "invalid batch");
  for (int b = 0; b < batch; ++b)
    SY_CHECK(t[b].source_width > 0 && t[b].source_height > 0 && t[b].target_width > 0 && t[b].target_height > 0 &&
                 std::isfinite(t[b].scale_x) && std::isfinite(t[b].scale_y) && t[b].scale_x > 0 && t[b].scale_y > 0 &&
                 o->max_detections > 0 && o->max_candidates > 0 && o->class_count >= 0,
             SY_EINVAL, "Invalid decode transform/options.");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "the decoder synchronises; it cannot be captured");
  const int cap = std::min(o->max_candidates, anchors);
  sy_decode_options oc = *o;
  oc.max_candidates = cap;
  SY_CHECK(head && batch > 0 && anchors > 0 && oc.max_candidates > 0, SY_EINVAL, "invalid candidate request");
  const size_t cand_bytes = (size_t)batch * cap * sizeof(sy_detection);
  const size_t count_off = (cand_bytes + 255) & ~size_t(255);
  const size_t keys_off = (count_off + (size_t)batch * sizeof(int) + 255) & ~size_t(255);
  SY_CHECK(anchors <= kCandMaxAnchors, SY_EUNSUPPORTED, "%d anchors exceed the %d the device sort handles", anchors,
           kCandMaxAnchors);
  SY_TRY(ensure_scratch(ctx, keys_off + nms_scratch_bytes(batch, anchors)));
  sy_detection* dcand = (sy_detection*)ctx->scratch;
  int* dcount = (int*)(ctx->scratch + count_off);
  SY_TRY(nms_candidates(ctx, head, batch, channels, anchors, &oc, dcand, dcount, ctx->scratch + keys_off));
  std::vector<int> n(batch);
  std::vector<sy_detection> all((size_t)batch * cap);
  SY_HIP(hipMemcpyAsync(n.data(), dcount, (size_t)batch * sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
  SY_HIP(hipMemcpyAsync(all.data(), dcand, cand_bytes, hipMemcpyDeviceToHost, ctx->stream));
  SY_HIP(hipStreamSynchronize(ctx->stream));
  for (int b = 0; b < batch; ++b) {
    std::vector<sy_detection> cand(all.begin() + (size_t)b * cap, all.begin() + (size_t)b * cap + n[b]);
    SY_TRY(finish_detections(cand, false, o, &t[b], out ? out + (size_t)b * max_out : nullptr, max_out, &counts[b]));
  }
  return SY_OK;
}

}  // extern "C"
