// Instance masks (YOLO segmentation heads): low-res logits on FP32 MFMA, then
// one kernel for every instance's bilinear resample to source pixels,
// sigmoid and box crop.  Semantics of CpuMaskDecoder.Decode
// (src/SimdYolo/CpuMaskDecoder.cs:18-81).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "sy_internal.h"

namespace sy {

struct MaskInst {
  int left, top, width, height;
  int begin_x, begin_y;
  long long offset;
};

// Source-axis -> prototype-axis mapping of CpuMaskDecoder.cs:33-38, float
// math in the reference's order: the low-res sample pair and weight of source
// coordinate i.
struct AxisMap {
  int start, end, length;
};
__device__ __forceinline__ void map_coord(const AxisMap m, int i, int& first, int& second, float& frac) {
#pragma clang fp contract(off)
  float c = m.start + (i + .5f) * (float)(m.end - m.start) / m.length - .5f;
  c = fminf(fmaxf(c, (float)m.start), (float)(m.end - 1));
  first = (int)c;
  second = min(first + 1, m.end - 1);
  frac = c - first;
}

// One workgroup row per instance; threads stride over its crop.
__global__ __launch_bounds__(256) void mask_crop_kernel(const float* __restrict__ low, int mw, int plane,
                                                        const AxisMap ax, const AxisMap ay,
                                                        const MaskInst* __restrict__ inst, float* __restrict__ out) {
#pragma clang fp contract(off)
  const MaskInst m = inst[blockIdx.y];
  const float* lp = low + (long long)blockIdx.y * plane;
  const long long count = (long long)m.width * m.height;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (long long)gridDim.x * blockDim.x) {
    const int ry = (int)(i / m.width), rx = (int)(i - (long long)ry * m.width);
    const int y = m.top + ry, x = m.left + rx;
    float v = 0.f;
    if (y >= m.begin_y && x >= m.begin_x) {
      int x0, x1, y0, y1;
      float f, g;
      map_coord(ax, x, x0, x1, f);
      map_coord(ay, y, y0, y1, g);
      const float* r0 = lp + (long long)y0 * mw;
      const float* r1 = lp + (long long)y1 * mw;
      const float upper = r0[x0] * (1.f - f) + r0[x1] * f;
      const float lower = r1[x0] * (1.f - f) + r1[x1] * f;
      const float z = upper * (1.f - g) + lower * g;
      v = 1.f / (1.f + __expf(-z));
    }
    out[m.offset + i] = v;
  }
}

}  // namespace sy

using namespace sy;

extern "C" int sy_mask_decode(sy_ctx* ctx, const sy_tensor* protos, const float* coeffs, int ld_coeff, int k,
                              const sy_detection* boxes, const sy_letterbox* t, float* masks, size_t capacity,
                              sy_mask_info* info) {
#pragma clang fp contract(off)
  SY_CHECK(ctx && t && (k == 0 || (coeffs && boxes && masks && info)), SY_EINVAL, "null argument");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "mask decode is not capturable (host tables, synchronous)");
  SY_TRY(check_view(protos, "mask prototypes", true));
  SY_CHECK(protos->n == 1, SY_EINVAL, "Single-image mask decoding only.");
  const int nm = protos->c, mh = protos->h, mw = protos->w, plane = mh * mw;
  SY_CHECK(k >= 0 && ld_coeff >= nm, SY_EINVAL, "invalid coefficient rows");
  SY_CHECK(nm % 4 == 0, SY_EUNSUPPORTED, "mask coefficient count must be a multiple of 4 (got %d)", nm);
  SY_CHECK(t->source_width > 0 && t->source_height > 0 && t->target_width > 0 && t->target_height > 0, SY_EINVAL,
           "invalid letterbox transform");
  if (k == 0) return SY_OK;
  // ROI of the letterboxed image inside the prototype grid (CpuMaskDecoder.cs:22-25).
  const int left_roi = std::clamp((int)std::nearbyint((float)t->pad_x * mw / t->target_width), 0, mw - 1);
  const int top_roi = std::clamp((int)std::nearbyint((float)t->pad_y * mh / t->target_height), 0, mh - 1);
  const int right_roi = std::clamp(
      (int)std::nearbyint((t->pad_x + t->source_width * t->scale_x) * mw / t->target_width), left_roi + 1, mw);
  const int bottom_roi = std::clamp(
      (int)std::nearbyint((t->pad_y + t->source_height * t->scale_y) * mh / t->target_height), top_roi + 1, mh);
  const AxisMap ax{left_roi, right_roi, t->source_width}, ay{top_roi, bottom_roi, t->source_height};
  std::vector<MaskInst> inst(k);
  long long total = 0, most = 0;
  for (int i = 0; i < k; ++i) {
    const sy_detection& b = boxes[i];
    MaskInst& m = inst[i];
    m.left = (int)std::floor(b.x);
    m.top = (int)std::floor(b.y);
    const int right = (int)std::ceil(b.x + b.width), bottom = (int)std::ceil(b.y + b.height);
    m.width = right - m.left;
    m.height = bottom - m.top;
    m.begin_x = std::max(m.left, (int)std::ceil(b.x));
    m.begin_y = std::max(m.top, (int)std::ceil(b.y));
    SY_CHECK(m.left >= 0 && m.top >= 0 && right <= t->source_width && bottom <= t->source_height && m.width > 0 &&
                 m.height > 0,
             SY_EINVAL, "instance %d box is empty or outside the source image", i);
    m.offset = total;
    const long long n = (long long)m.width * m.height;
    total += n;
    most = std::max(most, n);
    info[i] = sy_mask_info{m.left, m.top, m.width, m.height, m.offset};
  }
  SY_CHECK((size_t)total <= capacity, SY_EINVAL, "mask buffer holds %zu floats, %lld needed", capacity, total);
  // Scratch: low-res logits, packed coefficients, instance records.
  auto align = [](size_t v) { return (v + 255) & ~size_t(255); };
  const size_t low_b = align((size_t)k * plane * 4), coef_b = align((size_t)k * nm * 4);
  const size_t inst_b = align(sizeof(MaskInst) * k);
  // A dense NCHW prototype tensor (a Segment model's own output) is turned
  // channel-last first so the GEMM reads each pixel's coefficients contiguously.
  const bool nchw = protos->layout == SY_LAYOUT_NCHW;
  const size_t pt_b = nchw ? align((size_t)nm * plane * 4) : 0;
  SY_TRY(ensure_scratch(ctx, low_b + coef_b + inst_b + pt_b));
  SY_TRY(ensure_host_stage(ctx, sizeof(MaskInst) * k));
  char* s = ctx->scratch;
  float* low = (float*)s; s += low_b;
  float* cpk = (float*)s; s += coef_b;
  MaskInst* dinst = (MaskInst*)s; s += inst_b;
  hipStream_t st = ctx->stream;
  const float* pdata = protos->data;
  int pld = protos->ldc;
  if (nchw) {
    const sy_tensor pv{(float*)s, 1, nm, mh, mw, nm, SY_LAYOUT_NHWC};
    SY_TRY(op_nchw_to_view(ctx, protos->data, &pv));
    pdata = pv.data;
    pld = nm;
  }
  // One DMA from pinned staging (the call synchronises before returning, so
  // the staging is free again for the next call).
  memcpy(ctx->host_stage, inst.data(), sizeof(MaskInst) * k);
  SY_HIP(hipMemcpyAsync(dinst, ctx->host_stage, sizeof(MaskInst) * k, hipMemcpyHostToDevice, st));
  // Coefficient rows: used in place when aligned, else packed densely.
  const float* A = coeffs;
  int lda = ld_coeff;
  if ((ld_coeff & 3) != 0 || ((uintptr_t)coeffs & 15) != 0) {
    const sy_tensor src{(float*)coeffs, 1, nm, 1, k, ld_coeff, SY_LAYOUT_NHWC};
    const sy_tensor dst{cpk, 1, nm, 1, k, nm, SY_LAYOUT_NHWC};
    SY_TRY(op_copy(ctx, &src, &dst));
    A = cpk;
    lda = nm;
  }
  SY_TRY(gemm_nt(ctx, A, k, nm, lda, pdata, plane, pld, low, plane, "mask_gemm"));
  {
    const unsigned gx = (unsigned)std::min<long long>((most + 255) / 256, 256);
    ProfScope prof(ctx, "mask_crop", 0, 4.0 * (double)total + 4.0 * 4.0 * (double)total);
    hipLaunchKernelGGL(mask_crop_kernel, dim3(gx, k), dim3(256), 0, st, low, mw, plane, ax, ay, dinst, masks);
    SY_TRY(check_launch("mask_crop"));
  }
  SY_HIP(hipStreamSynchronize(st));
  return prof_collect(ctx);
}
