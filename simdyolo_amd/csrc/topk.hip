// End-to-end two-stage top-k (YOLO26 / v10 heads), bit-exact with
// CpuEndToEnd.SelectPt / SelectOnnx (src/SimdYolo/CpuEndToEnd.cs:26-241).
//
// One 1024-thread workgroup per image, everything in LDS:
//   * every candidate gets a unique 64-bit key: an order-preserving 32-bit
//     image of its score (-0 ties +0; NaN lowest under PT rules, highest under
//     ONNX rules) above the inverted tie index, so "larger key" is exactly the
//     reference's order (score descending, tie index ascending);
//   * an MSB-first radix select (eight 8-bit digit passes with LDS histograms)
//     finds the k-th largest key, one compaction pass collects the k keys at
//     or above it, and a bitonic sort orders them;
//   * stage 1 ranks anchors by their class maximum (.NET Max: NaN
//     propagates); stage 2 enumerates (anchor, class) candidates in tie order
//     (PT: anchors ascending, then class; ONNX: stage-1 rank, then class), so
//     the enumeration index is the tie index.
#include <cstdint>

#include "sy_internal.h"

namespace sy {

constexpr int kTkThreads = 1024;
constexpr int kTkCap = 32768;  // candidates per stage held in LDS
constexpr int kTkMaxK = 1024;

__device__ __forceinline__ uint32_t score_key(float f, bool onnx) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return onnx ? 0xffffffffu : 0u;  // NaN
  if (u == 0x80000000u) u = 0u;                                          // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long full_key(uint32_t k32, uint32_t idx) {
  return ((unsigned long long)k32 << 32) | (unsigned long long)(0xffffffffu - idx);
}

struct TopkShared {
  uint32_t keys[kTkCap];
  unsigned long long sel[kTkMaxK];
  int anchors[kTkMaxK];
  int hist[256];
  int count;
  int digit, need;
};

// k-th largest of the n keys full_key(keys[i], i), i < n (k <= n).
__device__ unsigned long long radix_select(TopkShared& s, int n, int k) {
  unsigned long long prefix = 0, mask = 0;
  if (threadIdx.x == 0) s.need = k;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) s.hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const unsigned long long key = full_key(s.keys[i], (uint32_t)i);
      if ((key & mask) == prefix) atomicAdd(&s.hist[(int)((key >> shift) & 255u)], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int need = s.need, cum = 0, d = 255;
      for (; d > 0; --d) {
        if (cum + s.hist[d] >= need) break;
        cum += s.hist[d];
      }
      s.digit = d;
      s.need = need - cum;
    }
    __syncthreads();
    prefix |= (unsigned long long)s.digit << shift;
    mask |= 255ull << shift;
  }
  return prefix;
}

// Gather the k keys >= threshold into s.sel and sort them descending.
__device__ void collect_sorted(TopkShared& s, int n, int k, unsigned long long threshold) {
  if (threadIdx.x == 0) s.count = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const unsigned long long key = full_key(s.keys[i], (uint32_t)i);
    if (key >= threshold) {
      const int slot = atomicAdd(&s.count, 1);
      if (slot < kTkMaxK) s.sel[slot] = key;
    }
  }
  __syncthreads();
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = k + threadIdx.x; i < P; i += blockDim.x) s.sel[i] = 0ull;  // below every real key
  __syncthreads();
  // Bitonic sort, descending.
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const unsigned long long a = s.sel[i], b = s.sel[j];
          if (desc ? (a < b) : (a > b)) {
            s.sel[i] = b;
            s.sel[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(kTkThreads) void e2e_topk_kernel(const float* __restrict__ head, int channels,
                                                             int anchors, int nc, int k, int onnx,
                                                             float* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  TopkShared& s = *reinterpret_cast<TopkShared*>(smem);
  const int b = blockIdx.x;
  const float* src = head + (long long)b * channels * anchors;
  const bool ox = onnx != 0;

  // Stage 1: class maximum per anchor (NaN propagates).
  for (int a = threadIdx.x; a < anchors; a += blockDim.x) {
    float m = -INFINITY;
    bool nan = false;
    for (int c = 0; c < nc; ++c) {
      const float v = src[(long long)(4 + c) * anchors + a];
      nan |= v != v;
      m = fmaxf(m, v);
    }
    s.keys[a] = nan ? score_key(__uint_as_float(0x7fc00000u), ox) : score_key(m, ox);
  }
  __syncthreads();
  unsigned long long t1 = radix_select(s, anchors, k);
  collect_sorted(s, anchors, k, t1);
  // Stage-1 anchors in enumeration order for stage 2.
  for (int i = threadIdx.x; i < k; i += blockDim.x) s.anchors[i] = (int)(0xffffffffu - (uint32_t)s.sel[i]);
  __syncthreads();
  if (!ox) {
    // PT ties by anchor*nc + c: enumerate anchors ascending (sort indices).
    for (int i = threadIdx.x; i < k; i += blockDim.x) s.sel[i] = full_key(0u, (uint32_t)s.anchors[i]);
    __syncthreads();
    int P = 1;
    while (P < k) P <<= 1;
    for (int i = k + threadIdx.x; i < P; i += blockDim.x) s.sel[i] = 0ull;
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1)
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = threadIdx.x; i < P; i += blockDim.x) {
          const int j = i ^ stride;
          if (j > i) {
            const bool desc = (i & size) == 0;
            const unsigned long long x = s.sel[i], y = s.sel[j];
            if (desc ? (x < y) : (x > y)) {
              s.sel[i] = y;
              s.sel[j] = x;
            }
          }
        }
        __syncthreads();
      }
    for (int i = threadIdx.x; i < k; i += blockDim.x) s.anchors[i] = (int)(0xffffffffu - (uint32_t)s.sel[i]);
    __syncthreads();
  }
  // Stage 2: candidate e = j * nc + c for the j-th enumerated anchor.
  const int n2 = k * nc;
  for (int e = threadIdx.x; e < n2; e += blockDim.x) {
    const int j = e / nc, c = e - (e / nc) * nc;
    s.keys[e] = score_key(src[(long long)(4 + c) * anchors + s.anchors[j]], ox);
  }
  __syncthreads();
  unsigned long long t2 = radix_select(s, n2, k);
  collect_sorted(s, n2, k, t2);
  const int extra = channels - nc - 4, fields = 6 + extra;
  float* dst = out + (long long)b * k * fields;
  for (int idx = threadIdx.x; idx < k * fields; idx += blockDim.x) {
    const int i = idx / fields, f = idx - (idx / fields) * fields;
    const int e = (int)(0xffffffffu - (uint32_t)s.sel[i]);
    const int j = e / nc, c = e - (e / nc) * nc;
    const int a = s.anchors[j];
    float v;
    if (f < 4) v = src[(long long)f * anchors + a];
    else if (f == 4) v = src[(long long)(4 + c) * anchors + a];
    else if (f == 5) v = (float)c;
    else v = src[(long long)(nc + 4 + (f - 6)) * anchors + a];
    dst[idx] = v;
  }
}

int op_e2e_topk(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum, int onnx,
                float* out) {
  SY_CHECK(head && out, SY_EINVAL, "null argument");
  SY_CHECK(batch >= 0 && anchors >= 0 && nc > 0 && channels >= nc + 4 && maximum >= 0, SY_EINVAL,
           "invalid top-k arguments");
  SY_CHECK(!onnx || maximum <= anchors, SY_EINVAL, "ONNX rules need maximum <= anchors");
  const int k = maximum < anchors ? maximum : anchors;
  if (batch == 0 || k == 0) return SY_OK;
  SY_CHECK(k <= kTkMaxK, SY_EUNSUPPORTED, "top-k of %d exceeds %d", k, kTkMaxK);
  SY_CHECK(anchors <= kTkCap && (long long)k * nc <= kTkCap, SY_EUNSUPPORTED,
           "top-k over %d anchors x %d classes exceeds the %d-candidate LDS tile", anchors, nc, kTkCap);
  const size_t lds = sizeof(TopkShared);
  static bool attr_set = false;
  if (!attr_set) {
    SY_HIP(hipFuncSetAttribute((const void*)e2e_topk_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set = true;
  }
  ProfScope prof(ctx, "e2e_topk", 0, 4.0 * (double)batch * ((double)anchors * nc + (double)k * nc + (double)k * (channels + 2)));
  hipLaunchKernelGGL(e2e_topk_kernel, dim3(batch), dim3(kTkThreads), lds, ctx->stream, head, channels, anchors, nc,
                     k, onnx ? 1 : 0, out);
  return check_launch("e2e_topk");
}

}  // namespace sy
