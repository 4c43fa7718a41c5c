// Generic device ops of the reference's IDeviceBackend (src/SimdYolo/
// DeviceExecution.cs:41,61): the operation codes of the reference's
// IDeviceBackend.Compute on dense row-major tensors, taking the same 32-slot
// parameter block its DeviceOps and callers build (DeviceExecution.cs:107-190),
// and the batched matrix product of DeviceMatMul (VulkanExecution.cs:499-541).
//
// They serve modules outside the fused YOLO paths (and the op-by-op route of a
// host that drives the backend one module at a time); the whole-model forward
// does not use them.
//
// Design.  The host decodes the parameter block once per call into a typed
// descriptor for one kernel family, and checks every extent the descriptor
// reaches against the buffer lengths (a block that would read or write past a
// buffer is refused with SY_EINVAL before any launch; only the gather's
// data-dependent source index is clamped on the device).  Shapes are
// collapsed on the host (size-1 axes dropped, axes that stay contiguous in
// every operand merged), so the kernels see the fewest axes the layout allows:
//   * element-wise and broadcast ops run as float4 streams when the collapsed
//     inner axis is contiguous (or broadcast) in every operand and aligned;
//   * transposes whose inner output axis is not contiguous in the input go
//     through 64 x 64 LDS tiles (float4 reads along the input's contiguous
//     axis, float4 writes along the output's); the others are row gathers;
//   * slice, concat and contiguous-row transposes share one row-copy kernel;
//   * softmax over contiguous rows and the row maximum run one wave per row
//     with cross-lane reductions; softmax over a strided axis runs one thread
//     per column, so neighbouring threads read neighbouring addresses;
//   * spatial ops (resize, pools, depthwise and transposed conv, depth to
//     space) give each workgroup one output plane's run of pixels, so the
//     channel, its weights and its bias are uniform across the workgroup;
//   * index decompositions use multiply-high division by host-prepared
//     constants (indices below 2^31).
#include <cmath>
#include <cstdint>
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <vector>

#include "sy_internal.h"

namespace sy {

// --------------------------------------------------------------- helpers

// n / d for 0 <= n < 2^31 by a multiply-high and a shift (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994):
// with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> l; the sum stays below 2^32 for n < 2^31.
struct FastDiv {
  uint32_t d = 1, m = 1, s = 0;
};

static FastDiv make_div(uint32_t d) {
  FastDiv f;
  f.d = d ? d : 1;
  uint32_t l = 0;
  while ((1ull << l) < f.d) ++l;
  f.s = l;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << l) - f.d)) / f.d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) { return (__umulhi(n, f.m) + n) >> f.s; }

// q = n / d, r = n - q d.
__device__ __forceinline__ uint32_t fdivmod(uint32_t n, const FastDiv& f, uint32_t* r) {
  const uint32_t q = fdiv(n, f);
  *r = n - q * f.d;
  return q;
}

__device__ __forceinline__ float logistic(float x) { return 1.0f / (1.0f + expf(-x)); }

constexpr int kThreads = 256;
constexpr long long kMaxItems = 0x7fffffffLL;  // flat indices stay below 2^31

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static float bits_to_float(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static unsigned grid_for(long long work, int per_block = kThreads) {
  return (unsigned)((work + per_block - 1) / per_block);
}

// --------------------------------------------------------------- element-wise (ops 1-9)

template <int OP>
__device__ __forceinline__ float unary_fn(float x, float alpha) {
  if constexpr (OP == 1) return x * logistic(x);
  else if constexpr (OP == 2) return logistic(x);
  else if constexpr (OP == 3) return __builtin_elementwise_maximum(x, 0.f);  // NaN stays NaN
  else if constexpr (OP == 4) return x * alpha;
  else if constexpr (OP == 5) return expf(x);
  else if constexpr (OP == 6) return sqrtf(x);
  else if constexpr (OP == 7) return -x;
  else if constexpr (OP == 8) return fabsf(x);
  else return x >= 0.f ? x : x * alpha;  // 9: leaky
}

// VEC: each thread maps one float4 (both pointers 16-byte aligned); the last
// n % 4 elements go to the first threads of the scalar tail.
template <int OP, bool VEC>
__global__ __launch_bounds__(kThreads) void unary_kernel(const float* __restrict__ a, float* __restrict__ c,
                                                         uint32_t n, float alpha) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if constexpr (VEC) {
    const uint32_t n4 = n >> 2;
    if (t < n4) {
      const float4 v = reinterpret_cast<const float4*>(a)[t];
      reinterpret_cast<float4*>(c)[t] =
          make_float4(unary_fn<OP>(v.x, alpha), unary_fn<OP>(v.y, alpha), unary_fn<OP>(v.z, alpha),
                      unary_fn<OP>(v.w, alpha));
    }
    const uint32_t tail = (n4 << 2) + t;
    if (t < (n & 3u)) c[tail] = unary_fn<OP>(a[tail], alpha);
  } else {
    if (t < n) c[t] = unary_fn<OP>(a[t], alpha);
  }
}

// --------------------------------------------------------------- broadcast binary (ops 10-16)

template <int OP>
__device__ __forceinline__ float binary_fn(float x, float y) {
  if constexpr (OP == 10) return x + y;
  else if constexpr (OP == 11) return x - y;
  else if constexpr (OP == 12) return x * y;
  else if constexpr (OP == 13) return x / y;
  else if constexpr (OP == 14) return powf(x, y);
  else if constexpr (OP == 15) return __builtin_elementwise_maximum(x, y);
  else return __builtin_elementwise_minimum(x, y);  // 16
}

// A collapsed broadcast: `rank` axes (outer first), sizes and the strides of
// A and B along each (0 on broadcast axes).  The output is dense.
struct Bcast {
  int rank;
  uint32_t size[4];
  FastDiv div[4];
  uint32_t sa[4], sb[4];
};

// Source offsets of flat output element e.
__device__ __forceinline__ void bcast_offsets(const Bcast& g, uint32_t e, uint32_t* oa, uint32_t* ob) {
  uint32_t a = 0, b = 0;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    if (j < g.rank) {
      uint32_t coord;
      e = fdivmod(e, g.div[j], &coord);
      a += coord * g.sa[j];
      b += coord * g.sb[j];
    }
  }
  *oa = a;
  *ob = b;
}

// One output float4 per thread, inside one row of the inner axis (its length
// a multiple of 4): the offsets are found once per float4, and an operand
// whose inner stride is 0 contributes one value to all four lanes.
template <int OP>
__global__ __launch_bounds__(kThreads) void binary_vec_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                              float* __restrict__ c, const Bcast g, uint32_t n4) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= n4) return;
  uint32_t oa, ob;
  bcast_offsets(g, t << 2, &oa, &ob);
  const int in = g.rank - 1;
  float4 x, y;
  if (g.sa[in]) x = *reinterpret_cast<const float4*>(a + oa);
  else x = make_float4(a[oa], a[oa], a[oa], a[oa]);
  if (g.sb[in]) y = *reinterpret_cast<const float4*>(b + ob);
  else y = make_float4(b[ob], b[ob], b[ob], b[ob]);
  reinterpret_cast<float4*>(c)[t] =
      make_float4(binary_fn<OP>(x.x, y.x), binary_fn<OP>(x.y, y.y), binary_fn<OP>(x.z, y.z), binary_fn<OP>(x.w, y.w));
}

template <int OP>
__global__ __launch_bounds__(kThreads) void binary_flat_kernel(const float* __restrict__ a,
                                                               const float* __restrict__ b, float* __restrict__ c,
                                                               const Bcast g, uint32_t n) {
  const uint32_t e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  uint32_t oa, ob;
  bcast_offsets(g, e, &oa, &ob);
  c[e] = binary_fn<OP>(a[oa], b[ob]);
}

// --------------------------------------------------------------- row copies (slice 24, concat 26, transpose 23)

// Element x of row r: dst[r * dst_row + x] = src[base(r) + x], where base(r)
// decomposes r over up to three outer axes (outer first) with their source
// strides.  Rows have `len` elements; `n` elements are copied in all (the
// last row may be partial).
struct RowCopy {
  int outer_rank;
  FastDiv odiv[3];
  uint32_t ost[3];
  FastDiv len;
  uint32_t dst_row;
  uint32_t n;
};

__device__ __forceinline__ uint32_t row_source(const RowCopy& g, uint32_t r) {
  uint32_t off = 0;
#pragma unroll
  for (int j = 2; j >= 0; --j) {
    if (j < g.outer_rank) {
      uint32_t coord;
      r = fdivmod(r, g.odiv[j], &coord);
      off += coord * g.ost[j];
    }
  }
  return off;
}

// VEC: row length, row strides and both bases are multiples of 4 floats, so a
// float4 never straddles rows and both accesses are 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void row_copy_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                            const RowCopy g) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t e = VEC ? t << 2 : t;
  if (e >= g.n) return;
  uint32_t x;
  const uint32_t r = fdivmod(e, g.len, &x);
  const uint32_t so = row_source(g, r) + x, dofs = r * g.dst_row + x;
  if constexpr (VEC) {
    *reinterpret_cast<float4*>(dst + dofs) = *reinterpret_cast<const float4*>(src + so);
  } else {
    dst[dofs] = src[so];
  }
}

// --------------------------------------------------------------- tiled transpose (op 23)

// Output axes (collapsed): `inner` (contiguous in the output) and `q`
// (contiguous in the input, stride 1), plus up to two batch axes.  A
// workgroup moves a 64 (inner) x 64 (q) tile: it reads 64 runs of 64
// consecutive input floats (one per inner coordinate), holds them in LDS and
// writes 64 runs of 64 consecutive output floats (one per q coordinate).
struct TileT {
  uint32_t n_inner, n_q;        // axis lengths
  uint32_t in_st_inner;         // input stride of the inner axis
  uint32_t out_st_q;            // output stride of the q axis
  int nb;                       // batch axes (0..2), outer first
  FastDiv bdiv[2];
  uint32_t b_in[2], b_out[2];   // batch strides in the input and the output
  uint32_t tiles_inner, tiles_q;
};

constexpr int kTile = 64;

// TQ: the tile's extent along q (64, or 32 when 64-wide tiles would give too
// few workgroups to keep every CU busy).
template <bool VIN, bool VOUT, int TQ>
__global__ __launch_bounds__(kThreads) void transpose_tile_kernel(const float* __restrict__ src,
                                                                  float* __restrict__ dst, const TileT g) {
  constexpr int Q4 = TQ / 4;           // float4 per input run
  constexpr int RP = kThreads / Q4;    // input runs per pass
  constexpr int OP = kThreads / 16;    // output runs per pass (16 float4 = 64 inner floats)
  __shared__ float tile[kTile][TQ + 1];
  uint32_t blk = blockIdx.x;
  const uint32_t ti = blk % g.tiles_inner;
  blk /= g.tiles_inner;
  const uint32_t tq = blk % g.tiles_q;
  uint32_t batch = blk / g.tiles_q;
  uint32_t in_base = 0, out_base = 0;
#pragma unroll
  for (int j = 1; j >= 0; --j) {
    if (j < g.nb) {
      uint32_t coord;
      batch = fdivmod(batch, g.bdiv[j], &coord);
      in_base += coord * g.b_in[j];
      out_base += coord * g.b_out[j];
    }
  }
  const uint32_t i0 = ti * kTile, q0 = tq * TQ;
  // Load: run (inner coordinate i0 + r) covers q0 .. q0 + TQ - 1.
  const int lq = threadIdx.x % Q4, lr = threadIdx.x / Q4;
#pragma unroll
  for (int pass = 0; pass < kTile / RP; ++pass) {
    const int r = lr + RP * pass;
    const uint32_t ic = i0 + r, qc = q0 + 4 * lq;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ic < g.n_inner) {
      const float* p = src + in_base + ic * g.in_st_inner + qc;
      if (VIN && qc + 3 < g.n_q) {
        const float4 w = *reinterpret_cast<const float4*>(p);
        v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (qc + u < g.n_q) v[u] = p[u];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) tile[r][4 * lq + u] = v[u];
  }
  __syncthreads();
  // Store: run (q coordinate q0 + r) covers i0 .. i0 + 63.
  const int lane4 = threadIdx.x & 15, row = threadIdx.x >> 4;
#pragma unroll
  for (int pass = 0; pass < TQ / OP; ++pass) {
    const int r = row + OP * pass;
    const uint32_t qc = q0 + r, ic = i0 + 4 * lane4;
    if (qc >= g.n_q) continue;
    float* p = dst + out_base + qc * g.out_st_q + ic;
    const float v0 = tile[4 * lane4][r], v1 = tile[4 * lane4 + 1][r], v2 = tile[4 * lane4 + 2][r],
                v3 = tile[4 * lane4 + 3][r];
    if (VOUT && ic + 3 < g.n_inner) {
      *reinterpret_cast<float4*>(p) = make_float4(v0, v1, v2, v3);
    } else {
      const float v[4] = {v0, v1, v2, v3};
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (ic + u < g.n_inner) p[u] = v[u];
    }
  }
}

// Any permutation (no axis contiguous in the input): one gather per element.
struct Gather4 {
  int rank;
  FastDiv div[4];
  uint32_t st[4];
};

__global__ __launch_bounds__(kThreads) void permute_flat_kernel(const float* __restrict__ src,
                                                                float* __restrict__ dst, const Gather4 g, uint32_t n) {
  uint32_t e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  const uint32_t out = e;
  uint32_t off = 0;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    if (j < g.rank) {
      uint32_t coord;
      e = fdivmod(e, g.div[j], &coord);
      off += coord * g.st[j];
    }
  }
  dst[out] = src[off];
}

// --------------------------------------------------------------- gather elements (op 37)

// Like permute_flat_kernel, but the coordinate along `axis` comes from the
// index tensor (float; negative counts from the end of an axis of length
// `axis_len`).  The index is data, so the source offset is clamped into the
// input (an out-of-range index reads an edge element instead of faulting).
struct GatherE {
  FastDiv div[4];
  uint32_t st[4];
  int axis;
  long long axis_len;
  long long src_len;
};

__global__ __launch_bounds__(kThreads) void gather_elements_kernel(const float* __restrict__ src,
                                                                   const float* __restrict__ idx,
                                                                   float* __restrict__ dst, const GatherE g,
                                                                   uint32_t n) {
  uint32_t e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  const uint32_t out = e;
  long long off = 0;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    uint32_t coord;
    e = fdivmod(e, g.div[j], &coord);
    long long c = coord;
    if (j == g.axis) {
      c = (long long)idx[out];
      if (c < 0) c += g.axis_len;
    }
    off += c * (long long)g.st[j];
  }
  off = off < 0 ? 0 : off >= g.src_len ? g.src_len - 1 : off;
  dst[out] = src[off];
}

// --------------------------------------------------------------- softmax (op 25), row maximum (op 36)

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Contiguous rows of `len` floats, one wave per row.  Up to 64 * PER values
// stay in registers between the passes; longer rows are read again.
template <int PER>
__global__ __launch_bounds__(kThreads) void softmax_rows_kernel(const float* __restrict__ src,
                                                                float* __restrict__ dst, uint32_t rows,
                                                                uint32_t len) {
  const uint32_t row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* x = src + (size_t)row * len;
  float* y = dst + (size_t)row * len;
  float v[PER];
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const uint32_t j = lane + 64 * u;
    v[u] = j < len ? x[j] : -INFINITY;
    m = fmaxf(m, v[u]);
  }
  for (uint32_t j = lane + 64 * PER; j < len; j += 64) m = fmaxf(m, x[j]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    v[u] = lane + 64 * u < len ? expf(v[u] - m) : 0.f;
    s += v[u];
  }
  for (uint32_t j = lane + 64 * PER; j < len; j += 64) s += expf(x[j] - m);
  s = wave_sum(s);
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (lane + 64 * u < len) y[lane + 64 * u] = v[u] / s;
  for (uint32_t j = lane + 64 * PER; j < len; j += 64) y[j] = expf(x[j] - m) / s;
}

// Softmax along an axis of stride `inner` (> 1): thread t owns column t
// (outer t / inner, position t % inner) and walks the axis; neighbouring
// threads read neighbouring floats.
__global__ __launch_bounds__(kThreads) void softmax_cols_kernel(const float* __restrict__ src,
                                                                float* __restrict__ dst, uint32_t cols,
                                                                uint32_t len, FastDiv inner) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= cols) return;
  uint32_t pos;
  const uint32_t outer = fdivmod(t, inner, &pos);
  const size_t base = (size_t)outer * len * inner.d + pos;
  const float* x = src + base;
  float* y = dst + base;
  float m = -INFINITY;
  for (uint32_t j = 0; j < len; ++j) m = fmaxf(m, x[(size_t)j * inner.d]);
  float s = 0.f;
  for (uint32_t j = 0; j < len; ++j) s += expf(x[(size_t)j * inner.d] - m);
  for (uint32_t j = 0; j < len; ++j) y[(size_t)j * inner.d] = expf(x[(size_t)j * inner.d] - m) / s;
}

// MathF.Max over a row: NaN wins, +0 beats -0, otherwise the larger value.
// The rule is associative and commutative, so a reduction tree gives the
// sequential result (up to which NaN payload is kept).
__device__ __forceinline__ float dotnet_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == b) return __uint_as_float(__float_as_uint(a) & __float_as_uint(b));  // +0 if either is +0
  return a > b ? a : b;
}

__global__ __launch_bounds__(kThreads) void row_max_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                           uint32_t rows, uint32_t len) {
  const uint32_t row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* x = src + (size_t)row * len;
  float m = -INFINITY;
  for (uint32_t j = lane; j < len; j += 64) m = dotnet_max(m, x[j]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = dotnet_max(m, __shfl_xor(m, o));
  if (lane == 0) dst[row] = m;
}

// --------------------------------------------------------------- spatial ops: one plane's pixels per workgroup

// Launch shape shared by the per-plane kernels: `planes` output planes of
// `plane` pixels, ceil(plane / 256) workgroups per plane; `n` pixels in all
// (the last plane may be partial).
struct Planes {
  uint32_t plane, per_plane, n;
  FastDiv width;  // output row length
};

__device__ __forceinline__ bool plane_pixel(const Planes& g, uint32_t* p, uint32_t* oy, uint32_t* ox, uint32_t* e) {
  *p = blockIdx.x / g.per_plane;
  const uint32_t local = (blockIdx.x - *p * g.per_plane) * kThreads + threadIdx.x;
  *e = *p * g.plane + local;
  if (local >= g.plane || *e >= g.n) return false;
  *oy = fdivmod(local, g.width, ox);
  return true;
}

// Op 20, nearest resize: out[p][oy][ox] = in[p][oy * ih / oh][ox * iw / ow].
__global__ __launch_bounds__(kThreads) void resize_nearest_kernel(const float* __restrict__ src,
                                                                  float* __restrict__ dst, const Planes g,
                                                                  uint32_t ih, uint32_t iw, FastDiv oh,
                                                                  FastDiv ow) {
  uint32_t p, oy, ox, e;
  if (!plane_pixel(g, &p, &oy, &ox, &e)) return;
  const uint32_t sy = fdiv(oy * ih, oh), sx = fdiv(ox * iw, ow);
  dst[e] = src[((size_t)p * ih + sy) * iw + sx];
}

// Ops 21 / 22: max (IEEE maximum: NaN propagates) or average pool with
// padding excluded from the maximum; the average divides by the window
// (count_include_pad) or by the taps inside the input.
template <bool AVG>
__global__ __launch_bounds__(kThreads) void pool_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                        const Planes g, int ih, int iw, int kh, int kw, int sh,
                                                        int sw, int pt, int pl, int include_pad) {
  uint32_t p, oy, ox, e;
  if (!plane_pixel(g, &p, &oy, &ox, &e)) return;
  const float* x = src + (size_t)p * ih * iw;
  const int y0 = (int)oy * sh - pt, x0 = (int)ox * sw - pl;
  const int ya = max(y0, 0), yb = min(y0 + kh, ih), xa = max(x0, 0), xb = min(x0 + kw, iw);
  float acc = AVG ? 0.f : -INFINITY;
  for (int y = ya; y < yb; ++y)
    for (int xx = xa; xx < xb; ++xx) {
      const float v = x[y * iw + xx];
      acc = AVG ? acc + v : __builtin_elementwise_maximum(acc, v);
    }
  if constexpr (AVG) {
    const int taps = max(yb - ya, 0) * max(xb - xa, 0);
    acc = acc / (float)(include_pad ? kh * kw : taps);
  }
  dst[e] = acc;
}

// Op 32: depthwise conv over NCHW planes (input plane p = b * C + ch), weights
// [C][kh][kw] and an optional bias; SiLU on request.
__global__ __launch_bounds__(kThreads) void depthwise_nchw_kernel(const float* __restrict__ src,
                                                                  const float* __restrict__ wts,
                                                                  const float* __restrict__ bias,
                                                                  float* __restrict__ dst, const Planes g,
                                                                  uint32_t channels, int ih, int iw, int kh, int kw,
                                                                  int sh, int sw, int pt, int pl, int dh, int dw,
                                                                  int silu) {
  uint32_t p, oy, ox, e;
  if (!plane_pixel(g, &p, &oy, &ox, &e)) return;
  const uint32_t ch = p % channels;
  const float* x = src + (size_t)p * ih * iw;
  const float* w = wts + (size_t)ch * kh * kw;
  float acc = bias ? bias[ch] : 0.f;
  const int y0 = (int)oy * sh - pt, x0 = (int)ox * sw - pl;
  for (int ky = 0; ky < kh; ++ky) {
    const int y = y0 + ky * dh;
    if (y < 0 || y >= ih) continue;
    for (int kx = 0; kx < kw; ++kx) {
      const int xx = x0 + kx * dw;
      if (xx >= 0 && xx < iw) acc += x[y * iw + xx] * w[ky * kw + kx];
    }
  }
  dst[e] = silu ? acc * logistic(acc) : acc;
}

// Op 33: transposed conv.  Output plane p = b * oc + co; input channels of
// co's group; weights [ic][oc / groups][kh][kw]; an optional bias.  Tap
// (ky, kx) reads input (y, x) with y * sh = oy + pt - ky * dh (and alike in
// x) when that divides exactly.
__global__ __launch_bounds__(kThreads) void conv_transpose_kernel(const float* __restrict__ src,
                                                                  const float* __restrict__ wts,
                                                                  const float* __restrict__ bias,
                                                                  float* __restrict__ dst, const Planes g, int ic,
                                                                  int ih, int iw, int oc, int kh, int kw, int sh,
                                                                  int sw, int pt, int pl, int dh, int dw,
                                                                  int groups) {
  uint32_t p, oy, ox, e;
  if (!plane_pixel(g, &p, &oy, &ox, &e)) return;
  const int co = (int)(p % (uint32_t)oc), b = (int)(p / (uint32_t)oc);
  const int cog = oc / groups, cig = ic / groups, grp = co / cog, col = co - grp * cog;
  float acc = bias ? bias[co] : 0.f;
  const size_t plane_in = (size_t)ih * iw;
  const float* xb = src + ((size_t)b * ic + (size_t)grp * cig) * plane_in;
  const float* wb = wts + ((size_t)grp * cig * cog + col) * kh * kw;
  for (int ky = 0; ky < kh; ++ky) {
    const int yn = (int)oy + pt - ky * dh;
    if (yn < 0 || yn % sh) continue;
    const int y = yn / sh;
    if (y >= ih) continue;
    for (int kx = 0; kx < kw; ++kx) {
      const int xn = (int)ox + pl - kx * dw;
      if (xn < 0 || xn % sw) continue;
      const int xx = xn / sw;
      if (xx >= iw) continue;
      const float* xp = xb + (size_t)y * iw + xx;
      const float* wp = wb + ky * kw + kx;
      for (int q = 0; q < cig; ++q) acc += xp[q * plane_in] * wp[(size_t)q * cog * kh * kw];
    }
  }
  dst[e] = acc;
}

// Op 35: depth to space by 2.  Output plane p = b * C + co, pixel (y, x)
// comes from input channel 4 co + 2 (y & 1) + (x & 1) at (y / 2, x / 2).
__global__ __launch_bounds__(kThreads) void depth_to_space_kernel(const float* __restrict__ src,
                                                                  float* __restrict__ dst, const Planes g, int h,
                                                                  int w) {
  uint32_t p, y, x, e;
  if (!plane_pixel(g, &p, &y, &x, &e)) return;
  const int hh = h / 2, wh = w / 2;
  const size_t sub = (size_t)p * 4 + (y & 1) * 2 + (x & 1);
  dst[e] = src[(sub * hh + (y >> 1)) * wh + (x >> 1)];
}

// --------------------------------------------------------------- head decodes (ops 30, 31, 34)

// Softmax expectation sum_j j softmax(l)_j over `bins` logits l_j = x[j * step].
template <int BINS>
__device__ __forceinline__ float dfl_expect(const float* x, uint32_t step, int bins) {
  const int nb = BINS > 0 ? BINS : bins;
  if (nb == 1) return x[0];
  if constexpr (BINS > 0) {
    float l[BINS];
#pragma unroll
    for (int j = 0; j < BINS; ++j) l[j] = x[(size_t)j * step];
    float m = l[0];
#pragma unroll
    for (int j = 1; j < BINS; ++j) m = fmaxf(m, l[j]);
    float s = 0.f, num = 0.f;
#pragma unroll
    for (int j = 0; j < BINS; ++j) {
      const float q = expf(l[j] - m);
      s += q;
      num += q * (float)j;
    }
    return num / s;
  } else {
    float m = -INFINITY;
    for (int j = 0; j < nb; ++j) m = fmaxf(m, x[(size_t)j * step]);
    float s = 0.f, num = 0.f;
    for (int j = 0; j < nb; ++j) {
      const float q = expf(x[(size_t)j * step] - m);
      s += q;
      num += q * (float)j;
    }
    return num / s;
  }
}

// Op 30: one level of a detect head, one thread per (image, anchor) of the
// level: boxes [B][4 bins][sp], scores [B][nc][sp] -> rows of the joined
// [B][nc + 4][os] output at anchor offset `a0` (x, y, w, h or x1, y1, x2, y2
// in pixels, then the class sigmoids).
struct LevelDecode {
  FastDiv spatial, width;
  uint32_t n, bins, nc, os, a0;
  float stride;
  int xyxy;
};

template <int BINS>
__global__ __launch_bounds__(kThreads) void level_decode_kernel(const float* __restrict__ boxes,
                                                                const float* __restrict__ scores,
                                                                float* __restrict__ out, const LevelDecode g) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= g.n) return;
  uint32_t anchor, col;
  const uint32_t b = fdivmod(t, g.spatial, &anchor);
  const uint32_t row = fdivmod(anchor, g.width, &col);
  const uint32_t sp = g.spatial.d;
  const float* bx = boxes + (size_t)b * 4 * g.bins * sp + anchor;
  float d[4];
#pragma unroll
  for (int side = 0; side < 4; ++side) d[side] = dfl_expect<BINS>(bx + (size_t)side * g.bins * sp, sp, (int)g.bins);
  const float cx = (float)col + .5f, cy = (float)row + .5f;
  const float x1 = (cx - d[0]) * g.stride, y1 = (cy - d[1]) * g.stride;
  const float x2 = (cx + d[2]) * g.stride, y2 = (cy + d[3]) * g.stride;
  float* o = out + (size_t)b * (g.nc + 4) * g.os + g.a0 + anchor;
  if (g.xyxy) {
    o[0] = x1;
    o[g.os] = y1;
    o[2 * (size_t)g.os] = x2;
    o[3 * (size_t)g.os] = y2;
  } else {
    o[0] = (x1 + x2) * .5f;
    o[g.os] = (y1 + y2) * .5f;
    o[2 * (size_t)g.os] = x2 - x1;
    o[3 * (size_t)g.os] = y2 - y1;
  }
  const float* sc = scores + (size_t)b * g.nc * sp + anchor;
  for (uint32_t j = 0; j < g.nc; ++j) o[(size_t)(4 + j) * g.os] = logistic(sc[(size_t)j * sp]);
}

// Op 34: the DFL expectation alone, [B][4 bins][sp] -> [B][4][sp].
template <int BINS>
__global__ __launch_bounds__(kThreads) void dfl_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                       FastDiv spatial, uint32_t bins, uint32_t n) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= n) return;
  uint32_t a;
  const uint32_t row = fdivmod(t, spatial, &a);  // row = b * 4 + side
  dst[t] = dfl_expect<BINS>(src + (size_t)row * bins * spatial.d + a, spatial.d, (int)bins);
}

// Op 31: pose keypoints [B][K * dim][sp] in place of layout: x and y become
// pixels ((v * f + cell + o) * stride; YOLO26: f = 1, o = .5, else f = 2,
// o = 0), the other fields their sigmoid.
__global__ __launch_bounds__(kThreads) void pose_decode_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                               FastDiv spatial, FastDiv dim, FastDiv width,
                                                               float stride, float factor, float offset, uint32_t n) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= n) return;
  uint32_t anchor, field, col;
  const uint32_t rowk = fdivmod(t, spatial, &anchor);
  fdivmod(rowk, dim, &field);
  const uint32_t row = fdivmod(anchor, width, &col);
  const float v = src[t];
  float y;
  if (field == 0) y = (v * factor + ((float)col + offset)) * stride;
  else if (field == 1) y = (v * factor + ((float)row + offset)) * stride;
  else y = logistic(v);
  dst[t] = y;
}

// --------------------------------------------------------------- host: decode, check, launch

// Parameter block as read by the host: P[i], binding lengths and offsets.
struct Block {
  uint32_t P[32];
  const float *a, *b, *d;
  float* c;
  long long la, lb, ld, lc;  // lengths in floats (0: not bound)
  long long items;
};

// Highest offset reached by flat elements [0, n) of a collapsed strided
// view (0 for an empty view).
static long long span_max(int rank, const uint32_t* size, const uint32_t* st) {
  long long m = 0;
  for (int j = 0; j < rank; ++j) m += (long long)(size[j] - 1) * st[j];
  return m;
}

// Drops size-1 axes and merges axis j into j + 1 where every operand's
// stride satisfies st[j] == st[j + 1] * size[j + 1] (the pair is one run).
// `ops` stride arrays of length 4 (outer first); returns the new rank.
static int collapse(uint32_t* size, std::vector<uint32_t*> ops, int rank) {
  int r = 0;
  uint32_t sz[4];
  std::vector<std::vector<uint32_t>> st(ops.size(), std::vector<uint32_t>(4));
  for (int j = 0; j < rank; ++j) {
    if (size[j] == 1) continue;
    if (r > 0) {
      bool merge = true;
      for (size_t o = 0; o < ops.size(); ++o)
        merge &= (unsigned long long)st[o][r - 1] == (unsigned long long)ops[o][j] * size[j];
      if (merge) {
        sz[r - 1] *= size[j];
        for (size_t o = 0; o < ops.size(); ++o) st[o][r - 1] = ops[o][j];
        continue;
      }
    }
    sz[r] = size[j];
    for (size_t o = 0; o < ops.size(); ++o) st[o][r] = ops[o][j];
    ++r;
  }
  if (r == 0) {  // a single element
    sz[0] = 1;
    for (size_t o = 0; o < ops.size(); ++o) st[o][0] = 0;
    r = 1;
  }
  for (int j = 0; j < r; ++j) {
    size[j] = sz[j];
    for (size_t o = 0; o < ops.size(); ++o) ops[o][j] = st[o][j];
  }
  return r;
}

static long long shape_count(const uint32_t* P) { return (long long)P[1] * P[2] * P[3] * P[4]; }

static int launch_unary(sy_ctx* ctx, const Block& k, int op) {
  SY_CHECK((long long)k.P[28] + k.items <= k.la && (long long)k.P[30] + k.items <= k.lc, SY_EINVAL,
           "op %d: work items exceed a buffer", op);
  const float* a = k.a + k.P[28];
  float* c = k.c + k.P[30];
  const float alpha = bits_to_float(k.P[1]);
  const uint32_t n = (uint32_t)k.items;
  const bool vec = aligned16(a) && aligned16(c);
  ProfScope prof(ctx, "compute_unary", 0, 8.0 * n);
  const unsigned grid = grid_for(vec ? (n + 3) / 4 : n);
#define SY_UNARY(OP)                                                                               \
  case OP:                                                                                         \
    if (vec) hipLaunchKernelGGL((unary_kernel<OP, true>), dim3(grid), dim3(kThreads), 0, ctx->stream, a, c, n, alpha); \
    else hipLaunchKernelGGL((unary_kernel<OP, false>), dim3(grid), dim3(kThreads), 0, ctx->stream, a, c, n, alpha); \
    break;
  switch (op) {
    SY_UNARY(1) SY_UNARY(2) SY_UNARY(3) SY_UNARY(4) SY_UNARY(5) SY_UNARY(6) SY_UNARY(7) SY_UNARY(8) SY_UNARY(9)
  }
#undef SY_UNARY
  return check_launch("compute_unary");
}

static int launch_binary(sy_ctx* ctx, const Block& k, int op) {
  const uint32_t* P = k.P;
  SY_CHECK(P[1] && P[2] && P[3] && P[4], SY_EINVAL, "op %d needs a positive 4-d shape", op);
  SY_CHECK(k.items == shape_count(P), SY_EINVAL, "op %d: work items %lld differ from the shape's %lld elements", op,
           k.items, shape_count(P));
  Bcast g{};
  uint32_t size[4] = {P[1], P[2], P[3], P[4]}, sa[4] = {P[5], P[6], P[7], P[8]}, sb[4] = {P[9], P[10], P[11], P[12]};
  SY_CHECK(P[28] + span_max(4, size, sa) < k.la && P[29] + span_max(4, size, sb) < k.lb, SY_EINVAL,
           "broadcast strides reach past an input");
  SY_CHECK((long long)P[30] + k.items <= k.lc, SY_EINVAL, "broadcast output exceeds its buffer");
  g.rank = collapse(size, {sa, sb}, 4);
  for (int j = 0; j < g.rank; ++j) {
    g.size[j] = size[j];
    g.div[j] = make_div(size[j]);
    g.sa[j] = sa[j];
    g.sb[j] = sb[j];
  }
  const float* a = k.a + P[28];
  const float* b = k.b + P[29];
  float* c = k.c + P[30];
  const uint32_t n = (uint32_t)k.items;
  // float4 path: inner axis a multiple of 4 with unit or zero strides, every
  // other stride of a unit-stride operand a multiple of 4, aligned bases.
  const int in = g.rank - 1;
  bool vec = g.size[in] % 4 == 0 && aligned16(c);
  for (int o = 0; o < 2; ++o) {
    const uint32_t* st = o ? g.sb : g.sa;
    const float* base = o ? b : a;
    if (st[in] > 1) vec = false;
    if (st[in] == 1) {
      vec &= aligned16(base);
      for (int j = 0; j < in; ++j) vec &= st[j] % 4 == 0;
    }
  }
  ProfScope prof(ctx, "compute_binary", 0, 12.0 * n);
#define SY_BINARY(OP)                                                                                         \
  case OP:                                                                                                    \
    if (vec) hipLaunchKernelGGL((binary_vec_kernel<OP>), dim3(grid_for(n / 4)), dim3(kThreads), 0, ctx->stream, a, b, \
                                c, g, n / 4);                                                                 \
    else hipLaunchKernelGGL((binary_flat_kernel<OP>), dim3(grid_for(n)), dim3(kThreads), 0, ctx->stream, a, b, c, g, \
                            n);                                                                               \
    break;
  switch (op) {
    SY_BINARY(10) SY_BINARY(11) SY_BINARY(12) SY_BINARY(13) SY_BINARY(14) SY_BINARY(15) SY_BINARY(16)
  }
#undef SY_BINARY
  return check_launch("compute_binary");
}

// Row copies: rows of `len` floats, `n` floats in all; row r reads from
// src + base(r) (outer axes `osize` / `ost`, outer first) and writes to
// dst + r * dst_row.
static int launch_rows(sy_ctx* ctx, const float* src, float* dst, int outer_rank, const uint32_t* osize,
                       const uint32_t* ost, uint32_t len, uint32_t dst_row, uint32_t n, const char* name) {
  RowCopy g{};
  g.outer_rank = outer_rank;
  bool vec = len % 4 == 0 && dst_row % 4 == 0 && aligned16(src) && aligned16(dst) && n % 4 == 0;
  for (int j = 0; j < outer_rank; ++j) {
    g.odiv[j] = make_div(osize[j]);
    g.ost[j] = ost[j];
    vec &= ost[j] % 4 == 0;
  }
  g.len = make_div(len);
  g.dst_row = dst_row;
  g.n = n;
  ProfScope prof(ctx, name, 0, 8.0 * n);
  if (vec)
    hipLaunchKernelGGL(row_copy_kernel<true>, dim3(grid_for(n / 4)), dim3(kThreads), 0, ctx->stream, src, dst, g);
  else
    hipLaunchKernelGGL(row_copy_kernel<false>, dim3(grid_for(n)), dim3(kThreads), 0, ctx->stream, src, dst, g);
  return check_launch(name);
}

static int launch_transpose(sy_ctx* ctx, const Block& k) {
  const uint32_t* P = k.P;
  SY_CHECK(P[1] && P[2] && P[3] && P[4], SY_EINVAL, "op 23 needs a positive 4-d shape");
  SY_CHECK(k.items <= shape_count(P), SY_EINVAL, "op 23: more work items than the shape holds");
  uint32_t size[4] = {P[1], P[2], P[3], P[4]}, st[4] = {P[5], P[6], P[7], P[8]};
  SY_CHECK(P[28] + span_max(4, size, st) < k.la && (long long)P[30] + k.items <= k.lc, SY_EINVAL,
           "transpose extents exceed a buffer");
  // Output strides are the dense ones; collapse both together.
  uint32_t ost[4] = {P[2] * P[3] * P[4], P[3] * P[4], P[4], 1};
  const int rank = collapse(size, {st, ost}, 4);
  const float* a = k.a + P[28];
  float* c = k.c + P[30];
  const uint32_t n = (uint32_t)k.items;
  const int in = rank - 1;
  if (st[in] == 1) {  // inner runs contiguous in the input: row gathers
    return launch_rows(ctx, a, c, in, size, st, size[in], size[in], n, "compute_transpose_rows");
  }
  int q = -1;
  for (int j = 0; j < in; ++j)
    if (st[j] == 1) q = j;
  if (q >= 0 && k.items == shape_count(P)) {
    TileT g{};
    g.n_inner = size[in];
    g.n_q = size[q];
    g.in_st_inner = st[in];
    g.out_st_q = ost[q];
    for (int j = 0; j < in; ++j) {
      if (j == q) continue;
      g.bdiv[g.nb] = make_div(size[j]);
      g.b_in[g.nb] = st[j];
      g.b_out[g.nb] = ost[j];
      ++g.nb;
    }
    long long batches = 1;
    for (int j = 0; j < g.nb; ++j) batches *= g.bdiv[j].d;
    g.tiles_inner = (g.n_inner + kTile - 1) / kTile;
    // 64 x 64 tiles unless that leaves under four workgroups per CU.
    const bool narrow = (long long)g.tiles_inner * ((g.n_q + kTile - 1) / kTile) * batches < 4LL * ctx->cu_count;
    const int tq = narrow ? 32 : kTile;
    g.tiles_q = (g.n_q + tq - 1) / tq;
    const long long blocks = (long long)g.tiles_inner * g.tiles_q * batches;
    bool vin = g.in_st_inner % 4 == 0 && aligned16(a), vout = g.out_st_q % 4 == 0 && aligned16(c);
    for (int j = 0; j < g.nb; ++j) {
      vin &= g.b_in[j] % 4 == 0;
      vout &= g.b_out[j] % 4 == 0;
    }
    ProfScope prof(ctx, "compute_transpose_tiled", 0, 8.0 * n);
    const dim3 grid((unsigned)blocks);
#define SY_TILE(VI, VO)                                                                                          \
  do {                                                                                                           \
    if (narrow)                                                                                                  \
      hipLaunchKernelGGL((transpose_tile_kernel<VI, VO, 32>), grid, dim3(kThreads), 0, ctx->stream, a, c, g);   \
    else                                                                                                         \
      hipLaunchKernelGGL((transpose_tile_kernel<VI, VO, kTile>), grid, dim3(kThreads), 0, ctx->stream, a, c, g); \
  } while (0)
    if (vin && vout) SY_TILE(true, true);
    else if (vin) SY_TILE(true, false);
    else if (vout) SY_TILE(false, true);
    else SY_TILE(false, false);
#undef SY_TILE
    return check_launch("compute_transpose_tiled");
  }
  Gather4 g{};
  g.rank = rank;
  for (int j = 0; j < rank; ++j) {
    g.div[j] = make_div(size[j]);
    g.st[j] = st[j];
  }
  ProfScope prof(ctx, "compute_transpose_flat", 0, 8.0 * n);
  hipLaunchKernelGGL(permute_flat_kernel, dim3(grid_for(n)), dim3(kThreads), 0, ctx->stream, a, c, g, n);
  return check_launch("compute_transpose_flat");
}

// Highest destination (or source) offset of a strided row copy: element i of
// rows of `len` lands at (i / len) * row + (i % len); the maximum over i < n
// is the last element or the end of the row before it.
static long long rows_extent(long long n, long long len, long long row) {
  if (n <= 0) return -1;
  const long long last = n - 1, r = last / len;
  long long m = r * row + last % len;
  if (r > 0) m = std::max(m, (r - 1) * row + len - 1);
  return m;
}

static int launch_slice(sy_ctx* ctx, const Block& k) {  // op 24
  const uint32_t* P = k.P;
  SY_CHECK(P[2] > 0 && P[3] > 0, SY_EINVAL, "slice needs axis and inner sizes");
  const long long len = (long long)P[2] * P[3], srow = (long long)P[1] * P[3], soff = (long long)P[4] * P[3] + P[28];
  SY_CHECK(len <= kMaxItems && srow <= kMaxItems && soff <= kMaxItems, SY_EUNSUPPORTED, "slice rows too long");
  SY_CHECK(soff + rows_extent(k.items, len, srow) < k.la && (long long)P[30] + k.items <= k.lc, SY_EINVAL,
           "slice extents exceed a buffer");
  const uint32_t osize[1] = {(uint32_t)((k.items + len - 1) / len)}, ost[1] = {(uint32_t)srow};
  return launch_rows(ctx, k.a + soff, k.c + P[30], 1, osize, ost, (uint32_t)len, (uint32_t)len, (uint32_t)k.items,
                     "compute_slice");
}

static int launch_concat(sy_ctx* ctx, const Block& k) {  // op 26
  const uint32_t* P = k.P;
  SY_CHECK(P[1] > 0 && P[3] > 0, SY_EINVAL, "concat needs axis and inner sizes");
  const long long len = (long long)P[1] * P[3], drow = (long long)P[2] * P[3], doff = (long long)P[4] * P[3] + P[30];
  SY_CHECK(len <= kMaxItems && drow <= kMaxItems && doff <= kMaxItems, SY_EUNSUPPORTED, "concat rows too long");
  SY_CHECK((long long)P[28] + k.items <= k.la && doff + rows_extent(k.items, len, drow) < k.lc, SY_EINVAL,
           "concat extents exceed a buffer");
  const uint32_t osize[1] = {(uint32_t)((k.items + len - 1) / len)}, ost[1] = {(uint32_t)len};
  return launch_rows(ctx, k.a + P[28], k.c + doff, 1, osize, ost, (uint32_t)len, (uint32_t)drow, (uint32_t)k.items,
                     "compute_concat");
}

static int launch_softmax(sy_ctx* ctx, const Block& k) {  // op 25: one work item per row
  const uint32_t* P = k.P;
  const long long len = P[1], inner = P[2];
  SY_CHECK(len > 0 && inner > 0, SY_EINVAL, "softmax needs the axis and inner sizes");
  // Row i starts at (i / inner) * len * inner + i % inner; the last row ends last.
  const long long last = k.items == 0 ? -1 : (k.items - 1) / inner * len * inner + (k.items - 1) % inner + (len - 1) * inner;
  SY_CHECK(last < kMaxItems, SY_EUNSUPPORTED, "softmax extents beyond 2^31 elements");
  SY_CHECK(P[28] + last < k.la && P[30] + last < k.lc, SY_EINVAL, "softmax extents exceed a buffer");
  const float* a = k.a + P[28];
  float* c = k.c + P[30];
  const uint32_t rows = (uint32_t)k.items;
  ProfScope prof(ctx, "compute_softmax", 0, 8.0 * (double)k.items * len);
  if (inner == 1) {
    const unsigned grid = (unsigned)((rows + 3) / 4);
    if (len <= 64) hipLaunchKernelGGL(softmax_rows_kernel<1>, dim3(grid), dim3(kThreads), 0, ctx->stream, a, c, rows, (uint32_t)len);
    else if (len <= 256) hipLaunchKernelGGL(softmax_rows_kernel<4>, dim3(grid), dim3(kThreads), 0, ctx->stream, a, c, rows, (uint32_t)len);
    else hipLaunchKernelGGL(softmax_rows_kernel<8>, dim3(grid), dim3(kThreads), 0, ctx->stream, a, c, rows, (uint32_t)len);
  } else {
    hipLaunchKernelGGL(softmax_cols_kernel, dim3(grid_for(rows)), dim3(kThreads), 0, ctx->stream, a, c, rows,
                       (uint32_t)len, make_div((uint32_t)inner));
  }
  return check_launch("compute_softmax");
}

static int launch_row_max(sy_ctx* ctx, const Block& k) {  // op 36
  const long long len = k.P[1];
  SY_CHECK(len > 0, SY_EINVAL, "row max needs the row length");
  SY_CHECK(k.items * len <= kMaxItems, SY_EUNSUPPORTED, "row max beyond 2^31 elements");
  SY_CHECK(k.P[28] + k.items * len <= k.la && (long long)k.P[30] + k.items <= k.lc, SY_EINVAL,
           "row max extents exceed a buffer");
  ProfScope prof(ctx, "compute_row_max", 0, 4.0 * (double)k.items * (len + 1));
  hipLaunchKernelGGL(row_max_kernel, dim3((unsigned)((k.items + 3) / 4)), dim3(kThreads), 0, ctx->stream,
                     k.a + k.P[28], k.c + k.P[30], (uint32_t)k.items, (uint32_t)len);
  return check_launch("compute_row_max");
}

static int launch_gather(sy_ctx* ctx, const Block& k) {  // op 37
  const uint32_t* P = k.P;
  SY_CHECK(P[1] && P[2] && P[3] && P[4], SY_EINVAL, "op 37 needs a positive 4-d shape");
  SY_CHECK(P[9] < 4, SY_EINVAL, "gather axis out of range");
  SY_CHECK(k.items <= shape_count(P), SY_EINVAL, "op 37: more work items than the shape holds");
  SY_CHECK((long long)P[29] + k.items <= k.lb && (long long)P[30] + k.items <= k.lc, SY_EINVAL,
           "gather extents exceed a buffer");
  GatherE g{};
  for (int j = 0; j < 4; ++j) {
    g.div[j] = make_div(P[1 + j]);
    g.st[j] = P[5 + j];
  }
  g.axis = (int)P[9];
  g.axis_len = P[10];
  g.src_len = k.la - P[28];
  SY_CHECK(g.src_len > 0, SY_EINVAL, "gather input offset past its buffer");
  ProfScope prof(ctx, "compute_gather", 0, 12.0 * (double)k.items);
  hipLaunchKernelGGL(gather_elements_kernel, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, k.a + P[28],
                     k.b + P[29], k.c + P[30], g, (uint32_t)k.items);
  return check_launch("compute_gather");
}

static Planes make_planes(long long items, uint32_t oh, uint32_t ow) {
  Planes g{};
  g.plane = oh * ow;
  g.per_plane = (g.plane + kThreads - 1) / kThreads;
  g.n = (uint32_t)items;
  g.width = make_div(ow);
  return g;
}

static unsigned plane_grid(const Planes& g) {
  const long long planes = ((long long)g.n + g.plane - 1) / g.plane;
  return (unsigned)(planes * g.per_plane);
}

static int launch_spatial(sy_ctx* ctx, const Block& k, int op) {
  const uint32_t* P = k.P;
  const float* a = k.a + P[28];
  float* c = k.c + P[30];
  SY_CHECK((long long)P[30] + k.items <= k.lc, SY_EINVAL, "op %d output exceeds its buffer", op);
  if (op == 20 || op == 21 || op == 22) {
    SY_CHECK(P[1] > 0 && P[2] > 0 && P[3] > 0 && P[4] > 0, SY_EINVAL, "spatial op needs its input and output sizes");
    const long long plane = (long long)P[3] * P[4], planes = (k.items + plane - 1) / plane;
    SY_CHECK(plane <= kMaxItems && (long long)P[3] * P[1] <= kMaxItems && (long long)P[4] * P[2] <= kMaxItems,
             SY_EUNSUPPORTED, "spatial op sizes beyond 2^31");
    SY_CHECK(P[28] + planes * P[1] * P[2] <= k.la, SY_EINVAL, "op %d input planes exceed the buffer", op);
    const Planes g = make_planes(k.items, P[3], P[4]);
    if (op == 20) {
      ProfScope prof(ctx, "compute_resize", 0, 8.0 * (double)k.items);
      hipLaunchKernelGGL(resize_nearest_kernel, dim3(plane_grid(g)), dim3(kThreads), 0, ctx->stream, a, c, g, P[1],
                         P[2], make_div(P[3]), make_div(P[4]));
      return check_launch("compute_resize");
    }
    SY_CHECK(P[5] > 0 && P[6] > 0 && P[7] > 0 && P[8] > 0, SY_EINVAL, "pool needs its window and strides");
    ProfScope prof(ctx, op == 21 ? "compute_maxpool" : "compute_avgpool", 0,
                   4.0 * (double)(planes * P[1] * P[2] + k.items));
    if (op == 21)
      hipLaunchKernelGGL(pool_kernel<false>, dim3(plane_grid(g)), dim3(kThreads), 0, ctx->stream, a, c, g, (int)P[1],
                         (int)P[2], (int)P[5], (int)P[6], (int)P[7], (int)P[8], (int)P[9], (int)P[10], 0);
    else
      hipLaunchKernelGGL(pool_kernel<true>, dim3(plane_grid(g)), dim3(kThreads), 0, ctx->stream, a, c, g, (int)P[1],
                         (int)P[2], (int)P[5], (int)P[6], (int)P[7], (int)P[8], (int)P[9], (int)P[10],
                         P[11] == 1 ? 1 : 0);
    return check_launch("compute_pool");
  }
  if (op == 32 || op == 33) {
    const long long ic = P[1], ih = P[2], iw = P[3], oh = P[5], ow = P[6], kh = P[7], kw = P[8];
    SY_CHECK(ic > 0 && ih > 0 && iw > 0 && oh > 0 && ow > 0 && kh > 0 && kw > 0 && P[9] > 0 && P[10] > 0 &&
                 P[13] > 0 && P[14] > 0,
             SY_EINVAL, "conv op needs channels, sizes, strides and dilations");
    SY_CHECK(oh * ow <= kMaxItems && ih * iw <= kMaxItems, SY_EUNSUPPORTED, "conv planes beyond 2^31");
    const Planes g = make_planes(k.items, (uint32_t)oh, (uint32_t)ow);
    const long long planes = (k.items + g.plane - 1) / g.plane;
    const float* bias = k.d ? k.d + P[31] : nullptr;
    if (op == 32) {
      SY_CHECK(P[28] + planes * ih * iw <= k.la, SY_EINVAL, "depthwise input exceeds its buffer");
      SY_CHECK(k.b && P[29] + ic * kh * kw <= k.lb, SY_EINVAL, "depthwise weights exceed their buffer");
      SY_CHECK(!k.d || P[31] + ic <= k.ld, SY_EINVAL, "depthwise bias exceeds its buffer");
      ProfScope prof(ctx, "compute_depthwise", 2.0 * (double)k.items * kh * kw,
                     4.0 * (double)(planes * ih * iw + k.items));
      hipLaunchKernelGGL(depthwise_nchw_kernel, dim3(plane_grid(g)), dim3(kThreads), 0, ctx->stream, a, k.b + P[29],
                         bias, c, g, (uint32_t)ic, (int)ih, (int)iw, (int)kh, (int)kw, (int)P[9], (int)P[10],
                         (int)P[11], (int)P[12], (int)P[13], (int)P[14], P[16] == 1 ? 1 : 0);
      return check_launch("compute_depthwise");
    }
    const long long oc = P[4], groups = P[15] ? P[15] : 1;
    SY_CHECK(oc > 0 && ic % groups == 0 && oc % groups == 0, SY_EINVAL, "channels not divisible by groups");
    const long long images = (planes + oc - 1) / oc;
    SY_CHECK(P[28] + images * ic * ih * iw <= k.la, SY_EINVAL, "transposed conv input exceeds its buffer");
    SY_CHECK(k.b && P[29] + ic * (oc / groups) * kh * kw <= k.lb, SY_EINVAL,
             "transposed conv weights exceed their buffer");
    SY_CHECK(!k.d || P[31] + oc <= k.ld, SY_EINVAL, "transposed conv bias exceeds its buffer");
    ProfScope prof(ctx, "compute_conv_transpose", 2.0 * (double)k.items * (ic / groups) * kh * kw,
                   4.0 * (double)(images * ic * ih * iw + k.items));
    hipLaunchKernelGGL(conv_transpose_kernel, dim3(plane_grid(g)), dim3(kThreads), 0, ctx->stream, a, k.b + P[29],
                       bias, c, g, (int)ic, (int)ih, (int)iw, (int)oc, (int)kh, (int)kw, (int)P[9], (int)P[10],
                       (int)P[11], (int)P[12], (int)P[13], (int)P[14], (int)groups);
    return check_launch("compute_conv_transpose");
  }
  // op 35
  const long long h = P[1], w = P[2], ch = P[3];
  SY_CHECK(h > 0 && w > 0 && ch > 0, SY_EINVAL, "depth-to-space needs its shape");
  SY_CHECK(h * w <= kMaxItems, SY_EUNSUPPORTED, "depth-to-space plane beyond 2^31");
  const Planes g = make_planes(k.items, (uint32_t)h, (uint32_t)w);
  const long long planes = (k.items + g.plane - 1) / g.plane;
  // Sub-plane s holds (h / 2) x (w / 2) floats; the last pixel of the last
  // output plane reads sub-plane 4 planes - 1 at ((h - 1) / 2, (w - 1) / 2).
  const long long last = ((4 * planes - 1) * (h / 2) + (h - 1) / 2) * (w / 2) + (w - 1) / 2;
  SY_CHECK(P[28] + last < k.la, SY_EINVAL, "depth-to-space input exceeds its buffer");
  ProfScope prof(ctx, "compute_depth_to_space", 0, 8.0 * (double)k.items);
  hipLaunchKernelGGL(depth_to_space_kernel, dim3(plane_grid(g)), dim3(kThreads), 0, ctx->stream, a, c, g, (int)h,
                     (int)w);
  return check_launch("compute_depth_to_space");
}

static int launch_decode(sy_ctx* ctx, const Block& k, int op) {
  const uint32_t* P = k.P;
  const float* a = k.a + P[28];
  float* c = k.c + P[30];
  const long long spatial = P[1];
  if (op == 34) {
    const long long bins = P[2];
    SY_CHECK(spatial > 0 && bins > 0, SY_EINVAL, "decode needs spatial and bins");
    const long long rows = (k.items + spatial - 1) / spatial;
    SY_CHECK(rows * bins * spatial <= kMaxItems, SY_EUNSUPPORTED, "DFL input beyond 2^31");
    SY_CHECK(P[28] + ((rows - 1) * bins + bins - 1) * spatial + (k.items - 1 - (rows - 1) * spatial) < k.la &&
                 (long long)P[30] + k.items <= k.lc,
             SY_EINVAL, "DFL extents exceed a buffer");
    ProfScope prof(ctx, "compute_dfl", 0, 4.0 * (double)k.items * (bins + 1));
    const FastDiv sp = make_div((uint32_t)spatial);
    if (bins == 16)
      hipLaunchKernelGGL(dfl_kernel<16>, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, a, c, sp, 16u,
                         (uint32_t)k.items);
    else
      hipLaunchKernelGGL(dfl_kernel<0>, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, a, c, sp,
                         (uint32_t)bins, (uint32_t)k.items);
    return check_launch("compute_dfl");
  }
  if (op == 31) {
    const long long width = P[2], dim = P[3];
    SY_CHECK(spatial > 0 && width > 0 && dim > 0, SY_EINVAL, "pose decode needs spatial, width and fields");
    SY_CHECK((long long)P[28] + k.items <= k.la && (long long)P[30] + k.items <= k.lc, SY_EINVAL,
             "op 31 work items exceed a buffer");
    const bool y26 = P[5] == 1;
    ProfScope prof(ctx, "compute_pose_decode", 0, 8.0 * (double)k.items);
    hipLaunchKernelGGL(pose_decode_kernel, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, a, c,
                       make_div((uint32_t)spatial), make_div((uint32_t)dim), make_div((uint32_t)width),
                       bits_to_float(P[4]), y26 ? 1.f : 2.f, y26 ? .5f : 0.f, (uint32_t)k.items);
    return check_launch("compute_pose_decode");
  }
  // op 30
  const long long width = P[2], bins = P[3], nc = P[4], os = P[7] == 0 ? spatial : P[7], a0 = P[8];
  SY_CHECK(spatial > 0 && bins > 0, SY_EINVAL, "decode needs spatial and bins");
  SY_CHECK(width > 0, SY_EINVAL, "decode needs the row width");
  SY_CHECK(k.b || nc == 0, SY_EINVAL, "op 30 needs input 1");
  const long long images = (k.items + spatial - 1) / spatial, last_anchor = std::min(spatial, k.items) - 1;
  // Highest offsets: the last image's last side / class / output row.
  const long long box_last = ((images - 1) * 4 * bins + 4 * bins - 1) * spatial + last_anchor;
  const long long cls_last = nc ? ((images - 1) * nc + nc - 1) * spatial + last_anchor : -1;
  const long long out_last = (images - 1) * (nc + 4) * os + a0 + last_anchor + (nc + 3) * os;
  SY_CHECK(box_last < kMaxItems && out_last < kMaxItems, SY_EUNSUPPORTED, "decode extents beyond 2^31");
  SY_CHECK(P[28] + box_last < k.la && (nc == 0 || P[29] + cls_last < k.lb) && P[30] + out_last < k.lc, SY_EINVAL,
           "decode extents exceed a buffer");
  LevelDecode g{};
  g.spatial = make_div((uint32_t)spatial);
  g.width = make_div((uint32_t)width);
  g.n = (uint32_t)k.items;
  g.bins = (uint32_t)bins;
  g.nc = (uint32_t)nc;
  g.os = (uint32_t)os;
  g.a0 = (uint32_t)a0;
  g.stride = bits_to_float(P[5]);
  g.xyxy = P[6] == 1;
  const float* b = k.b ? k.b + P[29] : nullptr;
  ProfScope prof(ctx, "compute_level_decode", 0, 4.0 * (double)k.items * (4 * bins + 2 * nc + 4));
  if (bins == 16)
    hipLaunchKernelGGL(level_decode_kernel<16>, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, a, b, c, g);
  else if (bins == 1)
    hipLaunchKernelGGL(level_decode_kernel<1>, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, a, b, c, g);
  else
    hipLaunchKernelGGL(level_decode_kernel<0>, dim3(grid_for(k.items)), dim3(kThreads), 0, ctx->stream, a, b, c, g);
  return check_launch("compute_level_decode");
}

// Argument checks that need no device: known op, bindings, work items.
static int compute_args(int op, const float* const* in, const size_t* in_len, const uint32_t* params,
                        long long items, float* out, size_t out_len, Block* k) {
  SY_CHECK(params && out && out_len > 0 && items >= 0, SY_EINVAL, "null or empty compute arguments");
  SY_CHECK(!in || in_len, SY_EINVAL, "input lengths required");
  static const int known[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 20, 21, 22, 23, 24, 25, 26,
                              30, 31, 32, 33, 34, 35, 36, 37};
  bool ok = false;
  for (int q : known) ok |= q == op;
  SY_CHECK(ok, SY_EUNSUPPORTED, "device op %d is not implemented", op);
  const float* ptr[3] = {nullptr, nullptr, nullptr};
  long long len[3] = {0, 0, 0};
  for (int j = 0; j < 3 && in; ++j) {
    if (!in[j]) continue;
    // A bound buffer must hold something: a zero length would leave no
    // element to read.
    SY_CHECK(in_len[j] > 0, SY_EINVAL, "input %d is bound with length 0", j);
    ptr[j] = in[j];
    len[j] = (long long)in_len[j];
  }
  *k = Block{};
  for (int j = 0; j < 32; ++j) k->P[j] = params[j];
  // Slot 27 flags the third (bias) input, as the reference sets it from the
  // input count (VulkanExecution.cs:265).
  k->P[27] = ptr[2] ? 1u : 0u;
  k->a = ptr[0];
  k->b = ptr[1];
  k->d = ptr[2];
  k->la = len[0];
  k->lb = len[1];
  k->ld = len[2];
  k->c = out;
  k->lc = (long long)out_len;
  k->items = items;
  SY_CHECK(k->a, SY_EINVAL, "op %d needs input 0", op);
  const bool needs_b = (op >= 10 && op < 20) || op == 32 || op == 33 || op == 37;
  SY_CHECK(!needs_b || k->b, SY_EINVAL, "op %d needs input 1", op);
  SY_CHECK((long long)k->P[0] == items, SY_EINVAL, "work items %lld do not match params[0] %u", items, k->P[0]);
  SY_CHECK(items <= kMaxItems, SY_EUNSUPPORTED, "more than 2^31 work items");
  return SY_OK;
}

int op_compute(sy_ctx* ctx, int op, const float* const* in, const size_t* in_len, const uint32_t* params,
               long long items, float* out, size_t out_len) {
  Block k;
  SY_TRY(compute_args(op, in, in_len, params, items, out, out_len, &k));
  if (items == 0) return SY_OK;
  if (op < 10) return launch_unary(ctx, k, op);
  if (op < 20) return launch_binary(ctx, k, op);
  switch (op) {
    case 23: return launch_transpose(ctx, k);
    case 24: return launch_slice(ctx, k);
    case 25: return launch_softmax(ctx, k);
    case 26: return launch_concat(ctx, k);
    case 30: case 31: case 34: return launch_decode(ctx, k, op);
    case 36: return launch_row_max(ctx, k);
    case 37: return launch_gather(ctx, k);
    default: return launch_spatial(ctx, k, op);  // 20, 21, 22, 32, 33, 35
  }
}

// Batch decomposition of a matrix product: output matrix z has batch
// coordinates (row-major over shape[0..rank)); A and B matrix indices follow
// from their batch strides (0 on broadcast axes).
struct MatBatch {
  int rank;
  int shape[4];
  long long as[4], bs[4];
};

// Row-major C[m][n] = A[m][k] B[k][n] per batch matrix, for shapes the MFMA
// GEMM does not take (k % 4 != 0, unaligned, irregular batch strides):
// 16 x 16 output tiles, K staged through LDS 16 at a time.
__global__ __launch_bounds__(256) void matmul_tile_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ c, int m, int n, int k,
                                                          const MatBatch bt) {
  __shared__ float As[16][17], Bs[16][17];
  long long t = blockIdx.z, ai = 0, bi = 0;
  for (int j = bt.rank - 1; j >= 0; --j) {
    const long long coord = t % bt.shape[j];
    t /= bt.shape[j];
    ai += coord * bt.as[j];
    bi += coord * bt.bs[j];
  }
  const float* A = a + ai * m * k;
  const float* B = b + bi * k * n;
  float* C = c + (long long)blockIdx.z * m * n;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
  float acc = 0.f;
  for (int k0 = 0; k0 < k; k0 += 16) {
    As[ty][tx] = (row < m && k0 + tx < k) ? A[(long long)row * k + k0 + tx] : 0.f;
    Bs[ty][tx] = (k0 + ty < k && col < n) ? B[(long long)(k0 + ty) * n + col] : 0.f;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 16; ++q) acc += As[ty][q] * Bs[q][tx];
    __syncthreads();
  }
  if (row < m && col < n) C[(long long)row * n + col] = acc;
}

// B [k][n] -> Bt [n][kp] (zero K padding) for the MFMA GEMM, per batch matrix.
__global__ __launch_bounds__(256) void transpose_pad_kernel(const float* __restrict__ b, float* __restrict__ bt, int k,
                                                            int n, int kp, long long in_stride, long long out_stride) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)n * kp) return;
  const int col = (int)(i / kp), kk = (int)(i % kp);
  const float* src = b + (long long)blockIdx.y * in_stride;
  bt[(long long)blockIdx.y * out_stride + i] = kk < k ? src[(long long)kk * n + col] : 0.f;
}

int op_matmul(sy_ctx* ctx, const float* a, const float* b, float* c, int m, int n, int k, int nbatch,
              const int* batch_shape, const long long* a_strides, const long long* b_strides, size_t a_len,
              size_t b_len, size_t c_len) {
  SY_CHECK(a && b && c, SY_EINVAL, "null matrix");
  SY_CHECK(m > 0 && n > 0 && k > 0, SY_EUNSUPPORTED, "Empty device MatMul.");
  SY_CHECK(nbatch >= 0 && nbatch <= 4, SY_EUNSUPPORTED, "Device MatMul batch rank > 4.");
  // Per output matrix: offsets (floats) of its A, B and C matrices.
  long long count = 1;
  for (int j = 0; j < nbatch; ++j) {
    SY_CHECK(batch_shape[j] > 0, SY_EINVAL, "batch dims must be positive");
    count *= batch_shape[j];
  }
  SY_CHECK(count < 65536, SY_EUNSUPPORTED, "too many batch matrices");
  std::vector<long long> offs((size_t)count * 3);
  for (long long z = 0; z < count; ++z) {
    long long t = z, ao = 0, bo = 0;
    for (int j = nbatch - 1; j >= 0; --j) {
      const long long coord = t % batch_shape[j];
      t /= batch_shape[j];
      ao += coord * a_strides[j];
      bo += coord * b_strides[j];
    }
    offs[3 * z] = ao * (long long)m * k;
    offs[3 * z + 1] = bo * (long long)k * n;
    offs[3 * z + 2] = z * (long long)m * n;
    SY_CHECK(ao >= 0 && bo >= 0 && offs[3 * z] + (long long)m * k <= (long long)a_len &&
                 offs[3 * z + 1] + (long long)k * n <= (long long)b_len &&
                 offs[3 * z + 2] + (long long)m * n <= (long long)c_len,
             SY_EINVAL, "batch matrix %lld reaches past its buffer", z);
  }
  // Uniform batch strides and aligned operands: B transposed into scratch,
  // then the MFMA GEMM (C[m][n] = sum_k A[m][k] Bt[n][k]).
  bool uniform = true;
  for (long long z = 1; z < count; ++z)
    for (int q = 0; q < 3; ++q) uniform &= offs[3 * z + q] - offs[3 * (z - 1) + q] == offs[3 + q] - offs[q];
  const long long as = count > 1 ? offs[3] : 0, bs = count > 1 ? offs[4] : 0;
  const bool mfma = uniform && k % 4 == 0 && ((uintptr_t)a & 15) == 0 && as % 4 == 0 && !ctx->capturing;
  if (mfma) {
    const int kp = (k + 3) / 4 * 4;
    const long long bt_stride = (long long)n * kp;
    const long long bcount = bs == 0 ? 1 : count;
    SY_TRY(ensure_scratch(ctx, (size_t)(bcount * bt_stride) * sizeof(float)));
    float* bt = (float*)ctx->scratch;
    {
      ProfScope prof(ctx, "matmul_transpose", 0, 8.0 * (double)bcount * k * n);
      hipLaunchKernelGGL(transpose_pad_kernel, dim3((unsigned)((bt_stride + 255) / 256), (unsigned)bcount), dim3(256),
                         0, ctx->stream, b, bt, k, n, kp, bs, bt_stride);
      SY_TRY(check_launch("matmul_transpose"));
    }
    return gemm_nt(ctx, a, m, k, k, bt, n, kp, c, n, "matmul_gemm", (int)count, as, bs == 0 ? 0 : bt_stride,
                   count > 1 ? offs[5] - offs[2] : 0);
  }
  MatBatch bt{nbatch, {1, 1, 1, 1}, {0, 0, 0, 0}, {0, 0, 0, 0}};
  for (int j = 0; j < nbatch; ++j) {
    bt.shape[j] = batch_shape[j];
    bt.as[j] = a_strides[j];
    bt.bs[j] = b_strides[j];
  }
  ProfScope prof(ctx, "matmul_tile", 2.0 * count * m * n * k, 4.0 * count * ((double)m * k + (double)k * n + (double)m * n));
  hipLaunchKernelGGL(matmul_tile_kernel, dim3((unsigned)((n + 15) / 16), (unsigned)((m + 15) / 16), (unsigned)count),
                     dim3(256), 0, ctx->stream, a, b, c, m, n, k, bt);
  return check_launch("matmul_tile");
}

}  // namespace sy

using namespace sy;

extern "C" {

int sy_compute(sy_ctx* ctx, int op, const float* const* inputs, const size_t* input_lengths,
               const uint32_t* params, int64_t work_items, float* out, size_t out_length) {
  // The argument checks come first (they need no device), then the context.
  Block k;
  SY_TRY(compute_args(op, inputs, input_lengths, params, work_items, out, out_length, &k));
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_compute(ctx, op, inputs, input_lengths, params, work_items, out, out_length);
}

int sy_matmul(sy_ctx* ctx, const float* a, const float* b, float* c, int m, int n, int k, int batch_rank,
              const int32_t* batch_shape, const int64_t* a_batch_strides, const int64_t* b_batch_strides,
              size_t a_length, size_t b_length, size_t c_length) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_CHECK(batch_rank == 0 || (batch_shape && a_batch_strides && b_batch_strides), SY_EINVAL, "null batch arrays");
  long long as[4] = {0, 0, 0, 0}, bs[4] = {0, 0, 0, 0};
  int shape[4] = {1, 1, 1, 1};
  for (int j = 0; j < batch_rank && j < 4; ++j) {
    shape[j] = batch_shape[j];
    as[j] = a_batch_strides[j];
    bs[j] = b_batch_strides[j];
  }
  return op_matmul(ctx, a, b, c, m, n, k, batch_rank, shape, as, bs, a_length, b_length, c_length);
}

}  // extern "C"
