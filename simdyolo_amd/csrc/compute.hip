// Generic device ops of the reference's IDeviceBackend (src/SimdYolo/
// DeviceExecution.cs:41,61): the tensor.comp operation codes on dense
// row-major tensors, with the same 32-slot parameter block (the layouts
// DeviceOps and its callers build, DeviceExecution.cs:107-190), and the
// batched matrix product of DeviceMatMul (VulkanExecution.cs:499-541).
//
// These are the reference's fallback ops for modules outside the fused
// YOLO paths; the hot path does not use them.  One thread per work item, the
// operation a kernel argument (uniform per launch).  Every index is clamped
// to the buffer lengths the caller passes, so a wrong parameter block gives
// wrong values, never an access outside the buffers; the host checks the
// extents it can derive from the parameters and refuses the rest.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "sy_internal.h"

namespace sy {

struct ComputeArgs {
  const float* a;
  const float* b;
  const float* d;
  float* c;
  long long la, lb, ld, lc;  // lengths (floats); 0 for an absent buffer
  uint32_t p[32];
  int op;
  long long items;
};

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ __launch_bounds__(256) void tensor_op_kernel(const ComputeArgs g) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= g.items) return;
  const uint32_t* P = g.p;
  // Element offsets of the four bindings (tensor.comp A/B/C/D(i) add P(28..31)).
  auto A = [&](long long k) { return g.a[min(max(k + (long long)P[28], 0LL), g.la - 1)]; };
  auto B = [&](long long k) { return g.b[min(max(k + (long long)P[29], 0LL), g.lb - 1)]; };
  auto D = [&](long long k) { return g.d[min(max(k + (long long)P[31], 0LL), g.ld - 1)]; };
  auto C = [&](long long k, float v) {
    const long long j = k + (long long)P[30];
    if (j >= 0 && j < g.lc) g.c[j] = v;
  };
  const int op = g.op;
  if (op < 10) {
    const float x = A(i);
    float y = x;
    switch (op) {
      case 1: y = x * sigm(x); break;
      case 2: y = sigm(x); break;
      case 3: y = __builtin_elementwise_maximum(x, 0.f); break;
      case 4: y = x * u2f(P[1]); break;
      case 5: y = expf(x); break;
      case 6: y = sqrtf(x); break;
      case 7: y = -x; break;
      case 8: y = fabsf(x); break;
      case 9: y = x >= 0.f ? x : x * u2f(P[1]); break;
      default: break;
    }
    C(i, y);
  } else if (op < 20) {
    // Broadcast over four dims: P(1..4) output shape, P(5..8) / P(9..12) the
    // input strides (0 on broadcast axes).
    long long t = i, ai = 0, bi = 0;
    for (int j = 3; j >= 0; --j) {
      const long long coord = t % P[1 + j];
      t /= P[1 + j];
      ai += coord * P[5 + j];
      bi += coord * P[9 + j];
    }
    const float x = A(ai), y = B(bi);
    float r = 0.f;
    switch (op) {
      case 10: r = x + y; break;
      case 11: r = x - y; break;
      case 12: r = x * y; break;
      case 13: r = x / y; break;
      case 14: r = powf(x, y); break;
      case 15: r = __builtin_elementwise_maximum(x, y); break;
      case 16: r = __builtin_elementwise_minimum(x, y); break;
      default: break;
    }
    C(i, r);
  } else if (op == 20) {  // nearest resize: P(1,2) input h, w; P(3,4) output h, w
    const long long plane = (long long)P[3] * P[4];
    const long long ch = i / plane, oy = i % plane / P[4], ox = i % P[4];
    C(i, A((ch * P[1] + oy * P[1] / P[3]) * P[2] + ox * P[2] / P[4]));
  } else if (op == 21 || op == 22) {  // max / average pool
    const long long h = P[1], w = P[2], oh = P[3], ow = P[4], kh = P[5], kw = P[6], plane = oh * ow;
    const long long ch = i / plane, oy = i % plane / ow, ox = i % ow;
    const long long sy = oy * (long long)P[7] - P[9], sx = ox * (long long)P[8] - P[10];
    float v = op == 21 ? -INFINITY : 0.f;
    uint32_t count = 0;
    for (long long ky = 0; ky < kh; ++ky)
      for (long long kx = 0; kx < kw; ++kx) {
        const long long y = sy + ky, x = sx + kx;
        if (y >= 0 && x >= 0 && y < h && x < w) {
          const float e = A((ch * h + y) * w + x);
          v = op == 21 ? __builtin_elementwise_maximum(v, e) : v + e;
          ++count;
        }
      }
    C(i, op == 21 ? v : v / (float)(P[11] == 1 ? kh * kw : count));
  } else if (op == 23) {  // transpose: P(1..4) output shape, P(5..8) input strides
    long long t = i, src = 0;
    for (int j = 3; j >= 0; --j) {
      src += t % P[1 + j] * P[5 + j];
      t /= P[1 + j];
    }
    C(i, A(src));
  } else if (op == 24) {  // slice along an axis: P(1) input axis length, P(2) output axis length, P(3) inner, P(4) start
    const long long inner = P[3], outer = i / ((long long)P[2] * inner), rem = i % ((long long)P[2] * inner);
    C(i, A(outer * P[1] * inner + (long long)P[4] * inner + rem));
  } else if (op == 25) {  // softmax: P(1) axis length, P(2) inner; one work item per row
    const long long size = P[1], inner = P[2], base = i / inner * size * inner + i % inner;
    float m = -INFINITY, sum = 0.f;
    for (long long j = 0; j < size; ++j) m = fmaxf(m, A(base + j * inner));
    for (long long j = 0; j < size; ++j) sum += expf(A(base + j * inner) - m);
    for (long long j = 0; j < size; ++j) C(base + j * inner, expf(A(base + j * inner) - m) / sum);
  } else if (op == 26) {  // concat write: P(1) this input's axis length, P(2) output's, P(3) inner, P(4) offset
    const long long size = (long long)P[1] * P[3], outer = i / size;
    C(outer * P[2] * P[3] + (long long)P[4] * P[3] + i % size, A(i));
  } else if (op == 30 || op == 34) {
    // 30: one level's DFL decode + class sigmoid into [B][nc+4][out] (P(1)
    // spatial, P(2) width, P(3) bins, P(4) nc, P(5) stride bits, P(6) xyxy,
    // P(7) output spatial (0: spatial), P(8) anchor offset).  34: the DFL
    // expectation alone, P(1) spatial, P(2) bins.
    const long long spatial = P[1];
    const long long bins = op == 30 ? P[3] : P[2];
    auto dfl = [&](long long base) {
      if (bins == 1) return A(base);
      float m = -INFINITY, sum = 0.f, num = 0.f;
      for (long long j = 0; j < bins; ++j) m = fmaxf(m, A(base + j * spatial));
      for (long long j = 0; j < bins; ++j) {
        const float e = expf(A(base + j * spatial) - m);
        sum += e;
        num += e * (float)j;
      }
      return num / sum;
    };
    if (op == 34) {
      C(i, dfl(i / spatial * bins * spatial + i % spatial));
    } else {
      const long long width = P[2], nc = P[4], batch = i / spatial, anchor = i % spatial;
      float dist[4];
      for (int side = 0; side < 4; ++side) dist[side] = dfl((batch * 4 + side) * bins * spatial + anchor);
      const float stride = u2f(P[5]);
      const float cx = (float)(anchor % width) + .5f, cy = (float)(anchor / width) + .5f;
      const float x1 = (cx - dist[0]) * stride, y1 = (cy - dist[1]) * stride;
      const float x2 = (cx + dist[2]) * stride, y2 = (cy + dist[3]) * stride;
      const long long os = P[7] == 0 ? spatial : P[7];
      const long long dst = batch * (nc + 4) * os + P[8] + anchor;
      const bool xyxy = P[6] == 1;
      C(dst, xyxy ? x1 : (x1 + x2) * .5f);
      C(dst + os, xyxy ? y1 : (y1 + y2) * .5f);
      C(dst + 2 * os, xyxy ? x2 : x2 - x1);
      C(dst + 3 * os, xyxy ? y2 : y2 - y1);
      for (long long j = 0; j < nc; ++j) C(dst + (4 + j) * os, sigm(B((batch * nc + j) * spatial + anchor)));
    }
  } else if (op == 31) {  // pose keypoints: P(1) spatial, P(2) width, P(3) fields, P(4) stride bits, P(5) YOLO26
    const long long spatial = P[1], width = P[2], dim = P[3], axis = i / spatial % dim, anchor = i % spatial;
    const float v = A(i), stride = u2f(P[4]);
    const float factor = P[5] == 1 ? 1.f : 2.f, offset = P[5] == 1 ? .5f : 0.f;
    C(i, axis == 0   ? (v * factor + ((float)(anchor % width) + offset)) * stride
         : axis == 1 ? (v * factor + ((float)(anchor / width) + offset)) * stride
                     : sigm(v));
  } else if (op == 32) {  // depthwise conv: P(1..3) ic, ih, iw; P(5..8) oh, ow, kh, kw; P(9..14) stride, pad, dilation
    const long long ic = P[1], ih = P[2], iw = P[3], oh = P[5], ow = P[6], kh = P[7], kw = P[8];
    const long long spatial = oh * ow, bc = i / spatial, ch = bc % ic, oy = i % spatial / ow, ox = i % ow;
    float v = P[27] == 1 ? D(ch) : 0.f;
    for (long long ky = 0; ky < kh; ++ky)
      for (long long kx = 0; kx < kw; ++kx) {
        const long long y = oy * P[9] - (long long)P[11] + ky * P[13], x = ox * P[10] - (long long)P[12] + kx * P[14];
        if (y >= 0 && x >= 0 && y < ih && x < iw) v += A((bc * ih + y) * iw + x) * B((ch * kh + ky) * kw + kx);
      }
    C(i, P[16] == 1 ? v * sigm(v) : v);
  } else if (op == 33) {  // transposed conv (groups P(15)), weights [ic][oc/groups][kh][kw]
    const long long ic = P[1], ih = P[2], iw = P[3], oc = P[4], oh = P[5], ow = P[6], kh = P[7], kw = P[8];
    const long long groups = P[15] ? P[15] : 1;
    const long long spatial = oh * ow, co = i / spatial % oc, batch = i / (spatial * oc);
    const long long cog = oc / groups, cig = ic / groups, grp = co / cog, oy = i % spatial / ow, ox = i % ow;
    float v = P[27] == 1 ? D(co) : 0.f;
    for (long long ky = 0; ky < kh; ++ky)
      for (long long kx = 0; kx < kw; ++kx) {
        const long long yn = oy + P[11] - ky * P[13], xn = ox + P[12] - kx * P[14];
        if (yn < 0 || xn < 0 || yn % P[9] != 0 || xn % P[10] != 0) continue;
        const long long y = yn / P[9], x = xn / P[10];
        if (y >= ih || x >= iw) continue;
        for (long long ci = grp * cig; ci < (grp + 1) * cig; ++ci)
          v += A(((batch * ic + ci) * ih + y) * iw + x) * B(((ci * cog + co % cog) * kh + ky) * kw + kx);
      }
    C(i, v);
  } else if (op == 35) {  // depth to space by 2: input [B][4C][h/2][w/2] -> [B][C][h][w]
    const long long h = P[1], w = P[2], channels = P[3], plane = h * w;
    const long long co = i / plane % channels, batch = i / (plane * channels), y = i % plane / w, x = i % w;
    C(i, A(((batch * channels * 4 + co * 4 + y % 2 * 2 + x % 2) * (h / 2) + y / 2) * (w / 2) + x / 2));
  } else if (op == 36) {  // row maximum with MathF.Max semantics (NaN wins, +0 over -0)
    const long long size = P[1], base = i * size;
    float m = -INFINITY;
    for (long long j = 0; j < size; ++j) {
      const float v = A(base + j);
      if (v != v) {
        m = v;
        break;
      }
      if (v > m || (v == 0.f && m == 0.f && __float_as_uint(v) == 0u)) m = v;
    }
    C(i, m);
  } else if (op == 37) {  // gather along P(9) with indices in B (negative from the end, axis length P(10))
    long long t = i, src = 0;
    for (int dim = 3; dim >= 0; --dim) {
      long long coord = t % P[1 + dim];
      t /= P[1 + dim];
      if ((uint32_t)dim == P[9]) {
        long long idx = (long long)B(i);
        if (idx < 0) idx += P[10];
        coord = idx;
      }
      src += coord * P[5 + dim];
    }
    C(i, A(src));
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

static long long max_index(long long base, const uint32_t* shape, const uint32_t* strides) {
  long long m = base;
  for (int j = 0; j < 4; ++j)
    if (shape[j] > 0) m += (long long)(shape[j] - 1) * strides[j];
  return m;
}

int op_compute(sy_ctx* ctx, int op, const float* const* in, const size_t* in_len, const uint32_t* params,
               long long items, float* out, size_t out_len) {
  SY_CHECK(params && out && out_len > 0 && items >= 0, SY_EINVAL, "null or empty compute arguments");
  static const int known[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 20, 21, 22, 23, 24, 25, 26,
                              30, 31, 32, 33, 34, 35, 36, 37};
  bool ok = false;
  for (int k : known) ok |= k == op;
  SY_CHECK(ok, SY_EUNSUPPORTED, "device op %d is not implemented", op);
  ComputeArgs g{};
  g.a = in && in[0] ? in[0] : nullptr;
  g.b = in && in[1] ? in[1] : nullptr;
  g.d = in && in[2] ? in[2] : nullptr;
  g.la = g.a ? (long long)in_len[0] : 0;
  g.lb = g.b ? (long long)in_len[1] : 0;
  g.ld = g.d ? (long long)in_len[2] : 0;
  g.c = out;
  g.lc = (long long)out_len;
  g.op = op;
  g.items = items;
  for (int j = 0; j < 32; ++j) g.p[j] = params[j];
  // Slot 27 flags the third (bias) input, as the reference's Compute sets it
  // from the input count (VulkanExecution.cs:265).
  g.p[27] = g.d ? 1u : 0u;
  const uint32_t* P = g.p;
  // Inputs each op reads, and extents that follow from the parameters.
  const bool needs_b = (op >= 10 && op < 20) || op == 30 || op == 32 || op == 33 || op == 37;
  SY_CHECK(g.la > 0, SY_EINVAL, "op %d needs input 0", op);
  SY_CHECK(!needs_b || g.lb > 0, SY_EINVAL, "op %d needs input 1", op);
  SY_CHECK((long long)P[0] == items, SY_EINVAL, "work items %lld do not match params[0] %u", items, P[0]);
  if ((op >= 10 && op < 20) || op == 23 || op == 37)
    SY_CHECK(P[1] > 0 && P[2] > 0 && P[3] > 0 && P[4] > 0, SY_EINVAL, "op %d needs a positive 4-d shape", op);
  if (op < 10 || op == 31)
    SY_CHECK(items <= g.la && items + (long long)P[30] <= g.lc, SY_EINVAL, "op %d work items exceed a buffer", op);
  if (op >= 10 && op < 20) {
    SY_CHECK(items + (long long)P[30] <= g.lc, SY_EINVAL, "broadcast output exceeds its buffer");
    SY_CHECK(max_index(P[28], P + 1, P + 5) < g.la && max_index(P[29], P + 1, P + 9) < g.lb, SY_EINVAL,
             "broadcast strides reach past an input");
  }
  if (op == 23)
    SY_CHECK(max_index(P[28], P + 1, P + 5) < g.la && items + (long long)P[30] <= g.lc, SY_EINVAL,
             "transpose extents exceed a buffer");
  if (op == 25)
    SY_CHECK(P[1] > 0 && P[2] > 0 && items * P[1] + (long long)P[30] <= g.lc && items * P[1] <= g.la, SY_EINVAL,
             "softmax extents exceed a buffer");
  if (op == 30 || op == 34)
    SY_CHECK(P[1] > 0 && (op == 34 ? P[2] : P[3]) > 0, SY_EINVAL, "decode needs spatial and bins");
  if (op == 30 || op == 31)
    SY_CHECK(P[2] > 0, SY_EINVAL, "decode needs the row width");
  if (op == 20 || op == 21 || op == 22)
    SY_CHECK(P[3] > 0 && P[4] > 0, SY_EINVAL, "spatial op needs an output size");
  if (op == 24) SY_CHECK(P[2] > 0 && P[3] > 0, SY_EINVAL, "slice needs axis and inner sizes");
  if (op == 26) SY_CHECK(P[1] > 0 && P[3] > 0, SY_EINVAL, "concat needs axis and inner sizes");
  if (op == 31) SY_CHECK(P[1] > 0 && P[3] > 0, SY_EINVAL, "pose decode needs spatial and fields");
  if (op == 32 || op == 33)
    SY_CHECK(P[1] > 0 && P[5] > 0 && P[6] > 0 && P[9] > 0 && P[10] > 0 && (op == 32 || P[4] > 0), SY_EINVAL,
             "conv op needs channels, output size and strides");
  if (op == 33) {
    const uint32_t groups = P[15] ? P[15] : 1;
    SY_CHECK(P[1] % groups == 0 && P[4] % groups == 0, SY_EINVAL, "channels not divisible by groups");
  }
  if (op == 35) SY_CHECK(P[1] > 0 && P[2] > 0 && P[3] > 0, SY_EINVAL, "depth-to-space needs its shape");
  if (op == 36) SY_CHECK(P[1] > 0, SY_EINVAL, "row max needs the row length");
  if (op == 37) SY_CHECK(P[9] < 4, SY_EINVAL, "gather axis out of range");
  if (items == 0) return SY_OK;
  char name[24];
  snprintf(name, sizeof name, "tensor_op_%d", op);
  ProfScope prof(ctx, name, 0, 4.0 * (double)items * 2);
  const long long blocks = (items + 255) / 256;
  SY_CHECK(blocks < (1LL << 31), SY_EUNSUPPORTED, "too many work items");
  hipLaunchKernelGGL(tensor_op_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, g);
  return check_launch(name);
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
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_CHECK(!inputs || input_lengths, SY_EINVAL, "input lengths required");
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
