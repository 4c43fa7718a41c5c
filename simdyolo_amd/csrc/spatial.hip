// Bandwidth-bound kernels: layout changes, copy/add, nearest resize, max pool
// (generic and the fused SPPF chain) and the joined detect-head decode.
#include <cmath>

#include "sy_internal.h"

namespace sy {

typedef float f32x4 __attribute__((ext_vector_type(4)));

static bool vec4_ok(const sy_tensor* t) { return ((uintptr_t)t->data & 15) == 0 && (t->ldc & 3) == 0 && (t->c & 3) == 0; }

static unsigned blocks_for(long long threads, int per_block = 256) {
  return (unsigned)((threads + per_block - 1) / per_block);
}

// ------------------------------------------------------------ layout changes

// Dense NCHW (device) -> NHWC view.  One thread per destination element,
// channel fastest within a pixel run so stores coalesce.
__global__ void nchw_to_view_kernel(const float* __restrict__ src, int N, int C, int H, int W, float* __restrict__ dst,
                                    int ldc) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * C * H * W;
  if (i >= total) return;
  const int c = (int)(i % C);
  const long long p = i / C;  // pixel (n, h, w)
  const long long hw = (long long)H * W;
  const long long n = p / hw, s = p % hw;
  dst[p * ldc + c] = src[(n * C + c) * hw + s];
}

__global__ void view_to_nchw_kernel(const float* __restrict__ src, int ldc, int N, int C, int H, int W,
                                    float* __restrict__ dst) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * C * H * W;
  if (i >= total) return;
  const long long hw = (long long)H * W;
  const long long s = i % hw;
  const long long nc = i / hw;
  const int c = (int)(nc % C);
  const long long n = nc / C;
  dst[i] = src[(n * hw + s) * ldc + c];
}

int op_nchw_to_view(sy_ctx* ctx, const float* src, const sy_tensor* dst) {
  SY_TRY(check_view(dst, "layout destination"));
  const long long total = (long long)dst->n * dst->c * dst->h * dst->w;
  ProfScope prof(ctx, "nchw_to_nhwc", 0, 8.0 * total);
  hipLaunchKernelGGL(nchw_to_view_kernel, dim3(blocks_for(total)), dim3(256), 0, ctx->stream, src, dst->n, dst->c,
                     dst->h, dst->w, dst->data, dst->ldc);
  return check_launch("nchw_to_nhwc");
}

int op_view_to_nchw(sy_ctx* ctx, const sy_tensor* src, float* dst) {
  SY_TRY(check_view(src, "layout source"));
  const long long total = (long long)src->n * src->c * src->h * src->w;
  ProfScope prof(ctx, "nhwc_to_nchw", 0, 8.0 * total);
  hipLaunchKernelGGL(view_to_nchw_kernel, dim3(blocks_for(total)), dim3(256), 0, ctx->stream, src->data, src->ldc,
                     src->n, src->c, src->h, src->w, dst);
  return check_launch("nhwc_to_nchw");
}

// ------------------------------------------------------------ copy / add

template <bool ADD>
__global__ void binary4_kernel(const float* __restrict__ a, int lda, const float* __restrict__ b, int ldb,
                               float* __restrict__ y, int ldy, long long pixels, int C4) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pixels * C4) return;
  const int c = (int)(i % C4) * 4;
  const long long p = i / C4;
  f32x4 v = *(const f32x4*)(a + p * lda + c);
  if (ADD) v = v + *(const f32x4*)(b + p * ldb + c);
  *(f32x4*)(y + p * ldy + c) = v;
}

template <bool ADD>
__global__ void binary1_kernel(const float* __restrict__ a, int lda, const float* __restrict__ b, int ldb,
                               float* __restrict__ y, int ldy, long long pixels, int C) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pixels * C) return;
  const int c = (int)(i % C);
  const long long p = i / C;
  float v = a[p * lda + c];
  if (ADD) v = v + b[p * ldb + c];
  y[p * ldy + c] = v;
}

static bool same_shape(const sy_tensor* a, const sy_tensor* b) {
  return a->n == b->n && a->c == b->c && a->h == b->h && a->w == b->w;
}

template <bool ADD>
static int run_binary(sy_ctx* ctx, const sy_tensor* a, const sy_tensor* b, const sy_tensor* y, const char* name) {
  const long long px = pixels(*y);
  ProfScope prof(ctx, name, ADD ? (double)px * y->c : 0, 4.0 * px * y->c * (ADD ? 3 : 2));
  if (vec4_ok(a) && vec4_ok(y) && (!ADD || vec4_ok(b))) {
    const int C4 = y->c / 4;
    hipLaunchKernelGGL(binary4_kernel<ADD>, dim3(blocks_for(px * C4)), dim3(256), 0, ctx->stream, a->data, a->ldc,
                       ADD ? b->data : nullptr, ADD ? b->ldc : 0, y->data, y->ldc, px, C4);
  } else {
    hipLaunchKernelGGL(binary1_kernel<ADD>, dim3(blocks_for(px * y->c)), dim3(256), 0, ctx->stream, a->data, a->ldc,
                       ADD ? b->data : nullptr, ADD ? b->ldc : 0, y->data, y->ldc, px, y->c);
  }
  return check_launch(name);
}

int op_add(sy_ctx* ctx, const sy_tensor* a, const sy_tensor* b, const sy_tensor* y) {
  SY_TRY(check_view(a, "add a"));
  SY_TRY(check_view(b, "add b"));
  SY_TRY(check_view(y, "add output"));
  SY_CHECK(same_shape(a, b) && same_shape(a, y), SY_EINVAL, "add requires equal shapes");
  return run_binary<true>(ctx, a, b, y, "add");
}

int op_copy(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y) {
  SY_TRY(check_view(x, "copy source"));
  SY_TRY(check_view(y, "copy destination"));
  SY_CHECK(same_shape(x, y), SY_EINVAL, "copy requires equal shapes");
  return run_binary<false>(ctx, x, nullptr, y, "copy");
}

// ------------------------------------------------------------ nearest resize

// out[y][x] = in[y*ih/oh][x*iw/ow]  (src/SimdYolo/CpuSpatial.cs:21-47).
__global__ void resize4_kernel(const float* __restrict__ x, int ldx, int IH, int IW, float* __restrict__ y, int ldy,
                               int N, int OH, int OW, int C4) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * OH * OW * C4;
  if (i >= total) return;
  const int c = (int)(i % C4) * 4;
  const long long p = i / C4;
  const int ox = (int)(p % OW);
  const long long t = p / OW;
  const int oy = (int)(t % OH);
  const long long n = t / OH;
  const int iy = (int)((long long)oy * IH / OH), ix = (int)((long long)ox * IW / OW);
  *(f32x4*)(y + p * ldy + c) = *(const f32x4*)(x + ((n * IH + iy) * IW + ix) * ldx + c);
}

// Exact 2x nearest upsample (OH = 2 IH, OW = 2 IW: input pixel (iy, ix) is
// output pixels (2iy + dy, 2ix + dx)): one thread per input float4 writes its
// 2x2 output block, so each input value is read once and the index math is
// 32-bit (the caller checks that the element count fits).
__global__ void resize2x4_kernel(const float* __restrict__ x, int ldx, int IH, int IW, float* __restrict__ y,
                                 int ldy, int total, int C4) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c = (i % C4) * 4;
  const int p = i / C4;  // input pixel n * IH * IW + iy * IW + ix
  const int ix = p % IW, r = p / IW;
  const int iy = r % IH, n = r / IH;
  const f32x4 v = *(const f32x4*)(x + (long long)p * ldx + c);
  const int OW = 2 * IW;
  const long long o = ((long long)(n * 2 * IH + 2 * iy) * OW + 2 * ix) * ldy + c;
  *(f32x4*)(y + o) = v;
  *(f32x4*)(y + o + ldy) = v;
  *(f32x4*)(y + o + (long long)OW * ldy) = v;
  *(f32x4*)(y + o + (long long)(OW + 1) * ldy) = v;
}

__global__ void resize1_kernel(const float* __restrict__ x, int ldx, int IH, int IW, float* __restrict__ y, int ldy,
                               int N, int OH, int OW, int C) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * OH * OW * C;
  if (i >= total) return;
  const int c = (int)(i % C);
  const long long p = i / C;
  const int ox = (int)(p % OW);
  const long long t = p / OW;
  const int oy = (int)(t % OH);
  const long long n = t / OH;
  const int iy = (int)((long long)oy * IH / OH), ix = (int)((long long)ox * IW / OW);
  y[p * ldy + c] = x[((n * IH + iy) * IW + ix) * ldx + c];
}

int op_resize_nearest(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y) {
  SY_TRY(check_view(x, "resize input"));
  SY_TRY(check_view(y, "resize output"));
  SY_CHECK(x->n == y->n && x->c == y->c, SY_EINVAL, "resize keeps batch and channels");
  ProfScope prof(ctx, "resize_nearest", 0, 4.0 * ((double)pixels(*x) * x->c + (double)pixels(*y) * y->c));
  if (vec4_ok(x) && vec4_ok(y) && y->h == 2 * x->h && y->w == 2 * x->w &&
      pixels(*x) * (x->c / 4) < (1LL << 31) && pixels(*y) < (1LL << 31)) {
    const int total = (int)(pixels(*x) * (x->c / 4));
    hipLaunchKernelGGL(resize2x4_kernel, dim3(blocks_for(total)), dim3(256), 0, ctx->stream, x->data, x->ldc, x->h,
                       x->w, y->data, y->ldc, total, x->c / 4);
  } else if (vec4_ok(x) && vec4_ok(y)) {
    const long long total = pixels(*y) * (y->c / 4);
    hipLaunchKernelGGL(resize4_kernel, dim3(blocks_for(total)), dim3(256), 0, ctx->stream, x->data, x->ldc, x->h,
                       x->w, y->data, y->ldc, y->n, y->h, y->w, y->c / 4);
  } else {
    const long long total = pixels(*y) * y->c;
    hipLaunchKernelGGL(resize1_kernel, dim3(blocks_for(total)), dim3(256), 0, ctx->stream, x->data, x->ldc, x->h,
                       x->w, y->data, y->ldc, y->n, y->h, y->w, y->c);
  }
  return check_launch("resize_nearest");
}

// ------------------------------------------------------------ max pool

// Every max below is .NET MathF.Max's IEEE 754-2019 maximum (a NaN in the
// window propagates, +0 > -0), as the reference's pools use it
// (CpuSpatial.cs:370-400); gfx950 has it natively (v_maximum3_f32), and it
// does not depend on the order the window is visited in.
//
// Generic max pool, padding excluded (windows clipped to the image):
// src/SimdYolo/Compute.cs:677-708, CpuSpatial.cs:345-410.
__global__ void maxpool_kernel(const float* __restrict__ x, int ldx, int H, int W, float* __restrict__ y, int ldy,
                               int N, int OH, int OW, int C, int KH, int KW, int SH, int SW, int PT, int PL) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * OH * OW * C;
  if (i >= total) return;
  const int c = (int)(i % C);
  const long long p = i / C;
  const int ox = (int)(p % OW);
  const long long t = p / OW;
  const int oy = (int)(t % OH);
  const long long n = t / OH;
  float m = -INFINITY;
  for (int ky = 0; ky < KH; ++ky) {
    const int iy = oy * SH - PT + ky;
    if ((unsigned)iy >= (unsigned)H) continue;
    for (int kx = 0; kx < KW; ++kx) {
      const int ix = ox * SW - PL + kx;
      if ((unsigned)ix >= (unsigned)W) continue;
      m = __builtin_elementwise_maximum(m, x[((n * H + iy) * W + ix) * ldx + c]);
    }
  }
  y[p * ldy + c] = m;
}

// Four channels per thread (16-byte views): consecutive lanes take
// consecutive channel groups of one pixel, so every tap is a contiguous run
// of the NHWC row, and the window's loads are issued before the reduction.
__global__ __launch_bounds__(256) void maxpool4_kernel(const float* __restrict__ x, int ldx, int H, int W,
                                                       float* __restrict__ y, int ldy, int N, int OH, int OW, int CG,
                                                       int KH, int KW, int SH, int SW, int PT, int PL) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)N * OH * OW * CG;
  if (i >= total) return;
  const int c = 4 * (int)(i % CG);
  const long long p = i / CG;
  const int ox = (int)(p % OW);
  const long long t = p / OW;
  const int oy = (int)(t % OH);
  const long long n = t / OH;
  const float* img = x + n * H * W * ldx + c;
  f32x4 m = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  const int iy0 = oy * SH - PT, ix0 = ox * SW - PL;
  for (int ky = 0; ky < KH; ++ky) {
    const int iy = iy0 + ky;
    if ((unsigned)iy >= (unsigned)H) continue;
    const float* row = img + (long long)iy * W * ldx;
    for (int kx = 0; kx < KW; ++kx) {
      const int ix = ix0 + kx;
      if ((unsigned)ix >= (unsigned)W) continue;
      m = __builtin_elementwise_maximum(m, *(const f32x4*)(row + (long long)ix * ldx));
    }
  }
  *(f32x4*)(y + p * ldy + c) = m;
}

static bool launch_pool5_plane(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5, const sy_tensor* y9,
                               const sy_tensor* y13, int passes);

// 20x20 planes (the SPPF of a 640 input): PASSES chained clipped 5x5 max
// pools in registers.  A workgroup is one image's 16 channels; its four
// waves own five output rows each (quarter q: rows 5q .. 5q + 4), and a lane
// holds one channel of a block of 5 columns (lane = 16 * block + channel, so
// each pixel's 16 channels are 64 contiguous bytes).  A pass needs the two
// rows either side of a quarter: the first pass loads them, later passes
// take them from the neighbouring quarters through LDS.  Rows past the
// image's top and bottom repeat its edge row, and at its left and right
// edges a lane reuses its own edge column: a repeated edge value lies inside
// every window that reaches past the edge, so the windows stay exactly the
// clipped ones.  The two columns either side of a block come from the
// neighbouring lanes.
template <int PASSES>
__global__ __launch_bounds__(256) void sppf_rows20_kernel(const float* __restrict__ x, int ldx, int C,
                                                          float* __restrict__ y5, int ld5, float* __restrict__ y9,
                                                          int ld9, float* __restrict__ y13, int ld13) {
  constexpr int H = 20, W = 20, CW = 5, QR = 5, R = QR + 4;  // rows: own 5 and 2 either side
  __shared__ float S[4][4][CW][64];                        // [quarter][first 2, last 2 own rows][col][lane]
  const int lane = threadIdx.x & 63;
  const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int groups = C >> 4, n = blockIdx.x / groups, c0 = (blockIdx.x - n * groups) * 16;
  const int cb = lane >> 4;
  // Addresses: a wave-uniform base per pixel (scalar registers) plus one
  // 32-bit lane offset (the lane's column block and channel).
  const long long img = (long long)n * H * W;
  const int lane_px = cb * CW, lane_c = lane & 15;
  const float* xb = x + img * ldx + c0;
  const int xo = lane_px * ldx + lane_c;
  float v[R][CW];  // local row k is image row 5q - 2 + k
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int row = min(max(QR * q - 2 + k, 0), H - 1);
#pragma unroll
    for (int j = 0; j < CW; ++j) v[k][j] = xb[(long long)(row * W + j) * ldx + xo];
  }
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    if (pass > 0) {
      // Halo rows of this pass: the neighbours' edge rows of the last one.
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          S[q][k][j][lane] = v[2 + k][j];
          S[q][2 + k][j][lane] = v[QR + k][j];
        }
      __syncthreads();
      const int qa = max(q - 1, 0), qb = min(q + 1, 3);  // in bounds; edges keep their own rows
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          const float above = S[qa][2 + k][j][lane], below = S[qb][k][j][lane];
          v[k][j] = q > 0 ? above : v[2][j];
          v[QR + 2 + k][j] = q < 3 ? below : v[QR + 1][j];
        }
      __syncthreads();  // the next pass overwrites S
    }
    float t[QR][CW];
#pragma unroll
    for (int i = 0; i < QR; ++i)
#pragma unroll
      for (int j = 0; j < CW; ++j)
        t[i][j] = __builtin_elementwise_maximum(
            __builtin_elementwise_maximum(__builtin_elementwise_maximum(v[i][j], v[i + 1][j]),
                                          __builtin_elementwise_maximum(v[i + 2][j], v[i + 3][j])),
            v[i + 4][j]);
#pragma unroll
    for (int i = 0; i < QR; ++i) {
      float e[CW + 4];
      e[0] = __shfl(t[i][CW - 2], lane - 16);
      e[1] = __shfl(t[i][CW - 1], lane - 16);
      e[CW + 2] = __shfl(t[i][0], lane + 16);
      e[CW + 3] = __shfl(t[i][1], lane + 16);
      if (cb == 0) e[0] = e[1] = t[i][0];
      if (cb == 3) e[CW + 2] = e[CW + 3] = t[i][CW - 1];
#pragma unroll
      for (int j = 0; j < CW; ++j) e[j + 2] = t[i][j];
#pragma unroll
      for (int j = 0; j < CW; ++j)
        v[2 + i][j] = __builtin_elementwise_maximum(
            __builtin_elementwise_maximum(__builtin_elementwise_maximum(e[j], e[j + 1]),
                                          __builtin_elementwise_maximum(e[j + 2], e[j + 3])),
            e[j + 4]);
    }
    const int ldo = pass == 0 ? ld5 : pass == 1 ? ld9 : ld13;
    float* yb = (pass == 0 ? y5 : pass == 1 ? y9 : y13) + img * ldo + c0;
    const int yo = lane_px * ldo + lane_c;
#pragma unroll
    for (int i = 0; i < QR; ++i)
#pragma unroll
      for (int j = 0; j < CW; ++j) yb[(long long)((QR * q + i) * W + j) * ldo + yo] = v[2 + i][j];
  }
}

// Launches sppf_rows20_kernel for 20x20 planes whose channels come in whole
// groups of 16; false otherwise.  Any channel offset and pixel stride work
// (the kernel reads and writes single floats).
static bool launch_pool5_rows20(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5, const sy_tensor* y9,
                                const sy_tensor* y13, int passes) {
  if (x->h != 20 || x->w != 20 || x->c % 16 != 0) return false;
  const long long groups = (long long)x->n * (x->c / 16);
  if (groups > 0x7fffffffLL) return false;
  const sy_tensor* z9 = y9 ? y9 : y5;
  const sy_tensor* z13 = y13 ? y13 : y5;
  const dim3 grid((unsigned)groups);
  if (passes == 3)
    hipLaunchKernelGGL(sppf_rows20_kernel<3>, grid, dim3(256), 0, ctx->stream, x->data, x->ldc, x->c, y5->data,
                       y5->ldc, z9->data, z9->ldc, z13->data, z13->ldc);
  else
    hipLaunchKernelGGL(sppf_rows20_kernel<1>, grid, dim3(256), 0, ctx->stream, x->data, x->ldc, x->c, y5->data,
                       y5->ldc, z9->data, z9->ldc, z13->data, z13->ldc);
  return true;
}

int op_maxpool(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y, int kh, int kw, int sh, int sw, int pt, int pl,
               int pb, int pr, int ceil_mode) {
  SY_TRY(check_view(x, "pool input"));
  SY_TRY(check_view(y, "pool output"));
  SY_CHECK(kh > 0 && kw > 0 && sh > 0 && sw > 0 && pt >= 0 && pl >= 0 && pb >= 0 && pr >= 0, SY_EINVAL,
           "invalid pooling parameters");
  const long long oh = pool_out_size(x->h, kh, sh, pt, pb, ceil_mode);
  const long long ow = pool_out_size(x->w, kw, sw, pl, pr, ceil_mode);
  SY_CHECK(oh > 0 && ow > 0, SY_EINVAL, "pooling kernel exceeds the padded input dimensions");
  SY_CHECK(y->n == x->n && y->c == x->c && y->h == oh && y->w == ow, SY_EINVAL, "pool output shape mismatch");
  const long long total = pixels(*y) * y->c;
  ProfScope prof(ctx, "maxpool", 0, 4.0 * ((double)pixels(*x) * x->c + (double)total));
  // The SPPF pool (5x5, stride 1, pad 2): 20x20 planes in registers, other
  // small planes whole in LDS.
  const bool pool5 = kh == 5 && kw == 5 && sh == 1 && sw == 1 && pt == 2 && pl == 2 && pb == 2 && pr == 2 &&
                     oh == x->h && ow == x->w;
  if (pool5 && launch_pool5_rows20(ctx, x, y, nullptr, nullptr, 1)) return check_launch("maxpool");
  if (pool5 && vec4_ok(x) && vec4_ok(y) && launch_pool5_plane(ctx, x, y, nullptr, nullptr, 1))
    return check_launch("maxpool");
  if (vec4_ok(x) && vec4_ok(y)) {
    hipLaunchKernelGGL(maxpool4_kernel, dim3(blocks_for(total / 4)), dim3(256), 0, ctx->stream, x->data, x->ldc, x->h,
                       x->w, y->data, y->ldc, y->n, y->h, y->w, y->c / 4, kh, kw, sh, sw, pt, pl);
    return check_launch("maxpool");
  }
  hipLaunchKernelGGL(maxpool_kernel, dim3(blocks_for(total)), dim3(256), 0, ctx->stream, x->data, x->ldc, x->h, x->w,
                     y->data, y->ldc, y->n, y->h, y->w, y->c, kh, kw, sh, sw, pt, pl);
  return check_launch("maxpool");
}

// SPPF chain: three MaxPool2d(5, 1, 2) applied in sequence equal one pass of
// clipped 5x5, 9x9 and 13x13 windows (max is exact and the clipped window
// composition of two boxes is the larger clipped box).  One workgroup computes
// a 16x16 pixel tile for 4 channels from an LDS tile with a 6-pixel halo:
// separable row maxima (5/9/13) first, then column maxima.
constexpr int kSppfTile = 16, kSppfHalo = 6, kSppfIn = kSppfTile + 2 * kSppfHalo;  // 28

__global__ __launch_bounds__(256) void sppf_kernel(const float* __restrict__ x, int ldx, int N, int H, int W, int C,
                                                   float* __restrict__ y5, int ld5, float* __restrict__ y9, int ld9,
                                                   float* __restrict__ y13, int ld13) {
  __shared__ f32x4 tile[kSppfIn][kSppfIn];
  __shared__ f32x4 h5[kSppfIn][kSppfTile], h9[kSppfIn][kSppfTile], h13[kSppfIn][kSppfTile];
  const int tilesx = (W + kSppfTile - 1) / kSppfTile;
  const int bx = blockIdx.x % tilesx, by = blockIdx.x / tilesx;
  const int c = blockIdx.y * 4;
  const int n = blockIdx.z;
  const int x0 = bx * kSppfTile - kSppfHalo, y0 = by * kSppfTile - kSppfHalo;
  const float* img = x + (long long)n * H * W * ldx + c;
  const f32x4 ninf = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  for (int i = threadIdx.x; i < kSppfIn * kSppfIn; i += 256) {
    const int ty = i / kSppfIn, tx = i % kSppfIn;
    const int iy = y0 + ty, ix = x0 + tx;
    tile[ty][tx] = ((unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W)
                       ? *(const f32x4*)(img + ((long long)iy * W + ix) * ldx)
                       : ninf;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kSppfIn * kSppfTile; i += 256) {
    const int ty = i / kSppfTile, tx = i % kSppfTile;
    const int cx = tx + kSppfHalo;
    f32x4 m5 = tile[ty][cx];
#pragma unroll
    for (int d = 1; d <= 2; ++d) m5 = __builtin_elementwise_maximum(m5, __builtin_elementwise_maximum(tile[ty][cx - d], tile[ty][cx + d]));
    f32x4 m9 = m5;
#pragma unroll
    for (int d = 3; d <= 4; ++d) m9 = __builtin_elementwise_maximum(m9, __builtin_elementwise_maximum(tile[ty][cx - d], tile[ty][cx + d]));
    f32x4 m13 = m9;
#pragma unroll
    for (int d = 5; d <= 6; ++d) m13 = __builtin_elementwise_maximum(m13, __builtin_elementwise_maximum(tile[ty][cx - d], tile[ty][cx + d]));
    h5[ty][tx] = m5;
    h9[ty][tx] = m9;
    h13[ty][tx] = m13;
  }
  __syncthreads();
  const int ty = threadIdx.x / kSppfTile, tx = threadIdx.x % kSppfTile;
  const int oy = by * kSppfTile + ty, ox = bx * kSppfTile + tx;
  if (oy >= H || ox >= W) return;
  const int cy = ty + kSppfHalo;
  f32x4 m5 = h5[cy][tx], m9 = h9[cy][tx], m13 = h13[cy][tx];
#pragma unroll
  for (int d = 1; d <= 2; ++d) m5 = __builtin_elementwise_maximum(m5, __builtin_elementwise_maximum(h5[cy - d][tx], h5[cy + d][tx]));
#pragma unroll
  for (int d = 1; d <= 4; ++d) m9 = __builtin_elementwise_maximum(m9, __builtin_elementwise_maximum(h9[cy - d][tx], h9[cy + d][tx]));
#pragma unroll
  for (int d = 1; d <= 6; ++d) m13 = __builtin_elementwise_maximum(m13, __builtin_elementwise_maximum(h13[cy - d][tx], h13[cy + d][tx]));
  const long long pix = ((long long)n * H + oy) * W + ox;
  *(f32x4*)(y5 + pix * ld5 + c) = m5;
  *(f32x4*)(y9 + pix * ld9 + c) = m9;
  *(f32x4*)(y13 + pix * ld13 + c) = m13;
}

// Small planes (the 20x20 SPPF of a 640 input, up to 32x32): one workgroup
// holds a whole image plane of 16 channels in LDS, so every input pixel is
// read from HBM once (the halo tiles above would re-read most of such a
// plane).  Threads are numbered channel group fastest, so each pixel's 64
// contiguous bytes are read and written by four neighbouring lanes.  The
// three pools are chained 5x5 passes (a clipped 5x5 window of a clipped 5x5
// window is the clipped 9x9 window), each a row pass into a second LDS plane
// and a column pass back, written out as it is produced.  Workgroups are
// numbered so that the channel blocks of one image (which share the 128-byte
// lines of its NHWC rows) run on the same XCD (workgroup i runs on XCD i % 8).
// PASSES = 1 is a single MaxPool2d(5, 1, 2) into y5.
constexpr int kSppfPlaneMax = 32 * 32;
constexpr int kSppfCb = 16;  // channels per workgroup
constexpr int kSppfThreads = 1024;
constexpr size_t kSppfLds = 2 * sizeof(f32x4) * (kSppfCb / 4) * kSppfPlaneMax;  // 128 KiB

template <int PASSES>
__global__ __launch_bounds__(kSppfThreads) void sppf_plane_kernel(const float* __restrict__ x, int ldx, int H, int W,
                                                                  int CB, float* __restrict__ y5, int ld5,
                                                                  float* __restrict__ y9, int ld9,
                                                                  float* __restrict__ y13, int ld13) {
  extern __shared__ f32x4 sp[];
  constexpr int G = kSppfCb / 4;  // float4 groups per pixel
  const int HW = H * W, NE = HW * G;
  f32x4* a = sp;       // [HW][G]
  f32x4* t = sp + NE;  // [HW][G]
  const int GR = gridDim.x, L = blockIdx.x;
  const int xcd = L & 7, q8 = GR >> 3, rem = GR & 7;
  const int P = xcd * q8 + (xcd < rem ? xcd : rem) + (L >> 3);
  const int c = (P % CB) * kSppfCb;
  const long long base = (long long)(P / CB) * HW;
  // All of a thread's loads are issued before the first LDS store, so their
  // latencies overlap instead of adding up.
  constexpr int U = 4;
  for (int e0 = 0; e0 < NE; e0 += U * kSppfThreads) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = e0 + u * kSppfThreads + threadIdx.x;
      const int px = e / G, g = e - px * G;
      if (e < NE) v[u] = *(const f32x4*)(x + (base + px) * ldx + c + 4 * g);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = e0 + u * kSppfThreads + threadIdx.x;
      if (e < NE) a[e] = v[u];
    }
  }
  __syncthreads();
  for (int pass = 0; pass < PASSES; ++pass) {
    for (int e = threadIdx.x; e < NE; e += kSppfThreads) {
      const int px = e / G;
      const int xx = px - (px / W) * W;
      f32x4 m = a[e];
#pragma unroll
      for (int d = 1; d <= 2; ++d) {
        if (xx - d >= 0) m = __builtin_elementwise_maximum(m, a[e - d * G]);
        if (xx + d < W) m = __builtin_elementwise_maximum(m, a[e + d * G]);
      }
      t[e] = m;
    }
    __syncthreads();
    float* yo = pass == 0 ? y5 : pass == 1 ? y9 : y13;
    const int ldo = pass == 0 ? ld5 : pass == 1 ? ld9 : ld13;
    for (int e = threadIdx.x; e < NE; e += kSppfThreads) {
      const int px = e / G, g = e - px * G;
      const int py = px / W;
      f32x4 m = t[e];
#pragma unroll
      for (int d = 1; d <= 2; ++d) {
        if (py - d >= 0) m = __builtin_elementwise_maximum(m, t[e - d * W * G]);
        if (py + d < H) m = __builtin_elementwise_maximum(m, t[e + d * W * G]);
      }
      a[e] = m;
      *(f32x4*)(yo + (base + px) * ldo + c + 4 * g) = m;
    }
    __syncthreads();
  }
}

// Launches the whole-plane kernel (P chained 5x5 passes) when the plane and
// channel blocking allow it; false otherwise.
static bool launch_pool5_plane(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5, const sy_tensor* y9,
                               const sy_tensor* y13, int passes) {
  if (x->h * x->w > kSppfPlaneMax || x->c % kSppfCb != 0) return false;
  const size_t lds = 2 * sizeof(f32x4) * (kSppfCb / 4) * (size_t)x->h * x->w;
  // Set once per process (a function-local static: safe across threads).
  static const bool attr_set =
      hipFuncSetAttribute((const void*)sppf_plane_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)kSppfLds) == hipSuccess &&
      hipFuncSetAttribute((const void*)sppf_plane_kernel<3>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)kSppfLds) == hipSuccess;
  if (!attr_set) return false;
  const long long groups = (long long)(x->c / kSppfCb) * x->n;
  if (groups > 0x7fffffff) return false;
  const sy_tensor* z9 = y9 ? y9 : y5;
  const sy_tensor* z13 = y13 ? y13 : y5;
  if (passes == 3)
    hipLaunchKernelGGL(sppf_plane_kernel<3>, dim3((unsigned)groups), dim3(kSppfThreads), lds, ctx->stream, x->data,
                       x->ldc, x->h, x->w, x->c / kSppfCb, y5->data, y5->ldc, z9->data, z9->ldc, z13->data,
                       z13->ldc);
  else
    hipLaunchKernelGGL(sppf_plane_kernel<1>, dim3((unsigned)groups), dim3(kSppfThreads), lds, ctx->stream, x->data,
                       x->ldc, x->h, x->w, x->c / kSppfCb, y5->data, y5->ldc, z9->data, z9->ldc, z13->data,
                       z13->ldc);
  return true;
}

int op_sppf(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5, const sy_tensor* y9, const sy_tensor* y13) {
  SY_TRY(check_view(x, "sppf input"));
  SY_TRY(check_view(y5, "sppf y5"));
  SY_TRY(check_view(y9, "sppf y9"));
  SY_TRY(check_view(y13, "sppf y13"));
  SY_CHECK(same_shape(x, y5) && same_shape(x, y9) && same_shape(x, y13), SY_EINVAL, "sppf outputs must match input");
  if (x->h == 20 && x->w == 20 && x->c % 16 == 0) {
    ProfScope prof(ctx, "sppf_rows20", 0, 4.0 * 4.0 * pixels(*x) * x->c);
    if (launch_pool5_rows20(ctx, x, y5, y9, y13, 3)) return check_launch("sppf_pool");
  }
  if (!(vec4_ok(x) && vec4_ok(y5) && vec4_ok(y9) && vec4_ok(y13))) {
    // Unaligned views: three generic passes give the same values.
    SY_TRY(op_maxpool(ctx, x, y5, 5, 5, 1, 1, 2, 2, 2, 2, 0));
    SY_TRY(op_maxpool(ctx, y5, y9, 5, 5, 1, 1, 2, 2, 2, 2, 0));
    return op_maxpool(ctx, y9, y13, 5, 5, 1, 1, 2, 2, 2, 2, 0);
  }
  SY_CHECK(x->n <= 65535 && x->c / 4 <= 65535, SY_EUNSUPPORTED, "sppf grid too large");
  ProfScope prof(ctx, "sppf_pool", 0, 4.0 * 4.0 * pixels(*x) * x->c);
  if (launch_pool5_plane(ctx, x, y5, y9, y13, 3)) return check_launch("sppf_pool");
  const int tiles = ((x->w + kSppfTile - 1) / kSppfTile) * ((x->h + kSppfTile - 1) / kSppfTile);
  hipLaunchKernelGGL(sppf_kernel, dim3(tiles, x->c / 4, x->n), dim3(256), 0, ctx->stream, x->data, x->ldc, x->n,
                     x->h, x->w, x->c, y5->data, y5->ldc, y9->data, y9->ldc, y13->data, y13->ldc);
  return check_launch("sppf_pool");
}

// ------------------------------------------------------------ head decode

struct DecodeLevel {
  const float* data;
  int ldc, h, w, start;
  float stride;
};
struct DecodeArgs {
  DecodeLevel lv[4];
  int n_levels, N, bins, nc, extra, xyxy, total, vec4;
  float* out;
};

// One workgroup decodes 64 anchors of one level and one image.  The raw head
// rows (4*bins box logits + nc class logits per anchor, NHWC) are read
// coalesced (float4 when the view allows) into LDS rows padded to an odd
// stride, so that the per-anchor reads below (lane = anchor) hit 64 distinct
// banks; 4*64 threads each reduce one side's DFL distribution, then class
// sigmoids and coordinates are written channels-first so stores along the
// anchor axis coalesce.  Coordinate arithmetic follows CpuHead.cs:114-121
// exactly (no contraction).
constexpr int kDecAnchors = 64;

__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float sm[];
  const int C = 4 * a.bins + a.nc + a.extra;
  const int LD = C | 1;                      // odd row stride: conflict-free columns
  float* rows = sm;                          // [64][LD]
  float* dist = sm + kDecAnchors * LD;       // [4][64]
  // Locate level and anchor block.
  int blk = blockIdx.x, li = 0;
  for (; li < a.n_levels; ++li) {
    const int hw = a.lv[li].h * a.lv[li].w;
    const int nb = (hw + kDecAnchors - 1) / kDecAnchors;
    if (blk < nb) break;
    blk -= nb;
  }
  if (li >= a.n_levels) return;
  const DecodeLevel L = a.lv[li];
  const int hw = L.h * L.w;
  const int n = blockIdx.y;
  const int a0 = blk * kDecAnchors;
  const int cnt = min(kDecAnchors, hw - a0);
  const float* src = L.data + ((long long)n * hw + a0) * L.ldc;
  if (a.vec4) {
    // All of a thread's float4 loads (up to 12: 64 anchors x 48 float4s) are
    // issued before the first LDS store, from clamped in-range addresses, so
    // their latencies overlap instead of adding up.
    constexpr int U = 12;
    const int QC = C >> 2, NQ = cnt * QC;
    for (int i0 = 0; i0 < NQ; i0 += U * 256) {
      f32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = min(i0 + u * 256 + (int)threadIdx.x, NQ - 1);
        const int r = i / QC, q = i - r * QC;
        v[u] = *(const f32x4*)(src + (long long)r * L.ldc + 4 * q);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * 256 + (int)threadIdx.x;
        if (i < NQ) {
          const int r = i / QC, q = i - r * QC;
          float* d = rows + r * LD + 4 * q;
          d[0] = v[u][0];
          d[1] = v[u][1];
          d[2] = v[u][2];
          d[3] = v[u][3];
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < cnt * C; i += blockDim.x) {
      const int r = i / C, ch = i - r * C;
      rows[r * LD + ch] = src[(long long)r * L.ldc + ch];
    }
  }
  __syncthreads();
  {
    const int r = threadIdx.x & 63, side = threadIdx.x >> 6;
    if (r < cnt) {
      const float* v = rows + r * LD + side * a.bins;
      float d;
      if (a.bins == 1) {
        d = v[0];
      } else {
        float mx = -INFINITY;
        for (int b = 0; b < a.bins; ++b) mx = fmaxf(mx, v[b]);
        float s = 0.f, num = 0.f;
        for (int b = 0; b < a.bins; ++b) {
          const float e = __expf(v[b] - mx);
          s += e;
          num += e * (float)b;
        }
        d = num / s;
      }
      dist[side * kDecAnchors + r] = d;
    }
  }
  __syncthreads();
  float* ob = a.out + (long long)n * (a.nc + 4 + a.extra) * a.total + L.start + a0;
  {
    const int r = threadIdx.x & 63;
    if (r < cnt) {
      const float* zr = rows + r * LD + 4 * a.bins;
      for (int c = threadIdx.x >> 6; c < a.nc; c += 4)
        ob[(long long)(4 + c) * a.total + r] = 1.0f / (1.0f + __expf(-zr[c]));
      // Extra per-anchor channels (mask coefficients) pass through raw.
      for (int c = threadIdx.x >> 6; c < a.extra; c += 4)
        ob[(long long)(4 + a.nc + c) * a.total + r] = zr[a.nc + c];
    }
  }
  if (threadIdx.x < cnt) {
    const int r = threadIdx.x;
    const int an = a0 + r;
    const float cx = (float)(an % L.w) + .5f, cy = (float)(an / L.w) + .5f;
    const float s = L.stride;
    const float x1 = (cx - dist[r]) * s, y1 = (cy - dist[kDecAnchors + r]) * s;
    const float x2 = (cx + dist[2 * kDecAnchors + r]) * s, y2 = (cy + dist[3 * kDecAnchors + r]) * s;
    ob[r] = a.xyxy ? x1 : (x1 + x2) * .5f;
    ob[(long long)a.total + r] = a.xyxy ? y1 : (y1 + y2) * .5f;
    ob[2LL * a.total + r] = a.xyxy ? x2 : x2 - x1;
    ob[3LL * a.total + r] = a.xyxy ? y2 : y2 - y1;
  }
}

int op_detect_decode(sy_ctx* ctx, const sy_tensor* levels, const float* strides, int n_levels, int bins, int nc,
                     int xyxy, float* out, int total) {
  SY_CHECK(levels && strides && out, SY_EINVAL, "null argument");
  SY_CHECK(n_levels >= 1 && n_levels <= 4, SY_EUNSUPPORTED, "1..4 head levels supported, got %d", n_levels);
  SY_CHECK(bins >= 1 && nc >= 0, SY_EINVAL, "invalid bins/classes");
  SY_CHECK(levels[0].c >= 4 * bins + nc, SY_EINVAL, "head level has %d channels, fewer than 4*bins + nc = %d",
           levels[0].c, 4 * bins + nc);
  const int C = levels[0].c;  // 4*bins + nc + extra pass-through channels
  SY_CHECK(C <= 240, SY_EUNSUPPORTED, "head with %d channels per anchor exceeds the decode tile", C);
  DecodeArgs a;
  a.n_levels = n_levels;
  a.bins = bins;
  a.nc = nc;
  a.extra = C - 4 * bins - nc;
  a.xyxy = xyxy ? 1 : 0;
  a.total = total;
  a.out = out;
  a.N = levels[0].n;
  int start = 0, blocks = 0;
  for (int i = 0; i < n_levels; ++i) {
    SY_TRY(check_view(&levels[i], "head level"));
    SY_CHECK(levels[i].c == C, SY_EINVAL, "head level %d has %d channels, expected %d", i, levels[i].c, C);
    SY_CHECK(levels[i].n == a.N, SY_EINVAL, "head levels differ in batch");
    a.lv[i] = DecodeLevel{levels[i].data, levels[i].ldc, levels[i].h, levels[i].w, start, strides[i]};
    const int hw = levels[i].h * levels[i].w;
    start += hw;
    blocks += (hw + kDecAnchors - 1) / kDecAnchors;
  }
  SY_CHECK(start == total, SY_EINVAL, "levels hold %d anchors, output expects %d", start, total);
  a.vec4 = C % 4 == 0;
  for (int i = 0; i < n_levels; ++i)
    if (((uintptr_t)levels[i].data & 15) != 0 || levels[i].ldc % 4 != 0) a.vec4 = 0;
  const size_t lds = (size_t)(kDecAnchors * (C | 1) + 4 * kDecAnchors) * sizeof(float);
  ProfScope prof(ctx, "detect_decode", 0, 4.0 * (double)a.N * total * (C + nc + 4 + a.extra));
  hipLaunchKernelGGL(decode_kernel, dim3(blocks, a.N), dim3(256), lds, ctx->stream, a);
  return check_launch("detect_decode");
}

}  // namespace sy
