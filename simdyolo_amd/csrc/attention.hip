// Multi-head attention core of the C2PSA block (PtModel.Attention,
// src/SimdYolo/PtModel.cs:429-437): from the qkv 1x1 conv output, viewed as
// [B, heads, 2*kd + hd, N], compute S = q^T k * scale, softmax over the last
// axis, o = v S^T, written as an NHWC [B, heads*hd, H, W] view; also emits v
// as a dense NHWC tensor for the depthwise `pe` conv.  The reference runs
// this as DeviceMatMul + Scale (op 4) + Softmax (op 25) + DeviceMatMul
// (VulkanExecution.cs:499-541, tensor.comp:62-68).
//
// Both products run on the FP32-MFMA GEMM (gemm_nt); S rows and V^T rows are
// padded to N4 = round_up(N, 4) with zeros so K stays a multiple of 4.
#include <cmath>

#include "sy_internal.h"

namespace sy {

// One wavefront per row: y = softmax(x * scale) over n entries (max-subtracted),
// zeroing the padding columns [n, ld).
__global__ __launch_bounds__(256) void softmax_rows_kernel(float* __restrict__ s, long long rows, int n, int ld,
                                                           float scale) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  float* r = s + row * ld;
  float mx = -INFINITY;
  for (int j = lane; j < n; j += 64) mx = fmaxf(mx, r[j] * scale);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float sum = 0.f;
  for (int j = lane; j < n; j += 64) {
    const float e = expf(r[j] * scale - mx);
    r[j] = e;
    sum += e;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const float inv = 1.0f / sum;
  for (int j = lane; j < n; j += 64) r[j] *= inv;
  for (int j = n + lane; j < ld; j += 64) r[j] = 0.f;
}

// v of head h -> vt[b][h][d][j] (rows padded to ld with zeros) and the dense
// NHWC copy vd[b][j][h*hd + d].
__global__ __launch_bounds__(256) void split_v_kernel(const float* __restrict__ qkv, int ldq, int N, int heads,
                                                      int kd, int hd, int B, float* __restrict__ vt, int ld,
                                                      float* __restrict__ vd, int ldv) {
  const long long total = (long long)B * heads * hd * ld;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int j = (int)(i % ld);
  const long long r = i / ld;
  const int d = (int)(r % hd);
  const long long bh = r / hd;
  const int h = (int)(bh % heads);
  const long long b = bh / heads;
  float v = 0.f;
  if (j < N) {
    v = qkv[(b * N + j) * ldq + h * (2 * kd + hd) + 2 * kd + d];
    vd[(b * N + j) * ldv + h * hd + d] = v;
  }
  vt[i] = v;
}

int op_attention(sy_ctx* ctx, const sy_tensor* qkv, int heads, int kd, int hd, float scale, const sy_tensor* o,
                 const sy_tensor* v) {
  SY_TRY(check_view(qkv, "attention qkv"));
  SY_TRY(check_view(o, "attention output"));
  SY_TRY(check_view(v, "attention v"));
  SY_CHECK(heads > 0 && kd > 0 && hd > 0, SY_EINVAL, "invalid attention geometry");
  const int per = 2 * kd + hd;
  SY_CHECK(qkv->c == heads * per, SY_EINVAL, "qkv has %d channels, expected heads*(2*kd+hd) = %d", qkv->c,
           heads * per);
  const int B = qkv->n, N = qkv->h * qkv->w, C = heads * hd;
  SY_CHECK(o->n == B && o->c == C && o->h == qkv->h && o->w == qkv->w, SY_EINVAL, "attention output shape mismatch");
  SY_CHECK(v->n == B && v->c == C && v->h == qkv->h && v->w == qkv->w, SY_EINVAL, "attention v shape mismatch");
  SY_CHECK(qkv->ldc == qkv->c || qkv->ldc % 4 == 0, SY_EINVAL, "qkv view stride");
  SY_CHECK(kd % 4 == 0 && per % 4 == 0 && hd % 4 == 0, SY_EUNSUPPORTED,
           "attention needs key/head dims that are multiples of 4");
  const int N4 = (N + 3) / 4 * 4;
  const size_t s_floats = (size_t)B * heads * N * N4, vt_floats = (size_t)B * heads * hd * N4;
  SY_TRY(ensure_scratch(ctx, (s_floats + vt_floats) * sizeof(float) + 512));
  float* S = (float*)ctx->scratch;
  float* Vt = S + ((s_floats + 63) / 64 * 64);
  {
    const long long total = (long long)B * heads * hd * N4;
    ProfScope prof(ctx, "attn_split_v", 0, 4.0 * (double)B * N * C * 3);
    hipLaunchKernelGGL(split_v_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream, qkv->data,
                       qkv->ldc, N, heads, kd, hd, B, Vt, N4, v->data, v->ldc);
    SY_TRY(check_launch("attn_split_v"));
  }
  for (int h = 0; h < heads; ++h) {
    const float* q = qkv->data + h * per;
    SY_TRY(gemm_nt(ctx, q, N, kd, qkv->ldc, q + kd, N, qkv->ldc, S + (size_t)h * N * N4, N4, "attn_qk", B,
                   (long long)N * qkv->ldc, (long long)N * qkv->ldc, (long long)heads * N * N4));
  }
  {
    const long long rows = (long long)B * heads * N;
    ProfScope prof(ctx, "attn_softmax", 4.0 * rows * N, 8.0 * rows * N4);
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, ctx->stream, S, rows, N,
                       N4, scale);
    SY_TRY(check_launch("attn_softmax"));
  }
  for (int h = 0; h < heads; ++h)
    SY_TRY(gemm_nt(ctx, S + (size_t)h * N * N4, N, N4, N4, Vt + (size_t)h * hd * N4, hd, N4, o->data + h * hd,
                   o->ldc, "attn_av", B, (long long)heads * N * N4, (long long)heads * hd * N4,
                   (long long)N * o->ldc));
  return SY_OK;
}

size_t attention_scratch_bytes(int B, int H, int W, int heads, int hd) {
  const size_t N = (size_t)H * W, N4 = (N + 3) / 4 * 4;
  return ((size_t)B * heads * N * N4 + 64 + (size_t)B * heads * hd * N4) * sizeof(float) + 512;
}

}  // namespace sy

extern "C" int sy_attention(sy_ctx* ctx, const sy_tensor* qkv, int heads, int key_dim, int head_dim, float scale,
                            const sy_tensor* o, const sy_tensor* v) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return sy::op_attention(ctx, qkv, heads, key_dim, head_dim, scale, o, v);
}
