// Context, frame arena, memory, graphs, timing and the C ABI for the op layer.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>

#include "host_copy.h"
#include "sy_internal.h"

namespace sy {

static thread_local char g_error[1024] = "";

std::shared_timed_mutex& capture_lock() {
  static std::shared_timed_mutex m;
  return m;
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
}

int check_launch(const char* name) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("kernel %s launch failed: %s (%d)", name, hipGetErrorString(e), (int)e);
    return SY_EDEVICE;
  }
  return SY_OK;
}

int check_view(const sy_tensor* t, const char* what, bool allow_nchw) {
  SY_CHECK(t != nullptr, SY_EINVAL, "%s: null tensor", what);
  SY_CHECK(t->data != nullptr, SY_EINVAL, "%s: null data pointer", what);
  SY_CHECK(t->n > 0 && t->c > 0 && t->h > 0 && t->w > 0, SY_EINVAL, "%s: non-positive shape %dx%dx%dx%d", what,
           t->n, t->c, t->h, t->w);
  if (t->layout == SY_LAYOUT_NCHW) {
    SY_CHECK(allow_nchw, SY_EUNSUPPORTED, "%s: NCHW layout is only accepted by the direct stem conv", what);
  } else {
    SY_CHECK(t->layout == SY_LAYOUT_NHWC, SY_EINVAL, "%s: unknown layout %d", what, t->layout);
    SY_CHECK(t->ldc >= t->c, SY_EINVAL, "%s: ldc %d < c %d", what, t->ldc, t->c);
  }
  return SY_OK;
}

int ensure_host_stage(sy_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->host_stage_size) return SY_OK;
  SY_CHECK(!ctx->capturing, SY_ESTATE, "host staging needed during graph capture");
  if (ctx->host_stage) {
    SY_HIP(hipStreamSynchronize(ctx->stream));
    SY_HIP(hipHostFree(ctx->host_stage));
    ctx->host_stage = nullptr;
    ctx->host_stage_size = 0;
  }
  const size_t sz = (bytes + (1u << 16) - 1) & ~size_t((1u << 16) - 1);
  SY_HIP(hipHostMalloc((void**)&ctx->host_stage, sz, hipHostMallocDefault));
  ctx->host_stage_size = sz;
  return SY_OK;
}

int ensure_scratch(sy_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->scratch_size) return SY_OK;
  SY_CHECK(!ctx->capturing, SY_ESTATE,
           "scratch of %zu bytes needed during graph capture (have %zu); run the op once before capturing", bytes,
           ctx->scratch_size);
  if (ctx->scratch) {
    SY_HIP(hipStreamSynchronize(ctx->stream));
    SY_HIP(hipFree(ctx->scratch));
    ctx->scratch = nullptr;
    ctx->scratch_size = 0;
  }
  size_t sz = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
  SY_HIP(hipMalloc((void**)&ctx->scratch, sz));
  ctx->scratch_size = sz;
  ++ctx->scratch_gen;  // graphs captured before now hold the old address
  return SY_OK;
}

struct HostStage {
  static constexpr size_t kPiece = size_t(8) << 20;  // bytes per slot
  static constexpr int kSlots = 3;
  char* pin[kSlots] = {};
  hipEvent_t ev[kSlots] = {};
  bool used[kSlots] = {};
  int next = 0;
  std::unique_ptr<CopyPool> pool;
  ~HostStage() {
    for (int i = 0; i < kSlots; ++i) {
      if (ev[i]) (void)hipEventSynchronize(ev[i]);
      if (pin[i]) (void)hipHostFree(pin[i]);
      if (ev[i]) (void)hipEventDestroy(ev[i]);
    }
  }
  // Bytes per piece: a quarter of the copy (so that even a single image's
  // copy overlaps host copies with DMA), 1 to 8 MiB.
  static size_t piece(size_t bytes) {
    const size_t q = (bytes / 4 + (size_t(1) << 18) - 1) & ~((size_t(1) << 18) - 1);
    return std::min(kPiece, std::max(size_t(1) << 20, q));
  }
  // The next slot, once the host may touch it again.
  int take(int* out) {
    const int s = next;
    next = (next + 1) % kSlots;
    if (used[s]) SY_HIP(hipEventSynchronize(ev[s]));
    used[s] = true;
    *out = s;
    return SY_OK;
  }
};

static int ensure_stage(sy_ctx* ctx) {
  if (ctx->stage) return SY_OK;
  auto st = std::make_unique<HostStage>();
  for (int i = 0; i < HostStage::kSlots; ++i) {
    SY_HIP(hipHostMalloc((void**)&st->pin[i], HostStage::kPiece, hipHostMallocDefault));
    SY_HIP(hipEventCreateWithFlags(&st->ev[i], hipEventDisableTiming));
  }
  const unsigned hw = std::thread::hardware_concurrency();
  st->pool = std::make_unique<CopyPool>((int)std::min(5u, hw > 4 ? hw / 3 : 0u));
  ctx->stage = st.release();
  return SY_OK;
}

int staged_h2d(sy_ctx* ctx, void* dst, const void* src, size_t bytes) {
  SY_TRY(ensure_stage(ctx));
  HostStage& st = *ctx->stage;
  const size_t piece = HostStage::piece(bytes);
  for (size_t off = 0; off < bytes; off += piece) {
    const size_t len = std::min(piece, bytes - off);
    int s = 0;
    SY_TRY(st.take(&s));
    st.pool->copy(st.pin[s], (const char*)src + off, len);
    SY_HIP(hipMemcpyAsync((char*)dst + off, st.pin[s], len, hipMemcpyHostToDevice, ctx->stream));
    SY_HIP(hipEventRecord(st.ev[s], ctx->stream));
  }
  return SY_OK;
}

int staged_d2h(sy_ctx* ctx, void* dst, const void* src, size_t bytes) {
  SY_TRY(ensure_stage(ctx));
  HostStage& st = *ctx->stage;
  const size_t piece = HostStage::piece(bytes);
  const size_t n = (bytes + piece - 1) / piece;
  // Up to kSlots pieces in flight; the host empties them in order (piece p
  // reuses the slot of piece p - kSlots, which it has emptied already).
  std::vector<int> slot(n);
  size_t issued = 0;
  for (size_t done = 0; done < n; ++done) {
    for (; issued < n && issued < done + HostStage::kSlots; ++issued) {
      const size_t off = issued * piece;
      SY_TRY(st.take(&slot[issued]));
      SY_HIP(hipMemcpyAsync(st.pin[slot[issued]], (const char*)src + off, std::min(piece, bytes - off),
                            hipMemcpyDeviceToHost, ctx->stream));
      SY_HIP(hipEventRecord(st.ev[slot[issued]], ctx->stream));
    }
    const size_t off = done * piece;
    SY_HIP(hipEventSynchronize(st.ev[slot[done]]));
    st.pool->copy((char*)dst + off, st.pin[slot[done]], std::min(piece, bytes - off));
  }
  return SY_OK;
}

static hipEvent_t take_event(sy_ctx* ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void prof_begin(sy_ctx* ctx, const char* name, double flops, double bytes) {
  PendingEvent p;
  p.name = name;
  if (ctx->profile_shapes && !ctx->prof_tag.empty()) p.name += " " + ctx->prof_tag;
  p.flops = flops;
  p.bytes = bytes;
  p.start = take_event(ctx);
  p.stop = take_event(ctx);
  if (p.start) (void)hipEventRecord(p.start, ctx->stream);
  ctx->pending.push_back(p);
}

void prof_end(sy_ctx* ctx) {
  if (ctx->pending.empty()) return;
  PendingEvent& p = ctx->pending.back();
  if (p.stop) (void)hipEventRecord(p.stop, ctx->stream);
}

int prof_collect(sy_ctx* ctx) {
  if (ctx->pending.empty()) return SY_OK;
  SY_HIP(hipStreamSynchronize(ctx->stream));
  for (auto& p : ctx->pending) {
    float ms = 0;
    if (p.start && p.stop && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      auto& e = ctx->profile[p.name];
      e.count += 1;
      e.ms += ms;
      e.flops += p.flops;
      e.bytes += p.bytes;
    }
    if (p.start) ctx->event_pool.push_back(p.start);
    if (p.stop) ctx->event_pool.push_back(p.stop);
  }
  ctx->pending.clear();
  return SY_OK;
}

int64_t pool_out_size(int len, int k, int s, int before, int after, int ceil_mode) {
  int64_t num = (int64_t)len + before + after - k;
  if (ceil_mode) num += s - 1;
  if (num < 0) return -1;
  int64_t size = num / s + 1;
  if (ceil_mode) {
    int64_t lim = ((int64_t)len + before + s - 1) / s;
    if (lim < size) size = lim;
  }
  return size;
}

}  // namespace sy

using namespace sy;

extern "C" {

const char* sy_last_error(void) { return g_error; }

const char* sy_version(void) { return "simdyolo-hip 0.1 (gfx950)"; }

int sy_device_count(int* count) {
  SY_CHECK(count, SY_EINVAL, "null count");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return SY_OK;
}

int sy_create(int device, sy_ctx** out) {
  SY_CHECK(out, SY_EINVAL, "null output");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    set_error("no HIP device available");
    return SY_EDEVICE;
  }
  SY_CHECK(device >= 0 && device < n, SY_EINVAL, "device %d out of range (have %d)", device, n);
  SY_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  SY_HIP(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0) {
    set_error("device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    return SY_EUNSUPPORTED;
  }
  SY_TRY(topk_static_init(device));
  auto ctx = new sy_ctx();
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  ctx->name = std::string("HIP ") + prop.name + " (" + arch + ", " + std::to_string(prop.multiProcessorCount) +
              " CUs)";
  hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&ctx->t0);
  if (e == hipSuccess) e = hipEventCreate(&ctx->t1);
  if (e != hipSuccess) {
    set_error("stream/event creation failed: %s", hipGetErrorString(e));
    delete ctx;
    return SY_EDEVICE;
  }
  *out = ctx;
  return SY_OK;
}

void sy_destroy(sy_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->capturing) {  // a capture left open: end it and release its share of the lock
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(ctx->stream, &g);
    if (g) (void)hipGraphDestroy(g);
    ctx->capturing = false;
    capture_lock().unlock_shared();
  }
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  for (auto g : ctx->graphs)
    if (g) (void)hipGraphExecDestroy(g);
  for (auto& p : ctx->pending) {
    if (p.start) (void)hipEventDestroy(p.start);
    if (p.stop) (void)hipEventDestroy(p.stop);
  }
  for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
  for (auto* p : ctx->owned) (void)hipFree(p);
  ctx->convs.clear();
  if (ctx->side) (void)hipStreamSynchronize(ctx->side);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->side_scratch) (void)hipFree(ctx->side_scratch);
  if (ctx->host_stage) (void)hipHostFree(ctx->host_stage);
  delete ctx->stage;
  for (auto& b : ctx->blocks) (void)hipFree(b.first);
  if (ctx->t0) (void)hipEventDestroy(ctx->t0);
  if (ctx->t1) (void)hipEventDestroy(ctx->t1);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  if (ctx->side) (void)hipStreamDestroy(ctx->side);
  delete ctx;
}

const char* sy_name(const sy_ctx* ctx) { return ctx ? ctx->name.c_str() : "HIP (no context)"; }

int sy_frame_begin(sy_ctx* ctx, int64_t* frame_id) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_CHECK(!ctx->frame_active, SY_ESTATE, "a frame is already active");
  ctx->frame_active = true;
  ctx->frame_id += 1;
  ctx->block = 0;
  ctx->block_used = 0;
  if (frame_id) *frame_id = ctx->frame_id;
  return SY_OK;
}

int sy_frame_end(sy_ctx* ctx) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_CHECK(ctx->frame_active, SY_ESTATE, "no active frame");
  ctx->frame_active = false;
  SY_HIP(hipStreamSynchronize(ctx->stream));
  return prof_collect(ctx);
}

int sy_flush(sy_ctx* ctx) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_HIP(hipStreamSynchronize(ctx->stream));
  return prof_collect(ctx);
}

int sy_frame_alloc(sy_ctx* ctx, int n, int c, int h, int w, sy_tensor* out) {
  SY_CHECK(ctx && out, SY_EINVAL, "null argument");
  SY_CHECK(ctx->frame_active, SY_ESTATE, "frame allocation outside a frame");
  SY_CHECK(n > 0 && c > 0 && h > 0 && w > 0, SY_EINVAL, "non-positive shape");
  const size_t bytes = (size_t)n * c * h * w * sizeof(float);
  // First fit in the current block, then later blocks, else a new block
  // (VulkanExecution.cs:137-160 chains 32 MiB blocks the same way).
  while (ctx->block < ctx->blocks.size()) {
    size_t off = (ctx->block_used + 255) & ~size_t(255);
    if (off + bytes <= ctx->blocks[ctx->block].second) {
      ctx->block_used = off + bytes;
      *out = sy_tensor{(float*)(ctx->blocks[ctx->block].first + off), n, c, h, w, c, SY_LAYOUT_NHWC};
      return SY_OK;
    }
    ++ctx->block;
    ctx->block_used = 0;
  }
  SY_CHECK(!ctx->capturing, SY_ESTATE, "frame arena exhausted during graph capture");
  const size_t sz = bytes < (size_t)(32u << 20) ? (size_t)(32u << 20) : ((bytes + 255) & ~size_t(255));
  char* p = nullptr;
  SY_HIP(hipMalloc((void**)&p, sz));
  ctx->blocks.emplace_back(p, sz);
  ctx->block = ctx->blocks.size() - 1;
  ctx->block_used = bytes;
  *out = sy_tensor{(float*)p, n, c, h, w, c, SY_LAYOUT_NHWC};
  return SY_OK;
}

int sy_malloc(sy_ctx* ctx, size_t bytes, void** ptr) {
  SY_CHECK(ctx && ptr, SY_EINVAL, "null argument");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "allocation during graph capture");
  SY_HIP(hipSetDevice(ctx->device));
  SY_HIP(hipMalloc(ptr, bytes ? bytes : 1));
  return SY_OK;
}

int sy_free(sy_ctx* ctx, void* ptr) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  if (!ptr) return SY_OK;
  SY_HIP(hipStreamSynchronize(ctx->stream));
  SY_HIP(hipFree(ptr));
  return SY_OK;
}

int sy_memcpy(sy_ctx* ctx, void* dst, const void* src, size_t bytes, int kind) {
  SY_CHECK(ctx && (bytes == 0 || (dst && src)), SY_EINVAL, "null argument");
  if (bytes == 0) return SY_OK;
  SY_CHECK(kind >= 0 && kind <= 2, SY_EINVAL, "bad copy kind %d", kind);
  // A host copy waits for the stream, which a capture cannot do: refuse it
  // before anything is recorded, so the capture stays valid.
  SY_CHECK(kind == 2 || !ctx->capturing, SY_ESTATE, "host copy during graph capture");
  // Large host copies go through the pinned staging, which returns once the
  // caller's buffer has been read or written.
  if (kind == 0 && bytes >= kStageMin) return staged_h2d(ctx, dst, src, bytes);
  if (kind == 1 && bytes >= kStageMin) return staged_d2h(ctx, dst, src, bytes);
  hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  SY_HIP(hipMemcpyAsync(dst, src, bytes, k, ctx->stream));
  // Host buffers are caller-owned (a managed array is pinned only for the
  // call): wait until the copy has read or written them.
  if (kind != 2) SY_HIP(hipStreamSynchronize(ctx->stream));
  return SY_OK;
}

int sy_upload_nchw(sy_ctx* ctx, const float* host, const sy_tensor* dst) {
  SY_CHECK(ctx && host, SY_EINVAL, "null argument");
  SY_TRY(check_view(dst, "upload destination", true));
  SY_CHECK(!ctx->capturing, SY_ESTATE, "host upload during graph capture");
  size_t count = (size_t)dst->n * dst->c * dst->h * dst->w;
  // Returns once the host buffer has been read (as sy_memcpy).
  if (dst->layout == SY_LAYOUT_NCHW) return sy_memcpy(ctx, dst->data, host, count * 4, 0);
  SY_TRY(ensure_scratch(ctx, count * 4));
  SY_TRY(sy_memcpy(ctx, ctx->scratch, host, count * 4, 0));
  return op_nchw_to_view(ctx, (const float*)ctx->scratch, dst);
}

int sy_download_nchw(sy_ctx* ctx, const sy_tensor* src, float* host) {
  SY_CHECK(ctx && host, SY_EINVAL, "null argument");
  SY_TRY(check_view(src, "download source", true));
  SY_CHECK(!ctx->capturing, SY_ESTATE, "host download during graph capture");
  size_t count = (size_t)src->n * src->c * src->h * src->w;
  if (src->layout == SY_LAYOUT_NCHW) return sy_memcpy(ctx, host, src->data, count * 4, 1);
  SY_TRY(ensure_scratch(ctx, count * 4));
  SY_TRY(op_view_to_nchw(ctx, src, (float*)ctx->scratch));
  return sy_memcpy(ctx, host, ctx->scratch, count * 4, 1);
}

// ------------------------------------------------------------- conv ABI

static ConvPlan* find_conv(sy_ctx* ctx, uint64_t id) {
  if (!ctx || id == 0 || id > ctx->convs.size()) return nullptr;
  return ctx->convs[id - 1].get();
}

int sy_conv_create(sy_ctx* ctx, const float* weight, const float* bias, int oc, int ic, int kh, int kw, int sh,
                   int sw, int pt, int pl, int pb, int pr, int dh, int dw, int groups, int silu, uint64_t* conv) {
  SY_CHECK(ctx && weight && conv, SY_EINVAL, "null argument");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "conv preparation during graph capture");
  SY_CHECK(oc > 0 && ic > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && dh > 0 && dw > 0 && groups > 0, SY_EINVAL,
           "invalid convolution parameters");
  SY_CHECK(pt >= 0 && pl >= 0 && pb >= 0 && pr >= 0, SY_EINVAL, "negative padding");
  SY_CHECK(ic % groups == 0 && oc % groups == 0, SY_EINVAL, "channels not divisible by groups");
  auto p = std::make_unique<ConvPlan>();
  p->oc = oc; p->ic = ic; p->kh = kh; p->kw = kw; p->sh = sh; p->sw = sw;
  p->pt = pt; p->pl = pl; p->pb = pb; p->pr = pr; p->dh = dh; p->dw = dw;
  p->groups = groups; p->silu = silu ? 1 : 0;
  size_t wn = (size_t)oc * (ic / groups) * kh * kw;
  p->host_w.assign(weight, weight + wn);
  p->host_b.assign((size_t)oc, 0.0f);
  if (bias) p->host_b.assign(bias, bias + oc);
  p->algo = kAuto;
  SY_HIP(hipSetDevice(ctx->device));
  SY_TRY(conv_prepare(ctx, p.get()));
  ctx->convs.push_back(std::move(p));
  *conv = ctx->convs.size();
  return SY_OK;
}

int sy_conv_transpose2x2_create(sy_ctx* ctx, const float* weight, const float* bias, int ic, int oc,
                                uint64_t* conv) {
  SY_CHECK(ctx && weight && conv, SY_EINVAL, "null argument");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "conv preparation during graph capture");
  SY_CHECK(ic > 0 && oc > 0, SY_EINVAL, "invalid transposed convolution channels");
  auto p = std::make_unique<ConvPlan>();
  // A 1x1 conv over 4 * oc virtual channels (q * oc + o, q = 2 dy + dx).
  const int ocv = 4 * oc;
  p->oc = ocv; p->ic = ic; p->kh = p->kw = 1; p->sh = p->sw = 1;
  p->pt = p->pl = p->pb = p->pr = 0; p->dh = p->dw = 1;
  p->groups = 1; p->silu = 0; p->up2 = oc;
  p->host_w.assign((size_t)ocv * ic, 0.0f);
  p->host_b.assign((size_t)ocv, 0.0f);
  for (int c = 0; c < ic; ++c)
    for (int o = 0; o < oc; ++o)
      for (int q = 0; q < 4; ++q) p->host_w[(size_t)(q * oc + o) * ic + c] = weight[((size_t)c * oc + o) * 4 + q];
  if (bias)
    for (int q = 0; q < 4; ++q)
      for (int o = 0; o < oc; ++o) p->host_b[(size_t)q * oc + o] = bias[o];
  p->algo = kIgemm;
  SY_HIP(hipSetDevice(ctx->device));
  SY_TRY(conv_prepare(ctx, p.get()));
  ctx->convs.push_back(std::move(p));
  *conv = ctx->convs.size();
  return SY_OK;
}

int sy_conv_set_algo(sy_ctx* ctx, uint64_t conv, int algo) {
  ConvPlan* p = find_conv(ctx, conv);
  SY_CHECK(p, SY_EINVAL, "unknown conv handle %llu", (unsigned long long)conv);
  SY_CHECK(!ctx->capturing, SY_ESTATE, "algorithm change during capture");
  SY_CHECK(algo >= 0 && algo <= 6, SY_EINVAL, "unknown algorithm %d", algo);
  if (algo != kAuto) SY_CHECK(conv_supports(p, algo), SY_EUNSUPPORTED, "algorithm %d cannot run this conv", algo);
  p->algo = algo;
  p->user_algo = algo != kAuto;
  p->tuned.clear();
  return conv_prepare(ctx, p);
}

int sy_conv_get_algo(sy_ctx* ctx, uint64_t conv, int* algo) {
  ConvPlan* p = find_conv(ctx, conv);
  SY_CHECK(p && algo, SY_EINVAL, "unknown conv handle");
  *algo = p->algo;
  return SY_OK;
}

int sy_conv_out_size(sy_ctx* ctx, uint64_t conv, int h, int w, int* oh, int* ow) {
  ConvPlan* p = find_conv(ctx, conv);
  SY_CHECK(p && oh && ow, SY_EINVAL, "unknown conv handle");
  conv_out_size(p, h, w, oh, ow);
  SY_CHECK(*oh > 0 && *ow > 0, SY_EINVAL, "kernel exceeds the padded input");
  return SY_OK;
}

int sy_conv_run(sy_ctx* ctx, uint64_t conv, const sy_tensor* x, const sy_tensor* y, const sy_tensor* residual) {
  ConvPlan* p = find_conv(ctx, conv);
  SY_CHECK(p, SY_EINVAL, "unknown conv handle %llu", (unsigned long long)conv);
  return conv_run(ctx, p, x, y, residual);
}

int sy_conv_run_upsampled(sy_ctx* ctx, uint64_t conv, const sy_tensor* xu, const sy_tensor* x,
                          const sy_tensor* y, const sy_tensor* residual) {
  ConvPlan* p = find_conv(ctx, conv);
  SY_CHECK(p, SY_EINVAL, "unknown conv handle %llu", (unsigned long long)conv);
  return conv_run_upsampled(ctx, p, xu, x, y, residual);
}

int sy_tune_save(sy_ctx* ctx, const char* path) {
  SY_CHECK(ctx && path, SY_EINVAL, "null argument");
  return tune_save(ctx, path);
}

int sy_tune_load(sy_ctx* ctx, const char* path) {
  SY_CHECK(ctx && path, SY_EINVAL, "null argument");
  return tune_load(ctx, path);
}

// ------------------------------------------------------------- op ABI

int sy_add(sy_ctx* ctx, const sy_tensor* a, const sy_tensor* b, const sy_tensor* y) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_add(ctx, a, b, y);
}

int sy_resize_nearest(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_resize_nearest(ctx, x, y);
}

int sy_maxpool(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y, int kh, int kw, int sh, int sw, int pt, int pl,
               int pb, int pr, int ceil_mode) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_maxpool(ctx, x, y, kh, kw, sh, sw, pt, pl, pb, pr, ceil_mode);
}

int sy_sppf_pool(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5, const sy_tensor* y9, const sy_tensor* y13) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_sppf(ctx, x, y5, y9, y13);
}

int sy_copy(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_copy(ctx, x, y);
}

int sy_detect_decode(sy_ctx* ctx, const sy_tensor* levels, const float* strides, int n_levels, int bins, int nc,
                     int xyxy, float* out, int total_anchors) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_detect_decode(ctx, levels, strides, n_levels, bins, nc, xyxy, out, total_anchors);
}

int sy_e2e_topk(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum,
                int onnx_rules, float* out) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_e2e_topk(ctx, head, batch, channels, anchors, nc, maximum, onnx_rules, out);
}

int sy_e2e_topk_noalloc(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum,
                        int onnx_rules, float* out) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  return op_e2e_topk_noalloc(ctx, head, batch, channels, anchors, nc, maximum, onnx_rules, out);
}

// ------------------------------------------------------------- graphs

int sy_graph_begin(sy_ctx* ctx) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "capture already active");
  SY_CHECK(!ctx->profiling, SY_ESTATE, "per-kernel profiling cannot be captured");
  capture_lock().lock_shared();
  const hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    capture_lock().unlock_shared();
    set_error("hipStreamBeginCapture failed: %s (%d)", hipGetErrorString(e), (int)e);
    return SY_EDEVICE;
  }
  ctx->capturing = true;
  return SY_OK;
}

int sy_graph_end(sy_ctx* ctx, uint64_t* graph) {
  SY_CHECK(ctx && graph, SY_EINVAL, "null argument");
  SY_CHECK(ctx->capturing, SY_ESTATE, "no capture active");
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(ctx->stream, &g);
  capture_lock().unlock_shared();
  if (ec != hipSuccess) {
    set_error("hipStreamEndCapture failed: %s (%d)", hipGetErrorString(ec), (int)ec);
    return SY_EDEVICE;
  }
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    set_error("hipGraphInstantiate failed: %s", hipGetErrorString(e));
    return SY_EDEVICE;
  }
  ctx->graphs.push_back(exec);
  ctx->graph_gen.push_back(ctx->scratch_gen);
  *graph = ctx->graphs.size();
  return SY_OK;
}

int sy_graph_launch(sy_ctx* ctx, uint64_t graph) {
  SY_CHECK(ctx && graph > 0 && graph <= ctx->graphs.size() && ctx->graphs[graph - 1], SY_EINVAL,
           "unknown graph handle");
  SY_CHECK(!graph_stale(ctx, graph), SY_ESTATE,
           "the context's scratch buffer grew after graph %llu was captured; capture it again",
           (unsigned long long)graph);
  SY_HIP(hipGraphLaunch(ctx->graphs[graph - 1], ctx->stream));
  return SY_OK;
}

int sy_graph_destroy(sy_ctx* ctx, uint64_t graph) {
  SY_CHECK(ctx && graph > 0 && graph <= ctx->graphs.size(), SY_EINVAL, "unknown graph handle");
  if (ctx->graphs[graph - 1]) {
    SY_HIP(hipStreamSynchronize(ctx->stream));
    SY_HIP(hipGraphExecDestroy(ctx->graphs[graph - 1]));
    ctx->graphs[graph - 1] = nullptr;
  }
  return SY_OK;
}

// ------------------------------------------------------------- timing

int sy_timer_start(sy_ctx* ctx) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_HIP(hipEventRecord(ctx->t0, ctx->stream));
  return SY_OK;
}

int sy_timer_stop(sy_ctx* ctx, float* ms) {
  SY_CHECK(ctx && ms, SY_EINVAL, "null argument");
  SY_HIP(hipEventRecord(ctx->t1, ctx->stream));
  SY_HIP(hipEventSynchronize(ctx->t1));
  SY_HIP(hipEventElapsedTime(ms, ctx->t0, ctx->t1));
  return SY_OK;
}

int sy_profile_enable(sy_ctx* ctx, int enabled) {
  SY_CHECK(ctx, SY_EINVAL, "null context");
  SY_CHECK(!ctx->capturing, SY_ESTATE, "profiling toggled during capture");
  SY_TRY(prof_collect(ctx));
  ctx->profiling = enabled != 0;
  ctx->profile_shapes = enabled == 2;
  ctx->profile.clear();
  return SY_OK;
}

int sy_profile_read(sy_ctx* ctx, char* names, size_t names_len, int* counts, float* total_ms, double* flops,
                    double* bytes, int max_entries, int* n_entries) {
  SY_CHECK(ctx && n_entries, SY_EINVAL, "null argument");
  SY_TRY(prof_collect(ctx));
  int i = 0;
  size_t pos = 0;
  for (auto& kv : ctx->profile) {
    if (i >= max_entries) break;
    if (names) {
      size_t len = kv.first.size() + 1;
      if (pos + len > names_len) break;
      memcpy(names + pos, kv.first.c_str(), len);
      pos += len;
    }
    if (counts) counts[i] = kv.second.count;
    if (total_ms) total_ms[i] = (float)kv.second.ms;
    if (flops) flops[i] = kv.second.flops;
    if (bytes) bytes[i] = kv.second.bytes;
    ++i;
  }
  *n_entries = i;
  return SY_OK;
}

}  // extern "C"
