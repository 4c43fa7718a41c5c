// Internal declarations shared by the runtime, the kernels and the C++ host.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <map>
#include <memory>
#include <shared_mutex>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "../../include/simdyolo_hip.h"

namespace sy {

struct HostStage;

// ------------------------------------------------------------- errors

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

struct Status {
  int code;
};

#define SY_HIP(call)                                                         \
  do {                                                                       \
    hipError_t e_ = (call);                                                  \
    if (e_ != hipSuccess) {                                                  \
      ::sy::set_error("%s failed: %s (%d) at %s:%d", #call,                  \
                      hipGetErrorString(e_), (int)e_, __FILE__, __LINE__);   \
      return e_ == hipErrorOutOfMemory ? SY_ENOMEM : SY_EDEVICE;             \
    }                                                                        \
  } while (0)

#define SY_CHECK(cond, code, ...)        \
  do {                                   \
    if (!(cond)) {                       \
      ::sy::set_error(__VA_ARGS__);      \
      return (code);                     \
    }                                    \
  } while (0)

#define SY_TRY(expr)          \
  do {                        \
    int rc_ = (expr);         \
    if (rc_ != SY_OK) return rc_; \
  } while (0)

// Held shared by every open graph capture (sy_graph_begin to sy_graph_end)
// and exclusively by copies on the legacy null stream (the weight upload):
// HIP fails a capture open on one thread when another thread copies on the
// null stream, even into memory the capture never touches.
std::shared_timed_mutex& capture_lock();

// ------------------------------------------------------------- context

struct ConvPlan;

enum Algo { kAuto = 0, kIgemm = 1, kWinograd = 2, kDirect = 3, kWinograd3 = 4, kDepthwise = 5, kWinograd2 = 6 };

// Algorithm and GEMM tile (-1: size heuristic) for one input shape.
struct ConvChoice {
  int algo = kAuto;
  int tile = -1;
  int split = 1;  // implicit GEMM: K split over this many workgroups (1: none)
};

struct ProfileEntry {
  int count = 0;
  double ms = 0;
  double flops = 0, bytes = 0;  // algorithmic work of the launches
};

struct PendingEvent {
  std::string name;
  hipEvent_t start, stop;
  double flops, bytes;
};

}  // namespace sy

struct sy_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name;
  int cu_count = 0;
  // frame arena: chained blocks, reset (not freed) at every BeginFrame
  std::vector<std::pair<char*, size_t>> blocks;
  size_t block = 0, block_used = 0;
  int64_t frame_id = 0;
  bool frame_active = false;
  // persistent allocations owned by the context (weights)
  std::vector<void*> owned;
  std::vector<std::unique_ptr<sy::ConvPlan>> convs;
  // scratch (Winograd transforms, staging); grows outside capture only
  char* scratch = nullptr;
  size_t scratch_size = 0;
  char* host_stage = nullptr;  // pinned host staging for small uploads (hipHostMalloc)
  size_t host_stage_size = 0;
  uint64_t scratch_gen = 0;  // bumped whenever scratch moves
  // graphs, with the scratch generation each was captured under
  bool capturing = false;
  std::vector<hipGraphExec_t> graphs;
  std::vector<uint64_t> graph_gen;
  // timing
  hipEvent_t t0 = nullptr, t1 = nullptr;
  bool profiling = false;
  bool profile_shapes = false;  // key profile entries by kernel + shape tag
  std::string prof_tag;         // shape tag of the op being launched
  std::vector<sy::PendingEvent> pending;
  int force_tile = -1;  // GEMM tile forced by the conv's tuned choice
  int force_split = 1;  // split-K factor of the conv's tuned choice
  // While a 1x1 conv runs through conv_run_upsampled: the half-resolution
  // view whose 2x nearest upsample is the first up_src->c input channels.
  const sy_tensor* up_src = nullptr;
  std::map<std::string, sy::ProfileEntry> profile;
  std::vector<hipEvent_t> event_pool;
  // tuning decisions by conv geometry + input shape (sy_tune_save / sy_tune_load)
  std::map<std::string, sy::ConvChoice> tune_table;
  // Second stream (default priority) and scratch for model branches that run
  // concurrently with the main chain inside a captured graph; swapped into
  // `stream` / `scratch` while such a branch is being enqueued.
  hipStream_t side = nullptr;
  char* side_scratch = nullptr;
  size_t side_scratch_size = 0;
  // Pinned staging of large host copies (created on first use).
  sy::HostStage* stage = nullptr;
};

namespace sy {

// Scratch space for one op; never reallocates while a graph is being captured.
int ensure_scratch(sy_ctx* ctx, size_t bytes);

// While alive, ops enqueued on the context go to its side stream and use the
// side scratch buffer (the side stream is created on first use).
struct SideLane {
  sy_ctx* ctx;
  bool on = false;
  explicit SideLane(sy_ctx* c, bool enable) : ctx(c) {
    if (!enable) return;
    if (!ctx->side && hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking) != hipSuccess) {
      ctx->side = nullptr;
      return;
    }
    swap();
    on = true;
  }
  ~SideLane() {
    if (on) swap();
  }
  bool ok() const { return on; }
  void swap() {
    std::swap(ctx->stream, ctx->side);
    std::swap(ctx->scratch, ctx->side_scratch);
    std::swap(ctx->scratch_size, ctx->side_scratch_size);
  }
};
// Host <-> device copies of `bytes` through the context's pinned staging, on
// the context stream: the host buffer has been read (staged_h2d; the DMA may
// still run) or written (staged_d2h) when they return.
int staged_h2d(sy_ctx* ctx, void* dst, const void* src, size_t bytes);
int staged_d2h(sy_ctx* ctx, void* dst, const void* src, size_t bytes);
// Host copies at least this large go through the staging.
constexpr size_t kStageMin = size_t(1) << 20;
// Pinned host staging of at least `bytes`; growing it waits for the stream.
int ensure_host_stage(sy_ctx* ctx, size_t bytes);
// True when the scratch buffer moved after `graph` was captured.
inline bool graph_stale(const sy_ctx* ctx, uint64_t graph) {
  return graph > 0 && graph <= ctx->graph_gen.size() && ctx->graph_gen[graph - 1] != ctx->scratch_gen;
}

// Kernel-launch bracketing for per-kernel profiling.
void prof_begin(sy_ctx* ctx, const char* name, double flops, double bytes);
void prof_end(sy_ctx* ctx);
int prof_collect(sy_ctx* ctx);

struct ProfScope {
  sy_ctx* ctx;
  // flops / bytes: the launch's algorithmic work (not counting padding or
  // re-reads), reported next to its event time.
  // A null context times nothing (callers that must not create events).
  ProfScope(sy_ctx* c, const char* name, double flops = 0, double bytes = 0) : ctx(c) {
    if (ctx && ctx->profiling) prof_begin(ctx, name, flops, bytes);
  }
  ~ProfScope() {
    if (ctx && ctx->profiling) prof_end(ctx);
  }
};

int check_launch(const char* name);

// View validation helpers.
int check_view(const sy_tensor* t, const char* what, bool allow_nchw = false);

inline int64_t pixels(const sy_tensor& t) { return (int64_t)t.n * t.h * t.w; }

// ------------------------------------------------------------- convolution


struct ConvPlan {
  int oc, ic, kh, kw, sh, sw, pt, pl, pb, pr, dh, dw, groups, silu;
  int algo = kIgemm;
  bool user_algo = false;  // fixed by sy_conv_set_algo: never retuned
  // 2x2 stride-2 transposed conv: stored as a 1x1 conv with oc = 4 * up2
  // virtual channels (q * up2 + o, q = 2 dy + dx) whose GEMM epilogue writes
  // the pixel-shuffled [2h, 2w, up2] output; 0 for ordinary convs.
  int up2 = 0;
  // Fastest (algorithm, tile) per input (n, h, w) and residual presence,
  // measured on first use.
  std::map<std::tuple<int, int, int, int>, ConvChoice> tuned;
  // implicit GEMM: weights [ocp][kp], K ordered (ky, kx, ic)
  float* w_gemm = nullptr;
  int kp = 0, ocp = 0;
  // Winograd: U [36][ocw][kpw] (ocw = oc rounded to the GEMM tile, kpw = ic
  // rounded to the deepest K tile)
  float* w_wino = nullptr;
  int ocw = 0, kpw = 0;
  // Winograd, GEMM fused with the inverse transform: U in MFMA-operand blocks
  // [36][ceil(oc/32)][ic/8][64 lanes][4]
  float* w_wino_b = nullptr;
  // direct low-channel: [kh*kw*ic][ocd] (ocd = oc rounded up to 16)
  float* w_direct = nullptr;
  int ocd = 0;
  // depthwise: [kh*kw][round_up(oc, 4)]
  float* w_dw = nullptr;
  float* bias = nullptr;  // [round_up(oc, 128)] zero padded
  std::vector<float> host_w, host_b;  // OIHW copy kept to repack on algo change
};

int conv_prepare(sy_ctx* ctx, ConvPlan* p);
bool conv_supports(const ConvPlan* p, int algo);
int conv_run(sy_ctx* ctx, ConvPlan* p, const sy_tensor* x, const sy_tensor* y, const sy_tensor* res);
// A 1x1 conv whose input x is concat(upsample2x(xu), rest): channels
// [0, xu->c) of x are the 2x nearest upsample of xu and need not be written;
// the GEMM reads them from xu at half resolution.  Shapes the kernel cannot
// take write the upsample into x first and run conv_run.
int conv_run_upsampled(sy_ctx* ctx, ConvPlan* p, const sy_tensor* xu, const sy_tensor* x, const sy_tensor* y,
                       const sy_tensor* res);
int tune_save(const sy_ctx* ctx, const char* path);
int tune_load(sy_ctx* ctx, const char* path);
size_t conv_scratch_bytes(const ConvPlan* p, int n, int h, int w);
// C[m][n] = sum_k A[m][k] B[n][k] on FP32 MFMA; `batch` GEMMs with strides.
int gemm_nt(sy_ctx* ctx, const float* A, int M, int K, int lda, const float* B, int N, int ldb, float* C, int ldc,
            const char* name, int batch = 1, long long a_stride = 0, long long b_stride = 0, long long c_stride = 0);
void conv_out_size(const ConvPlan* p, int h, int w, int* oh, int* ow);

// ------------------------------------------------------------- other ops

int op_add(sy_ctx* ctx, const sy_tensor* a, const sy_tensor* b, const sy_tensor* y);
int op_resize_nearest(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y);
int op_maxpool(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y, int kh, int kw, int sh, int sw, int pt,
               int pl, int pb, int pr, int ceil_mode);
int op_sppf(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5, const sy_tensor* y9, const sy_tensor* y13);
int op_copy(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y);
int op_nchw_to_view(sy_ctx* ctx, const float* src_dev, const sy_tensor* dst);
int op_view_to_nchw(sy_ctx* ctx, const sy_tensor* src, float* dst_dev);
int op_detect_decode(sy_ctx* ctx, const sy_tensor* levels, const float* strides, int n_levels, int bins, int nc,
                     int xyxy, float* out, int total);
int op_e2e_topk(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum,
                int onnx, float* out);
// Allocation-free top-k over a fixed per-GPU block of kTopkStaticScratchBytes.
constexpr size_t kTopkStaticScratchBytes = 32u << 20;
int topk_static_init(int device);
// Scratch bytes sy_e2e_topk needs for this request (PT rules).
int e2e_topk_scratch_bytes(int batch, int channels, int anchors, int nc, int maximum, size_t* bytes);
int op_e2e_topk_noalloc(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum,
                        int onnx, float* out);
int op_compute(sy_ctx* ctx, int op, const float* const* in, const size_t* in_len, const uint32_t* params,
               long long items, float* out, size_t out_len);
int op_matmul(sy_ctx* ctx, const float* a, const float* b, float* c, int m, int n, int k, int nbatch,
              const int* batch_shape, const long long* a_strides, const long long* b_strides, size_t a_len,
              size_t b_len, size_t c_len);
int op_attention(sy_ctx* ctx, const sy_tensor* qkv, int heads, int kd, int hd, float scale, const sy_tensor* o,
                 const sy_tensor* v);
size_t attention_scratch_bytes(int B, int H, int W, int heads, int hd);

int64_t pool_out_size(int len, int k, int s, int before, int after, int ceil_mode);

// Greedy NMS and letterbox mapping of candidates already sorted by confidence
// (descending, ties in anchor order).
int finish_detections(std::vector<sy_detection>& cand, bool e2e, const sy_decode_options* o, const sy_letterbox* t,
                      sy_detection* out, int max_out, int* count);

}  // namespace sy
