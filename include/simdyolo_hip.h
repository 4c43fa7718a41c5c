/*
 * libsimdyolo_hip — MI355X (gfx950) forward-inference backend for SimdYolo.
 *
 * C ABI only: plain pointers, sizes and status codes; no C++ or torch types.
 * The C# side binds it with LibraryImport; in this
 * repository Python (ctypes) and C++ drive it.
 *
 * Each entry point names the reference interface it replaces (paths are
 * relative to the SimdYolo repository root).
 *
 * Layout.  Device activations are NHWC "views": `data` points at element
 * (n=0, h=0, w=0, c=0) and consecutive pixels are `ldc` floats apart
 * (ldc >= c), so a channel slice of a wider tensor is a view with an offset
 * pointer and the wider tensor's ldc.  Channel concat and split therefore
 * cost nothing: producers write straight into their slice.  Only the network
 * input (dense NCHW, layout = SY_LAYOUT_NCHW) and the joined head output
 * ([B, nc+4, anchors], channels first) keep the reference's layouts.
 *
 * Errors.  Every int-returning call returns SY_OK (0) or one of the SY_E*
 * codes; sy_last_error() returns a thread-local message.  The C# binding maps
 * SY_EINVAL -> ArgumentException, SY_EUNSUPPORTED -> NotSupportedException and
 * the rest -> InvalidOperationException, as the Vulkan backend does
 * (src/SimdYolo/VulkanBackend.cs:323, VulkanExecution.cs:229).
 *
 * Threading.  A context is used by one thread at a time (the reference holds
 * its monitor from BeginFrame to EndFrame, VulkanExecution.cs:46,87).
 * Running separate contexts on separate threads at once is not supported:
 * it has ended in an intermittent host-side fault inside sy_model_predict_raw.
 * Weight uploads do wait (at most 60 s, then SY_ESTATE) until no other
 * context has a graph capture open, since their copies would make such a
 * capture fail.
 */
#ifndef SIMDYOLO_HIP_H
#define SIMDYOLO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SY_OK 0
#define SY_EINVAL 1       /* invalid argument or shape mismatch */
#define SY_EUNSUPPORTED 2 /* valid request this backend does not implement */
#define SY_EDEVICE 3      /* HIP runtime error */
#define SY_ENOMEM 4       /* device allocation failed */
#define SY_ESTATE 5       /* call not valid in the current frame/capture state */

#define SY_LAYOUT_NHWC 0
#define SY_LAYOUT_NCHW 1

typedef struct sy_ctx sy_ctx;
typedef struct sy_model sy_model;

/* A device tensor view (see "Layout" above).  For SY_LAYOUT_NCHW the tensor is
 * dense and ldc is ignored. */
typedef struct sy_tensor {
  float* data;
  int32_t n, c, h, w;
  int32_t ldc;
  int32_t layout;
} sy_tensor;

/* ----------------------------------------------------------- lifecycle */

/* Open device `device` and create a stream.  Replaces `new VulkanBackend()` +
 * Initialize (src/SimdYolo/VulkanBackend.cs:52-106) behind
 * ComputeBackends.Create (src/SimdYolo/YoloDetector.cs:419-428). */
int sy_create(int device, sy_ctx** out);
/* IComputeBackend.Dispose (src/SimdYolo/Compute.cs:11-25). */
void sy_destroy(sy_ctx* ctx);
/* IComputeBackend.Name (src/SimdYolo/Compute.cs:14-16). */
const char* sy_name(const sy_ctx* ctx);
/* Message of the last failed call on this thread. */
const char* sy_last_error(void);
/* Number of visible HIP devices (0 when none). */
int sy_device_count(int* count);
/* Library version string. */
const char* sy_version(void);

/* ------------------------------------------------------ frame and memory */

/* IDeviceBackend.BeginFrame / EndFrame / Flush and FrameId
 * (src/SimdYolo/DeviceExecution.cs:8-19).  BeginFrame resets the frame arena
 * (VulkanExecution.cs:43-68); views from earlier frames become invalid. */
int sy_frame_begin(sy_ctx* ctx, int64_t* frame_id);
int sy_frame_end(sy_ctx* ctx);
int sy_flush(sy_ctx* ctx);
/* Frame-arena allocation of a dense NHWC tensor, 256-byte aligned
 * (VulkanExecution.cs:137-160). */
int sy_frame_alloc(sy_ctx* ctx, int n, int c, int h, int w, sy_tensor* out);
/* Host NCHW floats -> device view (upload, VulkanExecution.cs:164-194);
 * returns once the host buffer has been read. */
int sy_upload_nchw(sy_ctx* ctx, const float* host, const sy_tensor* dst);
/* Device view -> host NCHW floats; synchronous.  IDeviceBackend.Download
 * (src/SimdYolo/DeviceExecution.cs:27). */
int sy_download_nchw(sy_ctx* ctx, const sy_tensor* src, float* host);
/* Persistent device memory outside the frame arena (weights, outputs). */
int sy_malloc(sy_ctx* ctx, size_t bytes, void** ptr);
int sy_free(sy_ctx* ctx, void* ptr);
/* Stream-ordered copies; kind: 0 host->device, 1 device->host, 2 device->device.
 * Copies that touch host memory return once the host buffer has been read or
 * written, so the caller may reuse or unpin it (a managed array is pinned
 * only for the call); device->device copies are asynchronous.  Host copies of
 * 1 MiB or more pass through the context's pinned staging (host threads fill
 * or empty 8 MiB pinned slots while the DMA of the slot before runs), so a
 * host->device copy may still be in flight on the context stream when it
 * returns; work on that stream is ordered after it. */
int sy_memcpy(sy_ctx* ctx, void* dst, const void* src, size_t bytes, int kind);

/* ---------------------------------------------------------- convolution */

#define SY_CONV_AUTO 0
#define SY_CONV_IGEMM 1    /* implicit-GEMM on FP32 MFMA */
#define SY_CONV_WINOGRAD 2  /* fused Winograd F(4x4,3x3): transforms + 36-plane MFMA GEMM in one kernel */
#define SY_CONV_DIRECT 3    /* direct low-channel conv (stem; NCHW input allowed) */
#define SY_CONV_WINOGRAD3 4 /* Winograd F(4x4,3x3) as three kernels (transform, batched GEMM, inverse) */
#define SY_CONV_DEPTHWISE 5 /* groups == channels (DWConv, attention pe) */
#define SY_CONV_WINOGRAD2 6 /* Winograd F(4x4,3x3) as two kernels: input transform, then the
                               36 plane GEMMs fused with the inverse transform (ic % 8 == 0) */

/* Prepare a convolution once: pack/transform the OIHW weights and bias
 * (already BN-folded) into the weight arena and choose the algorithm.  The
 * geometry arguments are those of IDeviceBackend.DeviceConv
 * (src/SimdYolo/DeviceExecution.cs:54): stride (h,w), pads (top, left,
 * bottom, right), dilation (h,w), groups, fused SiLU.  The default routing
 * mirrors DeviceConv (src/SimdYolo/VulkanExecution.cs:337-350): depthwise;
 * low-channel stem -> direct; constant 3x3 s1 p1 d1 g1 with ic >= 16 ->
 * Winograd; else implicit GEMM.  On the first run of each input shape an
 * auto-routed conv times its candidates (implicit GEMM tiles, the
 * weight-stationary row kernel for 1x1 and Winograd planes, the 16-channel
 * 3x3 kernel, the three Winograd forms) with HIP events and keeps the fastest,
 * as the Vulkan backend's timestamp autotune does (VulkanWinograd.cs:83-117);
 * SIMDYOLO_HIP_AUTOTUNE=0 keeps the routing rule.  SIMDYOLO_HIP_WINOGRAD=0
 * disables Winograd (as SIMDYOLO_WINOGRAD does for Vulkan,
 * VulkanWinograd.cs:16-35) and SIMDYOLO_HIP_WINO_FUSED=1 makes the routing
 * rule pick the fused kernel (SY_CONV_WINOGRAD) instead of the three-kernel
 * form (SY_CONV_WINOGRAD3).  A conv whose output overlaps its input or
 * residual (an in-place y += f(x)) is not re-run for timing and keeps the
 * routing rule. */
int sy_conv_create(sy_ctx* ctx, const float* weight_oihw, const float* bias,
                   int oc, int ic, int kh, int kw, int stride_h, int stride_w,
                   int pad_t, int pad_l, int pad_b, int pad_r, int dil_h,
                   int dil_w, int groups, int silu, uint64_t* conv);
/* nn.ConvTranspose2d(ic, oc, kernel 2, stride 2, padding 0) with bias: the
 * Proto upsample (src/SimdYolo/PtModel.cs:344), which the reference rewrites
 * as a 1x1 conv plus pixel shuffle (VulkanTransposeConv.cs:13-29).  weight is
 * PyTorch's [ic][oc][2][2]; sy_conv_run maps x [n, ic, h, w] to y
 * [n, oc, 2h, 2w] (no residual).  It runs as one MFMA GEMM over the input
 * pixels whose epilogue writes each 2x2 sub-pixel in place. */
int sy_conv_transpose2x2_create(sy_ctx* ctx, const float* weight_iohw, const float* bias, int ic, int oc,
                                uint64_t* conv);
/* Force an algorithm (SY_CONV_*); SY_EUNSUPPORTED when it cannot run this conv.
 * With a forced algorithm, SIMDYOLO_HIP_TILE=n also forces its n-th form: the
 * implicit-GEMM tile (or row-kernel width), the two-kernel Winograd's wave
 * layout (0 four waves, 1 eight), or the fused Winograd's form (0 four waves,
 * 1 warp-specialized, 2 two groups over 64 output channels). */
int sy_conv_set_algo(sy_ctx* ctx, uint64_t conv, int algo);
int sy_conv_get_algo(sy_ctx* ctx, uint64_t conv, int* algo);
/* y = [residual +] act(conv(x) + bias).  IDeviceBackend.DeviceConv
 * (src/SimdYolo/DeviceExecution.cs:54) with two fusions the reference runs
 * as separate passes: the Bottleneck residual add (PtModel.cs:303, op 10) and
 * the concat write (y may be a channel slice of the concat buffer).
 * `residual` may be NULL; it has y's shape.  Shapes are validated against the
 * conv geometry (Compute.cs:171-182). */
int sy_conv_run(sy_ctx* ctx, uint64_t conv, const sy_tensor* x,
                const sy_tensor* y, const sy_tensor* residual);
/* A 1x1 conv over concat(upsample2x(xu), rest) without the upsample: x is
 * the concat view, whose leading xu->c channels need not hold anything, and
 * the GEMM reads those channels from xu (half x's height and width) at
 * pixel (y / 2, x / 2).  No counterpart in the reference, which runs the
 * nearest Upsample (Compute.cs:715-721), the Concat and then cv1 of the
 * following C2f (PtModel.cs:260, 310-317) as separate passes; results are
 * those of sy_resize_nearest into x's leading channels followed by
 * sy_conv_run.  A conv or views the fused kernel cannot take (not a plain
 * 1x1 stride-1 GEMM, xu->c not a multiple of 32, unaligned views, an
 * algorithm forced with sy_conv_set_algo) runs as exactly that pair. */
int sy_conv_run_upsampled(sy_ctx* ctx, uint64_t conv, const sy_tensor* xu, const sy_tensor* x,
                          const sy_tensor* y, const sy_tensor* residual);
/* Output size of the conv for an input of h x w. */
int sy_conv_out_size(sy_ctx* ctx, uint64_t conv, int h, int w, int* oh, int* ow);

/* Tuning table: the autotuner's (algorithm, tile) decisions of this context,
 * keyed by conv geometry and input shape (n, h, w, residual).  sy_tune_save
 * writes them as text; sy_tune_load merges a table written by the same
 * library build, and later convs whose key it holds skip timing and use the
 * recorded choice when it is one of their candidates.  It is the persisted
 * form of the Vulkan backend's per-shape timestamp autotune and pipeline
 * cache (VulkanWinograd.cs:83-117, VulkanPipelineCache.cs), so a process can
 * reproduce another's kernel choices (profiler runs) or skip first-frame
 * tuning. */
int sy_tune_save(sy_ctx* ctx, const char* path);
int sy_tune_load(sy_ctx* ctx, const char* path);

/* ------------------------------------------------------------ other ops */

/* Elementwise y = a + b on equal shapes: DeviceOps.Binary op 10
 * (src/SimdYolo/DeviceExecution.cs:128-139). */
int sy_add(sy_ctx* ctx, const sy_tensor* a, const sy_tensor* b, const sy_tensor* y);
/* Nearest resize to y's h,w (index y*ih/h): op 20 (src/SimdYolo/Compute.cs:715-721). */
int sy_resize_nearest(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y);
/* Max pool, padding excluded: op 21 (src/SimdYolo/Compute.cs:677-708). */
int sy_maxpool(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y, int kh,
               int kw, int sh, int sw, int pt, int pl, int pb, int pr, int ceil_mode);
/* The SPPF chain of three MaxPool2d(5,1,2) (src/SimdYolo/PtModel.cs:310-311)
 * in one pass: y5 = pool5(x), y9 = pool5(y5), y13 = pool5(y9). */
int sy_sppf_pool(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y5,
                 const sy_tensor* y9, const sy_tensor* y13);
/* Copy x into view y of the same shape: DeviceConcat / DeviceSlice when the
 * producer could not write in place (src/SimdYolo/VulkanExecution.cs:433-492). */
int sy_copy(sy_ctx* ctx, const sy_tensor* x, const sy_tensor* y);

/* Joined detect-head decode: DFL softmax expectation, grid decode and class
 * sigmoid for every level into out[B][nc+4][total_anchors] (channels first).
 * Replaces VulkanBackend.DecodeHeadLevels (VulkanExecution.cs:295-324) and
 * tensor.comp op 30; semantics of CpuHead.DecodeInto (CpuHead.cs:57-124).
 * Level i's raw head is one NHWC view whose first 4*bins channels are the box
 * distribution (side-major) and next nc channels the class logits; any
 * further channels (a Segment head's mask coefficients) are copied raw to
 * output channels nc+4.., as CompleteInstanceHead's concat (PtModel.cs:523). */
int sy_detect_decode(sy_ctx* ctx, const sy_tensor* levels, const float* strides,
                     int n_levels, int bins, int nc, int xyxy, float* out,
                     int total_anchors);

/* Two-stage end-to-end top-k over a channels-first head [B][channels][anchors]
 * (nc class channels at 4.., extras after them) into out[B][k][6+extra],
 * k = min(maximum, anchors).  onnx_rules=0: PT rules (NaN last, ties by
 * anchor*nc+c; CpuEndToEnd.SelectPt, CpuEndToEnd.cs:26-140); 1: ONNX rules
 * (NaN first, ties by rank*nc+c; CpuEndToEnd.cs:147-241).  Replaces
 * VulkanBackend.TryEndToEndTopK (VulkanTopK.cs:37-70).  Bit-exact.  Limits:
 * k <= 1024, k * nc <= 32768, anchors <= 16777216 (stage 1 reads its keys from
 * LDS up to 32768 anchors, from global memory beyond). */
int sy_e2e_topk(sy_ctx* ctx, const float* head, int batch, int channels,
                int anchors, int nc, int maximum, int onnx_rules, float* out);

/* sy_e2e_topk without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, hosts that forbid hipMalloc).
 * Same arguments, results (bit-identical) and errors as sy_e2e_topk, except
 * that its scratch is a fixed 32 MiB block per GPU, part of the library's
 * code object and held until the process ends, instead of the context's
 * scratch: requests needing more (about 20 bytes per anchor and image, e.g.
 * batch 32 x 8400 anchors uses 5.4 MB) fail with SY_EUNSUPPORTED before any
 * launch.  Every call on one GPU shares that block.  Calls enqueued outside
 * graph capture are ordered on it by the library: each call's stream waits
 * on a per-GPU event that the previous call (any context or stream) recorded
 * after its kernels.  A call captured into a graph records no such wait, so
 * the caller must not launch that graph while another call on the same GPU
 * (eager or another graph holding one) can run: such overlaps race. */
int sy_e2e_topk_noalloc(sy_ctx* ctx, const float* head, int batch, int channels,
                        int anchors, int nc, int maximum, int onnx_rules, float* out);

/* IDeviceBackend.Compute(op, inputs, shape, params, workItems)
 * (src/SimdYolo/DeviceExecution.cs:41): one tensor.comp operation
 * (shaders/tensor.comp) on dense row-major device tensors, with the same
 * 32-slot parameter block the reference's DeviceOps and its callers build
 * (DeviceExecution.cs:107-190; Compute.cs:137,693,720): unary 1-9, broadcast
 * binary 10-16, nearest resize 20, max/average pool 21/22, transpose 23,
 * slice 24, softmax 25, concat write 26, head decode 30, pose decode 31,
 * depthwise conv 32, transposed conv 33, DFL 34, depth-to-space 35, row max
 * 36, gather 37.  inputs[0..2] are the A, B and D bindings (NULL when the op
 * does not read them) with their lengths in floats; params[0] must equal work_items;
 * params[27] is set from inputs[2] (1 when a bias is bound), as the
 * reference's Compute does; params[28..31] are element offsets of A, B, C and
 * D as in the shader (a caller that folds its offsets into the pointers
 * passes zeros).  Indices are clamped to the given lengths
 * on the device; parameter blocks whose extents the host can check against
 * them are refused with SY_EINVAL, unknown ops with SY_EUNSUPPORTED. */
int sy_compute(sy_ctx* ctx, int op, const float* const* inputs, const size_t* input_lengths,
               const uint32_t* params, int64_t work_items, float* out, size_t out_length);

/* IDeviceBackend.DeviceMatMul (src/SimdYolo/DeviceExecution.cs:61,
 * VulkanExecution.cs:499-541) and IComputeBackend.MatMul (Compute.cs:24):
 * c[z] = a[za] (m x k) . b[zb] (k x n), row-major, for every output matrix z
 * of the batch shape (up to 4 dims, row-major; rank 0 = one product).  za and
 * zb are the matrix indices sum(coord_j * a_batch_strides[j]) and likewise for
 * b, in matrices (0 on broadcast axes).  Lengths are in floats and bound every
 * matrix.  FP32 MFMA when k % 4 == 0 and a is 16-byte aligned, a tiled kernel
 * otherwise.  Empty dimensions: SY_EUNSUPPORTED, as the reference. */
int sy_matmul(sy_ctx* ctx, const float* a, const float* b, float* c, int m, int n, int k, int batch_rank,
              const int32_t* batch_shape, const int64_t* a_batch_strides, const int64_t* b_batch_strides,
              size_t a_length, size_t b_length, size_t c_length);

/* Multi-head attention core of C2PSA (PtModel.Attention, src/SimdYolo/
 * PtModel.cs:429-437; the reference runs it as DeviceMatMul + Scale op 4 +
 * Softmax op 25 + DeviceMatMul, VulkanExecution.cs:499-541).  qkv is the qkv
 * conv output viewed as [B, heads, 2*key_dim + head_dim, H*W] (per pixel:
 * head-major q | k | v channels).  Writes o = v softmax(q^T k * scale)^T as
 * the NHWC view o [B, heads*head_dim, H, W] and a dense copy of v into the
 * view v (same shape) for the depthwise positional conv. */
int sy_attention(sy_ctx* ctx, const sy_tensor* qkv, int heads, int key_dim,
                 int head_dim, float scale, const sy_tensor* o, const sy_tensor* v);

/* Per-instance mask geometry returned by sy_mask_decode: the crop in source
 * pixels and the offset (in floats) of its width*height probabilities in the
 * output buffer. */
typedef struct sy_mask_info {
  int32_t left, top, width, height;
  int64_t offset;
} sy_mask_info;

struct sy_letterbox;
struct sy_detection;

/* Instance masks of one image: low = coeffs[k][nm] . protos^T on FP32 MFMA,
 * then for every instance the letterbox-ROI half-pixel bilinear resample of
 * its low-res logits to source pixels, sigmoid, and the crop to its box
 * (CpuMaskDecoder.Decode, src/SimdYolo/CpuMaskDecoder.cs:18-81, which the
 * reference runs on the CPU).  protos: [1][nm][mh][mw] as an NHWC view or a
 * dense NCHW tensor (one image of a Segment model's prototype buffer, as
 * sy_model_proto returns it); coeffs: device rows of nm floats, ld_coeff apart (ld_coeff =
 * 6 + nm reads the mask coefficients straight out of an end-to-end top-k
 * output when coeffs points at its field 6); boxes: host, source
 * coordinates, clamped to the image.  Writes info[k] and the probabilities
 * into masks (device, capacity in floats); synchronous. */
int sy_mask_decode(sy_ctx* ctx, const sy_tensor* protos, const float* coeffs,
                   int ld_coeff, int k, const struct sy_detection* boxes,
                   const struct sy_letterbox* t, float* masks, size_t capacity,
                   sy_mask_info* info);

/* -------------------------------------------------------------- graphs */

/* hipGraph capture of everything issued on the context stream between begin
 * and end; the counterpart of BeginReplayCapture/TryReplay
 * (src/SimdYolo/VulkanReplay.cs:31-129).  Ops that need more scratch than
 * the context holds grow it outside capture; a graph captured before such a
 * growth is refused by sy_graph_launch with SY_ESTATE and must be captured
 * again (the model API does this by itself). */
int sy_graph_begin(sy_ctx* ctx);
int sy_graph_end(sy_ctx* ctx, uint64_t* graph);
int sy_graph_launch(sy_ctx* ctx, uint64_t graph);
int sy_graph_destroy(sy_ctx* ctx, uint64_t graph);

/* --------------------------------------------------------------- timing */

/* hipEvent pair on the context stream (the stream every kernel above is
 * launched on).  The GPU_TICKS counterpart of VulkanExecution.cs:77-85. */
int sy_timer_start(sy_ctx* ctx);
int sy_timer_stop(sy_ctx* ctx, float* ms);
/* Per-kernel event timing of eager launches: when enabled, every kernel the
 * library launches is bracketed by events on the context stream;
 * sy_profile_read returns, per kernel name (NUL-separated in `names`), the
 * launch count, total milliseconds and the launches' total algorithmic
 * FLOPs and HBM bytes (the unpadded work, for roofline fractions).
 * enabled = 2 keys convolution entries by kernel and layer shape. */
int sy_profile_enable(sy_ctx* ctx, int enabled);
int sy_profile_read(sy_ctx* ctx, char* names, size_t names_len, int* counts,
                    float* total_ms, double* flops, double* bytes,
                    int max_entries, int* n_entries);

/* ============================================ model (C++ host mirror) */

#define SY_ARCH_YOLOV8 0
#define SY_ARCH_YOLO11 1
#define SY_ARCH_YOLO26 2

/* (depth, width, max_channels) of the scaled families.  YOLOv8
 * (ultralytics yolov8.yaml): n = (0.33, 0.25, 1024), s = (0.33, 0.50, 1024),
 * m = (0.67, 0.75, 768).  YOLO11 (yolo11.yaml, with C3k2 / C2PSA):
 * n = (0.50, 0.25, 1024), s = (0.50, 0.50, 1024), m = (0.50, 1.00, 512).
 * YOLO26 (yolo26.yaml / yolo26-seg.yaml): YOLO11's scales, reg_max 1, an
 * end-to-end head (one2one branches, PtModel.cs:449-450) whose output is the
 * two-stage top-k selection (max_det 300, PtModel.cs:506-570) and, with
 * nm > 0, Segment26 with Proto26 (PtModel.cs:345-359). */
typedef struct sy_model_config {
  int32_t arch;
  float depth, width;
  int32_t max_channels, nc, reg_max;
  float bn_eps;
  /* Segment head (ultralytics Segment; PtModel.cs:353-360) when nm > 0: nm
   * mask coefficients per anchor appended to the head, and a Proto net of
   * make_divisible(min(npr, max_channels) * width, 8) channels. */
  int32_t nm, npr;
} sy_model_config;

/* Parameter kinds of sy_model_layout entries. */
#define SY_P_CONV_WEIGHT 0
#define SY_P_BN_GAMMA 1
#define SY_P_BN_BETA 2
#define SY_P_BN_MEAN 3
#define SY_P_BN_VAR 4
#define SY_P_BIAS_BOX 5
#define SY_P_BIAS_CLS 6
#define SY_P_BIAS 7 /* other biases: mask-coefficient Conv2d, Proto ConvTranspose2d */

/* Canonical (state_dict order) parameter tensors of the model: 6 ints each
 * (kind, d0, d1, d2, d3, fan_in).  `out` may be NULL to query the count.
 * The .pt loader's tensor walk (src/SimdYolo/PtModel.cs:84-105). */
int sy_model_layout(const sy_model_config* cfg, int32_t* out, int max_entries, int* count);
/* Build the model: fold BN (PtModel.Prepare, src/SimdYolo/PtModel.cs:124-145),
 * upload weights once (VulkanExecution.cs:169-183), prepare every conv. */
int sy_model_create(sy_ctx* ctx, const sy_model_config* cfg, const float* params,
                    size_t n_params, sy_model** out);
void sy_model_destroy(sy_model* model);
/* Dims 1 and 2 of the model output for an input of batch x 3 x h x w: the
 * head [batch, nc+4(+nm), anchors], or for end-to-end models (YOLO26) the
 * selected rows [batch, k, 6(+nm)] with k = min(300, anchors), each row
 * x1 y1 x2 y2 score class (mask coefficients), as PtModel's EndToEndTopK. */
int sy_model_output_shape(sy_model* model, int batch, int h, int w, int* channels, int* anchors);
/* The device buffer of the joined, decoded head [batch, nc+4(+nm), anchors]
 * of that shape's plan, filled by every run: the output itself for NMS
 * heads; for end-to-end models the head before selection (PtModel.Detect
 * with selectEndToEnd false, PtModel.cs:444-504, which CompleteInstanceHead
 * selects from, :506-523). */
int sy_model_head(sy_model* model, int batch, int h, int w, float** head, int* channels, int* anchors);
/* Segment models: the device prototype buffer [batch, nm, h/4, w/4] (NCHW, as
 * the reference's Proto output) of that shape's plan, filled by every run. */
int sy_model_proto(sy_model* model, int batch, int h, int w, float** proto, int* channels,
                   int* proto_h, int* proto_w);
/* IModel.Run / YoloDetector.PredictRaw (src/SimdYolo/YoloDetector.cs:262-313):
 * upload NCHW input, forward (graph replay from the second call of a shape),
 * download the joined head.  Host buffers in, host buffer out. */
int sy_model_predict_raw(sy_model* model, const float* input_nchw, int batch,
                         int h, int w, float* out);
/* predict_raw for Segment models: also downloads the prototypes
 * [batch, nm, h/4, w/4] into proto_out. */
int sy_model_predict_seg(sy_model* model, const float* input_nchw, int batch, int h, int w,
                         float* out, float* proto_out);
/* Device-resident forward: plan the shape (allocating its arena) and return
 * the device input buffer [batch,3,h,w] (NCHW) and output buffer. */
int sy_model_buffers(sy_model* model, int batch, int h, int w, float** input,
                     float** output);
/* Run the forward on the resident buffers of that shape (async on the ctx
 * stream; sy_flush waits). */
int sy_model_run(sy_model* model, int batch, int h, int w);
/* use_graph = 0 runs the op list eagerly (needed for per-kernel profiling). */
int sy_model_set_graph(sy_model* model, int use_graph);
/* Branches of the captured forward.  The stride-8 detect level (with the
 * Segment prototypes) and the stride-16 level depend only on the P3 and P4
 * features, so the graph may run them on a second stream beside the rest of
 * the neck: level 0 = one chain, 1 = the P3 head as a branch, 2 = the P3 and
 * P4 heads.  By default (-1) each planned shape captures every level, times
 * a few replays of each and keeps the fastest, as the convolutions are
 * autotuned; a level set here is used as given (existing graphs are
 * recaptured).  Outputs do not depend on the level.  The reference runs its
 * recorded command buffer in order (VulkanReplay.cs); this has no
 * counterpart there.  sy_model_branch_level reports the level of a captured
 * shape (-1 before its first graph run). */
int sy_model_set_branch_level(sy_model* model, int level);
int sy_model_branch_level(sy_model* model, int batch, int h, int w, int* level);
/* Bytes of device memory held by the model (weights + planned arenas). */
int sy_model_memory(sy_model* model, size_t* weight_bytes, size_t* arena_bytes);
/* The activation arena of one input shape (planned on first use), the
 * counterpart of the Vulkan backend's per-frame intermediate arena
 * (VulkanExecution.cs:137-160, reported in
 * artifacts/inference-forward-performance-2026-11-18.md:62-66):
 * arena_bytes = input, head, outputs and every activation, with activations
 * whose lifetimes are disjoint sharing bytes; unshared_bytes = the same with
 * every activation separate; scratch_bytes = the context scratch the plan
 * reserves (Winograd transforms, split-K partials, top-k), held once per
 * context and stream, not per plan. */
int sy_model_plan_memory(sy_model* model, int batch, int h, int w, size_t* arena_bytes,
                         size_t* unshared_bytes, size_t* scratch_bytes);

/* ============================================ host utilities (CPU) */

typedef struct sy_letterbox {
  int32_t source_width, source_height, target_width, target_height;
  float scale_x, scale_y;
  int32_t pad_x, pad_y;
} sy_letterbox;

typedef struct sy_detection {
  int32_t class_id;
  float confidence, x, y, width, height;
  int32_t anchor;
} sy_detection;

#define SY_OUTPUT_AUTO 0
#define SY_OUTPUT_CHANNELS_FIRST 1
#define SY_OUTPUT_CHANNELS_LAST 2
#define SY_OUTPUT_END_TO_END 3

typedef struct sy_decode_options {
  float confidence, iou;
  int32_t max_detections, max_candidates, class_count, agnostic, layout;
} sy_decode_options;

/* DetectionDecoder.DecodeIndexed (src/SimdYolo/YoloDetector.cs:539-652) on a
 * single image's [dim1, dim2] head. */
int sy_decode_detections(const float* head, int dim1, int dim2,
                         const sy_decode_options* options, const sy_letterbox* t,
                         sy_detection* out, int max_out, int* count);
/* ImagePreprocessor.Letterbox (src/SimdYolo/YoloDetector.cs:448-507) into a
 * [1,3,th,tw] NCHW float buffer. */
int sy_letterbox_rgb(const uint8_t* pixels, int width, int height, int tw, int th,
                     int bgr, int row_stride, float* out, sy_letterbox* t);
/* ImagePreprocessor.Letterbox (src/SimdYolo/YoloDetector.cs:448-507) on the
 * device: a width x height RGB24 (BGR24 when bgr != 0) image already in device
 * memory, row_stride bytes per row (0 = 3 * width), into [3, th, tw] NCHW
 * floats at `out` (device; e.g. one image of sy_model_buffers' input).
 * Bit-identical to sy_letterbox_rgb; *t receives the same transform. */
int sy_letterbox_device(sy_ctx* ctx, const uint8_t* pixels, int width, int height, int tw, int th,
                        int bgr, int row_stride, float* out, sy_letterbox* t);
/* The candidate stage of DetectionDecoder.DecodeIndexed
 * (src/SimdYolo/YoloDetector.cs:557-621) on the device for a channels-first
 * [batch, channels, anchors] head (device memory): per image, the anchors that
 * pass the class/confidence/size tests, sorted by confidence descending with
 * ties in anchor order, truncated to max_candidates.  cand (device) holds
 * [batch][max_candidates] records, counts (device) [batch].  Up to 4194304
 * anchors per image; above 16384 (e.g. a 1280x1280 input's 33600) the sort
 * runs through a global work buffer in the context scratch. */
int sy_nms_candidates(sy_ctx* ctx, const float* head, int batch, int channels, int anchors,
                      const sy_decode_options* options, sy_detection* cand, int* counts);
/* DecodeIndexed for a device head: candidates on the GPU (sy_nms_candidates),
 * greedy NMS and the letterbox mapping on the host as the reference runs them.
 * Equal to sy_decode_detections per image.  t: [batch] transforms; out:
 * [batch][max_out] host records; counts: [batch] host. */
int sy_decode_detections_device(sy_ctx* ctx, const float* head, int batch, int channels, int anchors,
                                const sy_decode_options* options, const sy_letterbox* t,
                                sy_detection* out, int max_out, int* counts);
/* BN fold of PtModel.Prepare (src/SimdYolo/PtModel.cs:135-143), float math. */
void sy_fold_bn(const float* w, int oc, int per_oc, const float* conv_bias,
                const float* gamma, const float* beta, const float* mean,
                const float* var, float eps, float* w_out, float* b_out);

#ifdef __cplusplus
}
#endif
#endif
