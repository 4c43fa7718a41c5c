/*
 * CPU restatement of SimdYolo's FP32 forward path, used ONLY as test
 * infrastructure: the parity checker for the HIP backend, and the
 * `cpu_baseline` leg of bench.py.  Nothing in the shipped library links,
 * loads or calls this code.
 *
 * Every function cites the reference file:line whose semantics it restates
 * (paths are relative to the SimdYolo repository root).  Arithmetic:
 *   - convolutions accumulate in double (the reference's own unit tests use a
 *     double scalar loop as the truth, tests/SimdYolo.Tests/Program.cs:210-221),
 *     then round to float once, then apply SiLU in float;
 *   - everything else is float arithmetic in the reference's operation order.
 *
 * Pinning: tests/test_oracle_pinning.py checks every function against the
 * reference's own known-answer vectors, torch.nn.functional (conv, pooling),
 * brute force (NMS, top-k full sorts), closed forms (BN fold, DFL with equal
 * logits, linear mask prototypes) and published parameter counts.
 * tests/golden/ holds the committed oracle outputs for the seeded networks.
 */
#ifndef SIMDYOLO_ORACLE_H
#define SIMDYOLO_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* BN fold: src/SimdYolo/PtModel.cs:128-145. */
void or_fold_bn(const float* w, int oc, int per_oc, const float* conv_bias,
                const float* gamma, const float* beta, const float* mean,
                const float* var, float eps, float* w_out, float* b_out);

/* NCHW/OIHW convolution + bias + optional SiLU: src/SimdYolo/Compute.cs:171-284. */
int or_conv2d(const float* x, int n, int c, int h, int w, const float* wt,
              const float* bias, int oc, int kh, int kw, int sh, int sw,
              int pt, int pl, int pb, int pr, int dh, int dw, int groups,
              int silu, float* y, int* oh_out, int* ow_out);

/* x * sigmoid(x): src/SimdYolo/Compute.cs:506,513. */
void or_silu(float* x, size_t count);

/* Max pool, padding excluded: src/SimdYolo/Compute.cs:677-708, CpuSpatial.cs:345-410. */
int or_maxpool(const float* x, int n, int c, int h, int w, int kh, int kw,
               int sh, int sw, int pt, int pl, int pb, int pr, int ceil_mode,
               float* y, int* oh_out, int* ow_out);

/* Nearest resize: src/SimdYolo/CpuSpatial.cs:21-47 (index y*ih/h). */
void or_resize_nearest(const float* x, int n, int c, int ih, int iw, int oh,
                       int ow, float* y);

/* Detect-head decode of one level into a joined [B, nc+4, total] tensor:
 * src/SimdYolo/CpuHead.cs:57-124 with CpuDfl.cs:19-61. */
void or_detect_decode(const float* boxes, const float* scores, int batch,
                      int nc, int h, int w, int bins, float stride, int xyxy,
                      float* out, int out_anchors, int start);

/* Two-stage end-to-end top-k, PT rules: src/SimdYolo/CpuEndToEnd.cs:26-140. */
int or_e2e_select_pt(const float* x, int batch, int channels, int anchors,
                     int classes, int maximum, float* out);
/* Two-stage end-to-end top-k, ONNX rules: src/SimdYolo/CpuEndToEnd.cs:147-241. */
int or_e2e_select_onnx(const float* x, int batch, int channels, int anchors,
                       int classes, int maximum, float* out);

/* Detection decode + greedy NMS: src/SimdYolo/YoloDetector.cs:539-652. */
typedef struct {
  int class_id;
  float confidence, x, y, width, height;
  int anchor;
} or_detection;
typedef struct {
  int source_width, source_height, target_width, target_height;
  float scale_x, scale_y;
  int pad_x, pad_y;
} or_letterbox_t;
/* layout: 0 auto, 1 channels-first, 2 channels-last, 3 end-to-end. */
int or_nms_decode(const float* data, int dim1, int dim2, int layout,
                  int class_count, float confidence, float iou,
                  int max_detections, int max_candidates, int agnostic,
                  const or_letterbox_t* t, or_detection* out, int* count);
float or_iou(const or_detection* a, const or_detection* b);

/* Instance mask decode: src/SimdYolo/CpuMaskDecoder.cs:18-81.  proto is one
 * image's [nm][mh][mw]; box in source coordinates.  Writes width*height
 * probabilities to out (when non-NULL) and the crop to info[0..3] =
 * (left, top, width, height). */
int or_mask_decode(const float* proto, int nm, int mh, int mw, const float* coeffs,
                   const or_detection* box, const or_letterbox_t* t, float* out,
                   int* info);

/* Letterbox preprocess: src/SimdYolo/YoloDetector.cs:448-507. */
int or_letterbox(const uint8_t* pixels, int width, int height, int tw, int th,
                 int bgr, int row_stride, float* out, or_letterbox_t* t);

/* YOLOv8-family detect network (module walk of src/SimdYolo/PtModel.cs:184-220,
 * 267-424, 444-504) on the topology of ultralytics' yolov8.yaml. */
typedef struct {
  float depth, width;
  int max_channels, nc, reg_max;
  float bn_eps;
  /* Segment head (ultralytics Segment, PtModel.cs:353-360) when nm > 0: nm
   * mask coefficients per anchor and a Proto net with npr channels (scaled
   * like any channel count, make_divisible(min(npr, max_channels) * width, 8)). */
  int nm, npr;
} or_yolo_cfg;

/* nn.ConvTranspose2d(ic, oc, 2, stride 2, pad 0, bias): weight [ic][oc][2][2];
 * NCHW [n, ic, h, w] -> [n, oc, 2h, 2w], double accumulation.  The Proto
 * upsample of PtModel.cs:344 (VulkanTransposeConv.cs:13-29 runs it as a 1x1
 * conv plus pixel shuffle). */
void or_conv_transpose2x2(const float* x, int n, int ic, int h, int w, const float* wt, const float* bias, int oc,
                          float* y);
/* Enumerate the parameter tensors in canonical (state_dict) order.  For each
 * tensor writes 6 ints: kind, d0, d1, d2, d3, fan_in (unused dims = 1).
 * Returns the number of tensors (also when `out` is NULL). */
int or_yolov8_layout(const or_yolo_cfg* cfg, int* out, int max_tensors);
/* Forward of a [batch,3,h,w] NCHW input.  Output [batch, nc+4(+nm), anchors]
 * (mask coefficients appended as in CompleteInstanceHead, PtModel.cs:506-526)
 * and, for nm > 0, the prototypes [batch, nm, h/4, w/4] into proto_out. */
int or_yolov8_forward(const or_yolo_cfg* cfg, const float* params,
                      size_t n_params, const float* input, int batch, int h,
                      int w, float* out, size_t out_capacity, float* proto_out);

/* CPU baseline (bench.py's cpu_baseline leg): the YOLOv8 detect walk above
 * with weights loaded once and every convolution on the restatement of the
 * reference's FP32 CPU algorithms in cpu_fast.c (Winograd F(4,3)/F(2,3)
 * routing, packed AVX2/FMA SGEMM, OpenMP).  Detect heads only (nm == 0). */
typedef struct or_fast_model or_fast_model;
or_fast_model* or_fast_yolov8_create(const or_yolo_cfg* cfg, const float* params, size_t n_params);
int or_fast_yolov8_forward(or_fast_model* m, const float* input, int batch, int h, int w, float* out,
                           size_t out_capacity);
void or_fast_yolov8_destroy(or_fast_model* m);
/* OpenMP threads the CPU baseline uses. */
int or_fast_threads(void);

/* YOLO11 detect network (ultralytics yolo11.yaml): C3k2, C2PSA attention
 * (PtModel.cs:339-341, 429-437) and the depthwise class branch of Detect. */
int or_yolo11_layout(const or_yolo_cfg* cfg, int* out, int max_tensors);
int or_yolo11_forward(const or_yolo_cfg* cfg, const float* params,
                      size_t n_params, const float* input, int batch, int h,
                      int w, float* out, size_t out_capacity, float* proto_out);

/* ultralytics yolo26.yaml / yolo26-seg.yaml restated (end-to-end Detect with
 * reg_max 1 and x1 y1 x2 y2 boxes, SPPF shortcut, attention C3k2, Segment26
 * with Proto26).  Writes the head before the end-to-end selection,
 * [B, nc+4(+nm), A]; or_e2e_select_pt selects from it. */
int or_yolo26_layout(const or_yolo_cfg* cfg, int* out, int max_tensors);
int or_yolo26_forward(const or_yolo_cfg* cfg, const float* params, size_t n_params, const float* input, int batch,
                      int h, int w, float* out, size_t out_capacity, float* proto_out);

#ifdef __cplusplus
}
#endif
#endif
