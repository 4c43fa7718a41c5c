/*
 * CPU baseline: restatement of the reference's FP32 CPU convolution
 * algorithms (Winograd F(4,3)/F(2,3) routing, packed SGEMM, implicit GEMM),
 * test infrastructure only.  See cpu_fast.c.
 */
#ifndef SIMDYOLO_CPU_FAST_H
#define SIMDYOLO_CPU_FAST_H
#ifdef __cplusplus
extern "C" {
#endif

typedef struct cf_conv cf_conv;

#define CF_IMPLICIT 0
#define CF_WINOGRAD4 1
#define CF_WINOGRAD2 2
#define CF_DEPTHWISE 3

/* A convolution with folded weights w [oc][ic/groups][k][k] and bias [oc]
 * (NULL: zero), stride s, padding k/2, groups 1 or oc == ic (depthwise). */
cf_conv* cf_conv_create(const float* w, const float* bias, int oc, int ic, int k, int s, int groups, int silu);
void cf_conv_destroy(cf_conv* c);
/* y [n][oc][oh][ow] = act(conv(x [n][ic][h][w]) + bias); y NULL only sizes. */
int cf_conv_run(cf_conv* c, const float* x, int n, int h, int w, float* y, int* oh, int* ow);
/* The algorithm the routing picks for an h x w input (CF_*). */
int cf_conv_algorithm(const cf_conv* c, int h, int w);
/* One detect level into the joined [batch][nc+4][out_anchors] head at anchor
 * offset start: boxes [batch][4*bins][h][w], scores [batch][nc][h][w]. */
void cf_detect_decode(const float* boxes, const float* scores, int batch, int nc, int h, int w, int bins, float stride,
                      int xyxy, float* out, int out_anchors, int start);
/* OpenMP threads a run uses. */
int cf_threads(void);

#ifdef __cplusplus
}
#endif
#endif
