/*
 * refcpu -- CPU restatement of Tensorium's fp32 convolution hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle and the
 * "port" CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libtensorium_hip.so)
 * never links or calls it.
 *
 * Every routine restates one reference routine (file:line relative to the
 * reference's source/ directory) with the same per-element operation order,
 * so that results are bit-identical to the reference CPU build
 * (USE_AVX2 + USE_MULTITHREADING, AVX2 present).  Pins for each routine are
 * listed in the header of refcpu.c.
 */
#ifndef TENSORIUM_REFCPU_H
#define TENSORIUM_REFCPU_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* worker count P of the steroids pool (steroids.pas:281-296); 0 = max(nproc,4) */
void ref_set_threads(int p);
int ref_get_threads(void);

/* cblas_saxpy -> saxpy_avx2 (ntensors.pas:1308): y = fma(a, x, y) */
void ref_axpy(int64_t n, float a, const float *x, float *y);

/* cblas_sgemm (ntensors.pas:2231-2286); trans flags: 0 = no, 1 = yes */
void ref_sgemm(int transA, int transB, int64_t M, int64_t N, int64_t K,
               float alpha, const float *A, int64_t lda, const float *B,
               int64_t ldb, float beta, float *C, int64_t ldc);
/* cblas_sgemm_batch_strided (ntensors.pas:2288-2304) */
void ref_sgemm_strided_batched(int transA, int transB, int64_t M, int64_t N,
                               int64_t K, float alpha, const float *A,
                               int64_t lda, int64_t strideA, const float *B,
                               int64_t ldb, int64_t strideB, float beta,
                               float *C, int64_t ldc, int64_t strideC,
                               int64_t batch);

/* sim2colStridedBatched (ntensors.pas:11493-11534) over sim2Col (:11415) */
void ref_im2col_batched(int64_t C, int64_t H, int64_t W, int64_t kh,
                        int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                        int64_t sX, int64_t dY, int64_t dX, const float *im,
                        int64_t imStride, float *col, int64_t colStride,
                        int64_t batch);
/* scol2imStridedBatched (ntensors.pas:11833-11879) over scol2im/c2i
 * (:11717, :11650); accumulates into im, serial (race-free) order */
void ref_col2im_batched(int64_t C, int64_t H, int64_t W, int64_t kh,
                        int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                        int64_t sX, int64_t dY, int64_t dX, const float *col,
                        int64_t colStride, float *im, int64_t imStride,
                        int64_t batch);

/* vsAddB / vssAddI_avx (ntensors.pas:4066-4092, 3799): x[b][i][*] += bias[i] */
void ref_forward_bias(float *x, int64_t nb, int64_t blockSize,
                      const float *bias, int64_t batch);
/* vsMulB / vssMulI_avx (ntensors.pas:4112-4135): x[b][i][*] *= scale[i] */
void ref_forward_scale(float *x, int64_t nb, int64_t blockSize,
                       const float *scale, int64_t batch);

/* activation ordinals of TActivationType (ntypes.pas:66) used here */
enum { REF_AC_LOGISTIC = 0, REF_AC_LINEAR = 4, REF_AC_LEAKY = 9 };
/* activate_array (nactivation.pas:508); logistic: exact=1 uses IEEE 1/x in
 * place of vrcpps (nactivation.pas:36-127) */
void ref_activate(float *x, int64_t n, int act, int exact);
/* gradient_array (nactivation.pas:624-670): delta[i] *= grad(x[i]) */
void ref_derive(const float *x, int64_t n, int act, float *delta);

/* TMaxPoolLayer forward (nMaxPoolLayer.pas:265-455): idx may be NULL */
void ref_maxpool_fwd(int64_t batch, int64_t C, int64_t H, int64_t W,
                     int64_t size, int64_t strideX, int64_t strideY,
                     int64_t pad, const float *in, float *out, int64_t *idx);
/* backwardMaxPool (nMaxPoolLayer.pas:501-512) */
void ref_maxpool_bwd(int64_t nOut, const int64_t *idx, const float *dOut,
                     float *dIn);

/* upsample (nupsamplelayer.pas:83-113); w,h = small-side dims */
void ref_upsample(float *in, int64_t w, int64_t h, int64_t C, int64_t batch,
                  int64_t stride, int forward, float scale, float *out);

/* addvv (naddlayer.pas:698): out = a + b */
void ref_addvv(int64_t n, const float *a, const float *b, float *out);

/* TYoloLayer.forward inference (nyololayer.pas:786-830): out = in with the
 * logistic on entries 0,1 and 4.. of each anchor (exact: IEEE reciprocal) */
void ref_yolo_fwd(int64_t batch, int64_t n, int64_t classes, int64_t h,
                  int64_t w, const float *in, float *out, int exact);

/* blockNormalize (ntensors.pas:8693) via _snormblkvv (:4357);
 * exact=1: IEEE division (snormvss :4315), exact=0: rcpss (snormvss_avx :4277) */
void ref_bn_normalize(float *x, int64_t nb, int64_t blockSize,
                      const float *mean, const float *var, int64_t batch,
                      int exact);
/* fuseBatchNorm (nConvolutionLayer.pas:102-126), in place */
void ref_fuse_bn(int64_t F, int64_t filterSize, float *W, float *bias,
                 const float *scales, const float *mean, const float *var);

/* Training-mode batch norm (avx2: 1 = the reference on an AVX2 host, with
 * srss / sVarinceDelta_avx dropping lanes 4..7 when the block length is a
 * multiple of 8; 0 = its Pascal loops, the parity target).
 * TTensor.MeansAndVars (ntensors.pas:9102-9180) over [groups][nch][block]. */
void ref_means_vars(const float *src, int64_t nch, int64_t block, int64_t groups, float *means, float *vars,
                    int avx2);
/* sMeanAndVarianceDelta (ntensors.pas:8831-8898) */
void ref_means_vars_delta(const float *delta, const float *x, const float *mean, const float *var, int64_t nch,
                          int64_t block, int64_t groups, float *mean_delta, float *variance_delta, int avx2);
/* TTensor.addDots (ntensors.pas:7783-7830): dst[i] += dots of channel i */
void ref_add_dots(float *dst, const float *a, const float *b, int64_t nch, int64_t block, int64_t groups,
                  int avx2);
/* softmax (nsoftmaxlayer.pas:81-105) row by row */
void ref_softmax_rows(const float *x, int64_t rows, int64_t n, float temp, float *out);

/* TConvolutionalLayer.forward (nConvolutionLayer.pas:457-566) with
 * Conv2D (ntensors.pas:8252-8345), forwardBias and activate; BN folded.
 * workspace: >= batch*C*k*k*OH*OW floats (unused for 1x1/s1). */
void ref_conv_forward(int64_t batch, int64_t C, int64_t H, int64_t W,
                      int64_t F, int64_t k, int64_t stride, int64_t pad,
                      const float *x, const float *Wt, const float *bias,
                      int act, float *out, float *workspace);

#ifdef __cplusplus
}
#endif
#endif
