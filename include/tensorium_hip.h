/*
 * tensorium_hip.h -- C ABI of libtensorium_hip.so, the MI355X (gfx950)
 * backend for Tensorium's fp32 convolution hot path.
 *
 * Drop-in boundary: the GPU backend object TNNCuda<T> (source/nncuda.pas:
 * 35-200, global singleton `cuda`, ntensors.pas:1055).  Every entry point
 * below names the TNNCuda method (or CPU op-table pointer) it replaces.
 *
 * Conventions (mirroring TNNCuda):
 *  - cdecl, plain C types only: int64_t for SizeInt, int32_t for longint /
 *    boolean / enum ordinals, float for T = single, raw pointers.
 *  - device buffers are (pointer, element offset) pairs; the library never
 *    frees or retains caller buffers.
 *  - all compute is enqueued in order on the context's single stream and is
 *    asynchronous; tnh_h2d / tnh_d2h are blocking, tnh_synchronize waits
 *    (TNNCuda.readBuffer/writeBuffer/finish, nncuda.pas:499-522, 1575).
 *  - every call returns a status (TNH_OK = 0); on failure
 *    tnh_last_error() returns a thread-local message.  This replaces the
 *    reference's SAFE_CALL -> assert (nncuda.pas:237-275).
 *  - matrices are row-major, as in cblas_sgemm with Order ignored
 *    (ntensors.pas:2231).  Tensors are NCHW fp32.
 */
#ifndef TENSORIUM_HIP_H
#define TENSORIUM_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  TNH_OK = 0,
  TNH_ERR_NOT_INITIALIZED = 1,
  TNH_ERR_INVALID_ARG = 2,
  TNH_ERR_HIP = 3,
  TNH_ERR_UNSUPPORTED = 4,
  TNH_ERR_OUT_OF_MEMORY = 5
};

/* TActivationType ordinals (ntypes.pas:66) accepted by the kernels. */
enum { TNH_AC_LOGISTIC = 0, TNH_AC_LINEAR = 4, TNH_AC_LEAKY = 9 };

/* ---- context ---------------------------------------------------------- */
/* TNNCuda.Create(deviceIndex) (nncuda.pas:448): selects the device, creates
 * the context's stream. Calling it again re-targets the context. */
int32_t tnh_init(int32_t device);
/* TNNCuda.Destroy (nncuda.pas:469) */
int32_t tnh_finalize(void);
/* TNNCuda.deviceCount (nncuda.pas:443) */
int32_t tnh_device_count(int32_t *count);
/* TNNCuda.finish (nncuda.pas:1575): waits for the context stream */
int32_t tnh_synchronize(void);
/* message of the last failing call on this thread ("" if none) */
const char *tnh_last_error(void);
/* the hipStream_t kernels are enqueued on */
int32_t tnh_get_stream(void **stream);
/* enqueue on a caller-owned stream instead; NULL selects the HIP null
 * (legacy default) stream, which orders with other blocking streams */
int32_t tnh_set_stream(void *stream);
/* go back to the context's own stream */
int32_t tnh_reset_stream(void);
/* number of compute units of the context device */
int32_t tnh_cu_count(int32_t *count);
/* No reference counterpart: deterministic mode (1) or not (0, default).
 * By default the first call for a conv / SGEMM shape times several tilings
 * and keeps the fastest; tilings that cut K into pieces (split-K, tail
 * split) sum in a different order, so which one wins can change the low
 * bits of the results from one process to the next (always within the
 * fp32 parity bound).  In deterministic mode no timing-based choice is made
 * and no K-cutting tiling is used (tilings forced with
 * tnh_conv2d_set_autotune / tnh_sgemm_set_autotune excepted): every process
 * runs the same kernels and produces the same bits, at some speed cost. */
int32_t tnh_set_deterministic(int32_t enable);

/* ---- HIP graphs (no reference counterpart: the reference launches every
 *      kernel eagerly).  Capture the context's own stream into an executable
 *      graph and replay it; kernels recorded this way skip autotuning, so run
 *      one eager pass first.  The null stream cannot be captured. ---------- */
int32_t tnh_graph_begin(void);
int32_t tnh_graph_end(void **graphExec);
int32_t tnh_graph_launch(void *graphExec);
int32_t tnh_graph_destroy(void *graphExec);

/* ---- memory (TNNCuda.createDeviceBuffer/freeDeviceBuffer/writeBuffer/
 *      readBuffer, nncuda.pas:488, 493, 512, 499) ----------------------- */
int32_t tnh_malloc(int64_t bytes, void **ptr);
int32_t tnh_free(void *ptr);
int32_t tnh_h2d(void *dst, const void *src, int64_t bytes);
int32_t tnh_d2h(void *dst, const void *src, int64_t bytes);

/* ---- timing on the context stream (replaces the telemetry clock,
 *      nopmetrics.pas:56-70, which had to synchronize the stream) ------- */
int32_t tnh_event_create(void **ev);
int32_t tnh_event_destroy(void *ev);
int32_t tnh_event_record(void *ev);
int32_t tnh_event_elapsed_ms(void *start, void *stop, float *ms);
/* No TNNCuda counterpart (it runs one stream): the context stream waits for
 * `ev`, recorded with tnh_event_record while another stream was selected.
 * Forks and joins independent work (a network's yolo head tails) onto a
 * second stream, eagerly or under graph capture.  Scratch is kept per
 * stream (split-K pieces, the channel reductions' partial sums), so calls on
 * different streams may overlap.  Split-K scratch is allocated on a stream's
 * first eager use; a stream captured before any eager call gets none and
 * runs whole-K tilings (correct, possibly slower).  Reduction partials come
 * from spares allocated by tnh_init (4 streams) or on a stream's first eager
 * reduction. */
int32_t tnh_stream_wait_event(void *ev);
/* No TNNCuda counterpart: a second stream (default priority, non-blocking)
 * for tnh_set_stream, so a caller with no other GPU runtime can fork work as
 * above.  tnh_stream_destroy waits for the stream's work, then destroys it;
 * it refuses the context's own stream and the selected one. */
int32_t tnh_stream_create(void **stream);
int32_t tnh_stream_destroy(void *stream);

/* ---- GEMM ------------------------------------------------------------- */
/* TNNCuda.gemm (nncuda.pas:624) / cblas_sgemm (ntensors.pas:2231):
 * C = alpha*op(A)*op(B) + beta*C, all four NN/NT/TN/TT variants.
 * beta = 0 overwrites C without reading it (BLAS semantics). */
int32_t tnh_sgemm(int32_t transA, int32_t transB, int64_t M, int64_t N,
                  int64_t K, float alpha, const float *A, int64_t aOff,
                  int64_t lda, const float *B, int64_t bOff, int64_t ldb,
                  float beta, float *C, int64_t cOff, int64_t ldc);
/* TNNCuda.gemmStridedBatched (nncuda.pas:809) /
 * cblas_sgemm_batch_strided (ntensors.pas:2288); strideA = 0 is legal. */
int32_t tnh_sgemm_strided_batched(int32_t transA, int32_t transB, int64_t M,
                                  int64_t N, int64_t K, float alpha,
                                  const float *A, int64_t aOff, int64_t lda,
                                  int64_t strideA, const float *B,
                                  int64_t bOff, int64_t ldb, int64_t strideB,
                                  float beta, float *C, int64_t cOff,
                                  int64_t ldc, int64_t strideC,
                                  int64_t batch);
/* No reference counterpart: enable (1, default) or disable per-shape timing
 * of the SGEMM tile configuration; forcedConfig >= 0 pins one: 0, 1 the
 * general 128x128 / 64x64 tiles (any K, alignment, size), 2..5 the lean
 * 128x128 / 128x64 / 64x128 / 64x64 tiles (need K % 32 == 0, 16-byte
 * aligned operands with ld % 4 == 0, M and N multiples of 4 where that
 * operand is row-contiguous, C within 2 GiB; other calls fall back to the
 * general tiles), 6..8 the wave-split 32x32 (4 or 8 waves) and 32x64 tiles
 * (K split over the waves of one workgroup; the lean tiles' requirements);
 * -1 lets the library choose.  The whole-K configurations sum k in the same
 * order; the wave-split ones (timed only for problems whose 64x64 tiles
 * number under two per CU, never in the deterministic mode) sum per-wave
 * partials.  The first call for a shape times the candidates as graph
 * replays into a scratch C. */
int32_t tnh_sgemm_set_autotune(int32_t enable, int32_t forcedConfig);

/* ---- im2col / col2im ---------------------------------------------------- */
/* TNNCuda.im2col (nncuda.pas:1144) / sim2Col (ntensors.pas:11415):
 * col[(c*kh+ky)*kw+kx][oy*OW+ox] = im[c][oy*sY-pH+ky*dY][ox*sX-pW+kx*dX] or 0 */
int32_t tnh_im2col(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw,
                   int64_t pH, int64_t pW, int64_t sY, int64_t sX, int64_t dY,
                   int64_t dX, const float *im, int64_t imOff, float *col,
                   int64_t colOff);
/* sim2colStridedBatched (ntensors.pas:11493) */
int32_t tnh_im2col_batched(int64_t C, int64_t H, int64_t W, int64_t kh,
                           int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                           int64_t sX, int64_t dY, int64_t dX, const float *im,
                           int64_t imOff, int64_t imStride, float *col,
                           int64_t colOff, int64_t colStride, int64_t batch);
/* TNNCuda.col2im (nncuda.pas:1212) / scol2im (ntensors.pas:11717):
 * ACCUMULATES into im, adding contributions per pixel in the reference CPU
 * order (existing value first, then ky, kx ascending): bit-exact. */
int32_t tnh_col2im(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw,
                   int64_t pH, int64_t pW, int64_t sY, int64_t sX, int64_t dY,
                   int64_t dX, const float *col, int64_t colOff, float *im,
                   int64_t imOff);
/* scol2imStridedBatched (ntensors.pas:11833) */
int32_t tnh_col2im_batched(int64_t C, int64_t H, int64_t W, int64_t kh,
                           int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                           int64_t sX, int64_t dY, int64_t dX,
                           const float *col, int64_t colOff, int64_t colStride,
                           float *im, int64_t imOff, int64_t imStride,
                           int64_t batch);

/* ---- fused convolution ------------------------------------------------- */
/* weight layouts accepted by tnh_conv2d_fwd */
enum { TNH_WEIGHTS_REFERENCE = 0, TNH_WEIGHTS_TAP_MAJOR = 1 };

/* Replaces the sequence im2col -> gemmStridedBatched -> forwardBias ->
 * ActivateArray of TConvolutionalLayer.forwardGPU
 * (nConvolutionLayer.pas:1051-1118) and the CPU forward
 * (nConvolutionLayer.pas:457-566, Conv2D ntensors.pas:8252) with one
 * implicit-GEMM kernel (BN folded, dilation 1, groups 1):
 *   out[b][f][p] = act(sum_k W[f][k]*col_b[k][p] + bias[f]) (+ residual[b][f][p])
 * x image b starts at x + xOff + b*xBatchStride; out/residual likewise, so a
 * route (concat) destination can be written in place.  bias and residual may
 * be NULL.  The residual add (a following shortcut layer, naddlayer.pas:698)
 * is applied after the activation, exactly as the separate layer would.
 * weightLayout: TNH_WEIGHTS_REFERENCE ([F][C][kh][kw], the reference's
 * storage, nConvolutionLayer.pas:206) or TNH_WEIGHTS_TAP_MAJOR
 * ([F][kh][kw][C], from tnh_conv2d_pack_weights; the fast path).
 * Kernels: any kh x kw from 1 to 32 per side, any stride/padding,
 * dilation 1 (1x1 and 3x3 run the fast tiles; other sizes the LDS-staged
 * tiles 0..5 with a run-time gather).  The first call for a shape may time
 * several tile shapes (see tnh_conv2d_set_autotune). */
int32_t tnh_conv2d_fwd(int64_t batch, int64_t C, int64_t H, int64_t W,
                       int64_t F, int64_t kh, int64_t kw, int64_t pH,
                       int64_t pW, int64_t sY, int64_t sX, const float *x,
                       int64_t xOff, int64_t xBatchStride,
                       const float *weights, int64_t wOff, int32_t weightLayout,
                       const float *bias, int64_t biasOff, int32_t act,
                       const float *residual, int64_t rOff,
                       int64_t rBatchStride, float *out, int64_t outOff,
                       int64_t outBatchStride);
/* output size of tnh_conv2d_fwd: (H + 2p - k)/s + 1 (standard formula) */
int32_t tnh_conv2d_out_dims(int64_t H, int64_t W, int64_t kh, int64_t kw,
                            int64_t pH, int64_t pW, int64_t sY, int64_t sX,
                            int64_t *OH, int64_t *OW);
/* No reference counterpart: the convolution of tnh_conv2d_fwd on
 * channels-last (NHWC) tensors, the layout a network keeps between its
 * layers on this device (the input image stays NCHW).  Pixel (b, y, x) of x
 * starts at x + xOff + ((b*H + y)*W + x)*xPix (xPix >= C: a tensor may be a
 * channel slice of a wider buffer, e.g. a route/concat destination); out
 * and residual likewise with outPix / rPix and the output geometry.
 * Weights are tap-major [F][kh][kw][C] (tnh_conv2d_pack_weights).  Supports
 * 3x3 (any stride/padding) and 1x1 stride 1; C % 4 == 0 (C % 32 == 0 runs
 * the tuned tiles, other C one fixed tile), x and weights 16-byte aligned
 * with xPix % 4 == 0, x, out and residual within 2 GiB each.
 * xPix == 0 with C <= 4 and a 3x3 kernel reads x as NCHW [batch][C][H][W]
 * (the network's first layer).  The results equal tnh_conv2d_fwd's on the
 * same data up to the fp32 summation order (the few-channel path: exactly). */
int32_t tnh_conv2d_fwd_nhwc(int64_t batch, int64_t C, int64_t H, int64_t W,
                            int64_t F, int64_t kh, int64_t kw, int64_t pH,
                            int64_t pW, int64_t sY, int64_t sX,
                            const float *x, int64_t xOff, int64_t xPix,
                            const float *weights, int64_t wOff,
                            const float *bias, int64_t biasOff, int32_t act,
                            const float *residual, int64_t rOff, int64_t rPix,
                            float *out, int64_t outOff, int64_t outPix);
/* No reference counterpart: tnh_conv2d_fwd_nhwc whose result is written only
 * as its nearest-upsampled image, the output of the TUpSampleLayer that
 * follows it (nupsamplelayer.pas:83-146, upsample forward): output pixel
 * (b, y, x), channel f goes to pixels (b, s*y + dy, s*x + dx), dy, dx < s,
 * of out (pixel stride outPix, a channel slice of a route buffer allowed),
 * times upScale; the convolution's own output is not stored.  One launch
 * instead of two (conv, then tnh_upsample_nhwc), the same values bit for
 * bit.  No residual. */
int32_t tnh_conv2d_fwd_nhwc_upsample(int64_t batch, int64_t C, int64_t H,
                                     int64_t W, int64_t F, int64_t kh,
                                     int64_t kw, int64_t pH, int64_t pW,
                                     int64_t sY, int64_t sX, const float *x,
                                     int64_t xOff, int64_t xPix,
                                     const float *weights, int64_t wOff,
                                     const float *bias, int64_t biasOff,
                                     int32_t act, int64_t upStride,
                                     float upScale, float *out,
                                     int64_t outOff, int64_t outPix);
/* No reference counterpart: tnh_conv2d_fwd_nhwc for a yolo head: besides out
 * it writes TYoloLayer.forward's head (nyololayer.pas:786-830, as
 * tnh_yolo_fwd_nhwc) to the NCHW tensor yoloOut + yoloOff
 * [batch][F][OH][OW], F = n * (5 + classes): one launch instead of two, the
 * same values bit for bit.  No residual. */
int32_t tnh_conv2d_fwd_nhwc_yolo(int64_t batch, int64_t C, int64_t H,
                                 int64_t W, int64_t F, int64_t kh, int64_t kw,
                                 int64_t pH, int64_t pW, int64_t sY,
                                 int64_t sX, const float *x, int64_t xOff,
                                 int64_t xPix, const float *weights,
                                 int64_t wOff, const float *bias,
                                 int64_t biasOff, int32_t act, float *out,
                                 int64_t outOff, int64_t outPix, int64_t n,
                                 int64_t classes, float *yoloOut,
                                 int64_t yoloOff);
/* No reference counterpart: tnh_conv2d_fwd_nhwc for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, results and kernels;
 * it calls no hipMalloc / hipFree / allocating library routine:
 *  - the K pieces of tail-split or split-K tiles go to a fixed device array
 *    of tnh_conv2d_noalloc_scratch_bytes() bytes (64 MiB) that each device
 *    holds from tnh_init until the process ends;
 *  - it never autotunes (a timing graph allocates): it runs the tiling forced
 *    by tnh_conv2d_set_autotune, else the one tnh_conv2d_fwd_nhwc tuned for
 *    the same call, else the cost model's choice, so after one tuning call of
 *    tnh_conv2d_fwd_nhwc its output equals that entry point's bit for bit;
 *  - a forced tiling whose pieces need more than the array fails with
 *    TNH_ERR_INVALID_ARG and launches nothing; a tuned one falls back to the
 *    cost model's choice (run whole-K if its pieces do not fit either), whose
 *    sums may differ from the tuned tiling's in the last bits.
 * Every call on a device shares that device's array and the array keeps the
 * last call's contents (nothing in it needs to start at zero): calls that
 * overlap on one device (several streams or host threads) race. */
int32_t tnh_conv2d_fwd_nhwc_noalloc(int64_t batch, int64_t C, int64_t H,
                                    int64_t W, int64_t F, int64_t kh,
                                    int64_t kw, int64_t pH, int64_t pW,
                                    int64_t sY, int64_t sX, const float *x,
                                    int64_t xOff, int64_t xPix,
                                    const float *weights, int64_t wOff,
                                    const float *bias, int64_t biasOff,
                                    int32_t act, const float *residual,
                                    int64_t rOff, int64_t rPix, float *out,
                                    int64_t outOff, int64_t outPix);
/* size of the static scratch of tnh_conv2d_fwd_nhwc_noalloc, in bytes */
int32_t tnh_conv2d_noalloc_scratch_bytes(int64_t *bytes);
/* No reference counterpart (layout helper): dst[f][ky][kx][c] =
 * src[f][c][ky][kx] on the device; src and dst must not overlap. */
int32_t tnh_conv2d_pack_weights(int64_t F, int64_t C, int64_t kh, int64_t kw,
                                const float *src, float *dst);
/* No reference counterpart (layout helper for the training step): from
 * src [F][C][kh][kw], tapMajor[f][ky][kx][c] = src[f][c][ky][kx] (as
 * tnh_conv2d_pack_weights; NULL to skip) and flipped[c][ky][kx][f] =
 * src[f][c][kh-1-ky][kw-1-kx], in one pass.  With the flipped copy the input
 * delta of a stride-1 convolution (backwardGPU's TN gemm + col2im,
 * nConvolutionLayer.pas:1240-1290) is tnh_conv2d_fwd of the output delta: F
 * input channels, C filters, padding kh-1-pad, tap-major weights. */
int32_t tnh_conv2d_pack_weights_dgrad(int64_t F, int64_t C, int64_t kh,
                                      int64_t kw, const float *src,
                                      float *tapMajor, float *flipped);
/* No reference counterpart: enable (1, default) or disable per-shape
 * autotuning of the conv tile shape; forcedConfig >= 0 pins one shape:
 * forcedConfig % 64 is the tile shape (0..5 LDS-staged, 11..19 lean
 * software-pipelined, 20..26 wave-split: K of one tile split over the waves
 * of its workgroup, for 3x3 tap-major or 1x1 layers with C % 32 == 0; 6..10
 * are retired and refused; a shape invalid for the call falls back to the
 * library's choice) and forcedConfig / 64 either the
 * split-K factor (0 or 1: none; up to 16) or a tail split (lean shapes only:
 * the tiles beyond the last whole round are cut into K pieces, summed in K
 * order by the workgroup that finishes a tile's last piece, or by a second
 * kernel where the stream has no arrival counters): 18..31 = forcedConfig / 64 - 16 pieces with
 * rounds of one tile per CU, 34..47 = forcedConfig / 64 - 32 pieces with
 * rounds of one tile per resident workgroup slot; -1 lets the library
 * choose.  Autotuning times each candidate as a graph replay of a few
 * launches on a private stream. */
int32_t tnh_conv2d_set_autotune(int32_t enable, int32_t forcedConfig);

/* ---- epilogue and element-wise ops ------------------------------------- */
/* TNNCuda.forwardBias (nncuda.pas:582): blockSize = dstSize/(srcSize*batch);
 * dst[offset+i] += src[((i/blockSize) % srcSize)*incb] */
int32_t tnh_forward_bias(int64_t dstSize, float *dst, int64_t offset,
                         int64_t srcSize, const float *src, int64_t incb,
                         int64_t batch);
/* TNNCuda.forwardScale (nncuda.pas:1468): dst *= scale[...] likewise */
int32_t tnh_forward_scale(int64_t dstSize, float *dst, int64_t offset,
                          int64_t scaleSize, const float *scale, int64_t incb,
                          int64_t batch);
/* TNNCuda.backwardBias (nncuda.pas:602): dst[f] += sum over batch and the
 * blockSize = srcSize/(dstSize*batch) elements of channel f of src. */
int32_t tnh_backward_bias(int64_t dstSize, float *dst, int64_t srcSize,
                          const float *src, int64_t srcOffset, int64_t incb,
                          int64_t batch);
/* TNNCuda.ActivateArray (nncuda.pas:524): act = ord(TActivationType);
 * acLINEAR launches nothing. Logistic is the IEEE 1/(1+exp(-x)) form. */
int32_t tnh_activate(int64_t N, float *x, int64_t offset, int32_t act);
/* TNNCuda.DeriveArray (nncuda.pas:562): delta[i] *= act'(x[offset+i]) */
int32_t tnh_derive(int64_t N, const float *x, int64_t offset, int32_t act,
                   float *delta);
/* TNNCuda.addvv (nncuda.pas:897): dst[i*incc] = src1[i*inca] + src2[i*incb] */
int32_t tnh_addvv(int64_t N, const float *src1, int64_t src1Offset,
                  int64_t inca, const float *src2, int64_t src2Offset,
                  int64_t incb, float *dst, int64_t dstOffset, int64_t incc);
/* TNNCuda.axpy (nncuda.pas:945): y[i*incy] += a*x[i*incx] */
int32_t tnh_axpy(int64_t N, float a, const float *x, int64_t xOffset,
                 int64_t incx, float *y, int64_t yOffset, int64_t incy);
/* TNNCuda.scale (nncuda.pas:986): x[i*stride] *= a */
int32_t tnh_scale(int64_t N, float a, float *x, int64_t stride);
/* TNNCuda.fill (nncuda.pas:1017): x[offset + i*stride] = val */
int32_t tnh_fill(int64_t N, float *x, int64_t offset, float val,
                 int64_t stride);
/* TNNCuda.copy (nncuda.pas:1037): dst[i*incb] = src[i*inca] */
int32_t tnh_copy(int64_t N, const float *src, int64_t srcOffset, int64_t inca,
                 float *dst, int64_t dstOffset, int64_t incb);
/* TTensor.concat of batched tensors (ntensors.pas:12045, used by
 * TConcatLayer.forward nconcatlayer.pas:115) in per-image (darknet) order:
 * dst[b] = [src0[b] | src1[b] | ...], each src_i holding sizes[i] floats per
 * image.  n <= 8. */
int32_t tnh_route(int64_t batch, int32_t n, const float *const *srcs,
                  const int64_t *sizes, float *dst);

/* ---- pooling / resampling --------------------------------------------- */
/* TNNCuda.forwardMaxPool (nncuda.pas:1088) with the CPU semantics of
 * TMaxPoolLayer.forwardMaxPool (nMaxPoolLayer.pas:363-455): window offset
 * -pad div 2, strict '>', -MaxSingle init, global int64 indices.
 * indexes may be NULL (inference).  outC != c selects maxpool_depth
 * (nMaxPoolLayer.pas:372-399; outH = h, outW = w required): output channel g
 * is the max over input channels g, g + outC, ... < c. */
int32_t tnh_maxpool_fwd(int64_t batch, int64_t outC, int64_t outH,
                        int64_t outW, const float *input, int64_t c,
                        int64_t h, int64_t w, int64_t strideX, int64_t strideY,
                        int64_t padding, int64_t kernelSize, int64_t *indexes,
                        float *output);
/* No reference counterpart: the values of tnh_maxpool_fwd on channels-last
 * tensors, bit for bit (same window scan, strict '>', -MaxSingle start; no
 * indices: the channels-last layout serves inference).  Pixel (b, y, x) of
 * in at in + inOff + ((b*h + y)*w + x)*inPix, of out at out + outOff +
 * ((b*outH + i)*outW + j)*outPix (channel slices of wider buffers allowed).
 * outH/outW as tnh_maxpool_fwd checks them; size, strides, padding <= 64. */
int32_t tnh_maxpool_fwd_nhwc(int64_t batch, int64_t channels, int64_t h,
                             int64_t w, int64_t outH, int64_t outW,
                             int64_t strideX, int64_t strideY, int64_t padding,
                             int64_t kernelSize, const float *in,
                             int64_t inOff, int64_t inPix, float *out,
                             int64_t outOff, int64_t outPix);
/* TNNCuda.backwardMaxPool (nncuda.pas:1121, called at nMaxPoolLayer.pas:699)
 * with its arguments: output = the pooled layer's input delta (accumulated),
 * delta = the layer's own delta.  Result: the CPU order of backwardMaxPool
 * (nMaxPoolLayer.pas:501-512), output[indexes[i]] += delta[i] in ascending
 * i, bit for bit; index -1 (a window of -inf) is skipped.  The library
 * remembers the geometry of the tnh_maxpool_fwd call that last wrote
 * `indexes` (keyed by the pointer, with batch and output shape checked;
 * tnh_free forgets it).  Windows that do not overlap (size <= stride) are
 * scattered, one thread per output (each input element receives at most one
 * delta, so no order matters); overlapping ones are gathered per input
 * element in ascending i.  Indexes that no tnh_maxpool_fwd wrote are
 * scattered with atomic adds: exact when no two windows name one input
 * element.  Only elements that some index names are read or written. */
int32_t tnh_maxpool_bwd(int64_t batch, int64_t outC, int64_t outH,
                        int64_t outW, float *output, const int64_t *indexes,
                        const float *delta);
/* No reference counterpart: tnh_maxpool_bwd with the forward geometry given
 * (h, w, strides, padding and size of the forward call), for indexes the
 * library did not write; the same gather and results. */
int32_t tnh_maxpool_bwd_geom(int64_t batch, int64_t outC, int64_t outH,
                             int64_t outW, float *output,
                             const int64_t *indexes, const float *delta,
                             int64_t h, int64_t w, int64_t strideX,
                             int64_t strideY, int64_t padding,
                             int64_t kernelSize);
/* TNNCuda.upSample (nncuda.pas:1267) / upsample (nupsamplelayer.pas:83):
 * h,w are the small-side dims.  isForward=1: out = scale*in (nearest);
 * isForward=0: in += scale*out summed per input pixel in raster order
 * (gather, bit-exact); zeroIn=1 clears `in` first. */
int32_t tnh_upsample(int64_t batch, int64_t channels, int64_t h, int64_t w,
                     float *in, int64_t stride, int32_t isForward, float scale,
                     float *out, int32_t zeroIn);
/* The forward of tnh_upsample on channels-last tensors (bit-identical
 * values): pixel (b, y, x) of in at in + inOff + ((b*h + y)*w + x)*inPix,
 * of out at out + outOff + ((b*h*stride + y)*w*stride + x)*outPix, so the
 * output can be a channel slice of a route (concat) buffer. */
int32_t tnh_upsample_nhwc(int64_t batch, int64_t channels, int64_t h, int64_t w,
                          int64_t stride, float scale, const float *in,
                          int64_t inOff, int64_t inPix, float *out,
                          int64_t outOff, int64_t outPix);

/* ---- YOLO head ------------------------------------------------------- */
/* TYoloLayer.forward inference part (nyololayer.pas:786-830): out = in, then
 * the logistic on entries x, y (0, 1) and obj + classes (4 .. 4+classes) of
 * each of the n anchors; w, h (2, 3) pass through.  The logistic restates
 * logistic_array (nactivation.pas:36-127): exp(-x) = 2^floor(t) * p(frac(t))
 * with t = -x*log2(e) clamped, p the reference's degree-2 polynomial, then
 * 1/(1+e) by IEEE division (the reference's vrcpps is CPU-specific). */
int32_t tnh_yolo_fwd(int64_t batch, int64_t n, int64_t classes, int64_t h,
                     int64_t w, const float *in, float *out);
/* TYoloLayer.forward (nyololayer.pas:786-830) as tnh_yolo_fwd, reading a
 * channels-last head (pixel (b, y, x) at in + inOff + ((b*h + y)*w + x)*inPix,
 * inPix >= n*(classes+5)) and writing the NCHW head layout
 * [batch][n*(classes+5)][h][w] that tnh_yolo_detections reads; bit-identical
 * values. */
int32_t tnh_yolo_fwd_nhwc(int64_t batch, int64_t n, int64_t classes, int64_t h,
                          int64_t w, const float *in, int64_t inOff,
                          int64_t inPix, float *out);
/* No reference counterpart (the channels-last form of TConcatLayer's copy,
 * nconcatlayer.pas:93-120): dst[dstOff + p*dstPix + c] =
 * src[srcOff + p*srcPix + c] for pixels p and channels c < C. */
int32_t tnh_copy_channels(int64_t pixels, int64_t C, const float *src,
                          int64_t srcOff, int64_t srcPix, float *dst,
                          int64_t dstOff, int64_t dstPix);
/* TNNet.Detections (nnet.pas:584-680) on the device: for every yolo head
 * (heads[i]: a device tensor [batch][n][classes+5][h][w] after tnh_yolo_fwd,
 * hw[2i], hw[2i+1] = h, w; anchors[(i*n + a)*2 + {0,1}] = the mask's anchor
 * width and height in network pixels) TYoloLayer.getDetections
 * (nyololayer.pas:399-450, getBox :105-122, correctBoxes :452-498): every
 * (location, anchor) whose objectness exceeds thresh, in the reference's
 * order (head, then location row-major, then anchor), gets box x, y, w, h
 * (image pixels unless relative; letterbox correction when letter),
 * objectness, and prob[j] = objectness*class_j if that exceeds thresh, else
 * 0.  Device outputs: boxes [batch][capacity][4], objectness
 * [batch][capacity], prob [batch][capacity][classes], counts [batch]
 * (int32, the number of detections; entries beyond capacity are not
 * written).  At most 8 heads and 16 anchors per head. */
int32_t tnh_yolo_detections(int64_t batch, int32_t nHeads,
                            const float *const *heads, const int64_t *hw,
                            int64_t n, int64_t classes, const float *anchors,
                            int64_t netW, int64_t netH, int64_t imgW,
                            int64_t imgH, float thresh, int32_t relative,
                            int32_t letter, int64_t capacity, float *boxes,
                            float *objectness, float *prob, int32_t *counts);
/* TDetectionsHelper.doNMSSort (ntypes.pas:1612-1649) on the device, in place
 * on prob: per class, the detections with a non-zero probability in
 * descending order of it (equal probabilities: detection order; the
 * reference's quicksort leaves that order unspecified), and every later one
 * whose box_iou with a kept one exceeds thresh gets probability 0.  Uses
 * the buffers and counts of tnh_yolo_detections; capacity <= 8192. */
int32_t tnh_yolo_nms_sort(int64_t batch, int64_t classes, int64_t capacity,
                          const float *boxes, float *prob,
                          const int32_t *counts, float thresh);

/* ---- batch norm --------------------------------------------------------- */
/* TNNCuda.normalize (nncuda.pas:1371, called by TBaseLayer.batchNormGPU
 * nbaselayer.pas:620, 632): dst[dstOffset ..] viewed as [groups][srcSize]
 * [blockSize], blockSize = dstSize/(srcSize*groups), normalized per channel
 * i with the CPU semantics of TTensor.blockNormalize (ntensors.pas:8693):
 * x = (x - means[i*meansStride]) / d, IEEE division, with
 * d = max(sqrt(v), 1e-6) (_snormblkvv :4357) when blockSize > 1 and
 * d = sqrt(max(v, 1e-6)) (_snormvv :4338) when blockSize == 1,
 * v = vars[i*varsStride].  (The reference CUDA kernel clamps the variance
 * in both cases; the CPU path is the parity target.) */
int32_t tnh_normalize(int64_t srcSize, int64_t dstSize, int64_t groups,
                      const float *means, int64_t meansStride,
                      const float *vars, int64_t varsStride, float *dst,
                      int64_t dstOffset);
/* TTensor.blockNormalize (ntensors.pas:8693-8718) in the argument order of
 * tnh_forward_bias: the same normalize over dst[offset ..] viewed as
 * [batch][N][dstSize/(N*batch)], unit-stride statistics. */
int32_t tnh_bn_normalize(int64_t dstSize, float *x, int64_t offset, int64_t N,
                         const float *mean, const float *variance,
                         int64_t batch);
/* TNNCuda.forwardScaleAdd (nncuda.pas:1490): dst[offset+i] =
 * fl(scales[f*incb] * dst[offset+i]) + biases[f*incb], f = (i/blockSize) %
 * scaleSize, blockSize = dstSize/(scaleSize*batch): the two roundings of the
 * CPU sequence forwardScale then forwardBias (nbaselayer.pas:366-367). */
int32_t tnh_forward_scale_add(int64_t dstSize, float *dst, int64_t offset,
                              int64_t scaleSize, const float *scales,
                              const float *biases, int64_t incb,
                              int64_t batch);
/* No reference counterpart: the batch-norm forward of TBaseLayer.batchNorm
 * (nbaselayer.pas:335-368) after the statistics, and the layer's
 * activation, in one pass over x [batch][N][block]:
 *   xNorm = (x - mean[f]) / d          (tnh_bn_normalize's arithmetic)
 *   out   = act(fl(scales[f] * xNorm) + biases[f])
 * xNorm may be NULL (inference with rolling statistics).  Bit-identical to
 * the reference's copy / blockNormalize / copy / forwardScale /
 * forwardBias / activate sequence; x, xNorm and out must not overlap. */
int32_t tnh_bn_forward(int64_t dstSize, int64_t N, int64_t batch,
                       const float *x, float *xNorm, float *out,
                       const float *mean, const float *variance,
                       const float *scales, const float *biases, int32_t act);
/* No reference counterpart: tnh_bn_forward over [batch][N][h][w] followed by
 * tnh_maxpool_fwd of its output with size 2, stride 2, padding 0 (the
 * config-3 blocks), in one pass and bit for bit: xNorm and out as
 * tnh_bn_forward writes them (either may be NULL: not stored; the batch-norm
 * backward can form both again), pooled [batch][N][h/2][w/2] and the int64
 * indexes (may be NULL) as the maxpool writes them; tnh_maxpool_bwd then
 * finds that geometry.  h even, w % 4 == 0, 16-byte aligned x, xNorm, out,
 * indexes, 8-byte aligned pooled. */
int32_t tnh_bn_forward_maxpool(int64_t batch, int64_t N, int64_t h, int64_t w,
                               const float *x, float *xNorm, float *out,
                               const float *mean, const float *variance,
                               const float *scales, const float *biases,
                               int32_t act, float *pooled, int64_t *indexes);
/* No reference counterpart: tnh_bn_forward over [batch][N][hw] (hw <= 64)
 * followed by tnh_avgpool_fwd of its output, in one pass and bit for bit:
 * xNorm and out as tnh_bn_forward writes them (either may be NULL: not
 * stored), avg[b][n] the plane's mean as tnh_avgpool_fwd forms it. */
int32_t tnh_bn_forward_avgpool(int64_t batch, int64_t N, int64_t hw,
                               const float *x, float *xNorm, float *out,
                               const float *mean, const float *variance,
                               const float *scales, const float *biases,
                               int32_t act, float *avg);
/* No reference counterpart: tnh_bn_statistics (batch statistics and the
 * rolling update) followed by tnh_bn_forward_maxpool, in three launches
 * instead of four and bit for bit: the statistics' final step is taken by
 * the normalize pass itself.  rollMean / rollVar may both be NULL. */
int32_t tnh_bn_train_forward_maxpool(int64_t batch, int64_t N, int64_t h,
                                     int64_t w, const float *x, float *xNorm,
                                     float *out, float *mean, float *variance,
                                     float *rollMean, float *rollVar,
                                     float momentum, const float *scales,
                                     const float *biases, int32_t act,
                                     float *pooled, int64_t *indexes);
/* No reference counterpart: tnh_bn_statistics followed by
 * tnh_bn_forward_avgpool (hw <= 64), in three launches, bit for bit. */
int32_t tnh_bn_train_forward_avgpool(int64_t batch, int64_t N, int64_t hw,
                                     const float *x, float *xNorm, float *out,
                                     float *mean, float *variance,
                                     float *rollMean, float *rollVar,
                                     float momentum, const float *scales,
                                     const float *biases, int32_t act,
                                     float *avg);

/* ---- the element-wise methods of TNNCuda for the layers around the
 *      convolution path (LRN, logistic / L2 cost, dropout, swish, a yolo
 *      layer with scale_x_y != 1) ------------------------------------- */
/* TNNCuda.subvv / mulvv (nncuda.pas:911, 924): dst = src1 - src2 / src1 * src2
 * element by element, each with its offset and stride. */
int32_t tnh_subvv(int64_t N, const float *src1, int64_t src1Offset,
                  int64_t inca, const float *src2, int64_t src2Offset,
                  int64_t incb, float *dst, int64_t dstOffset, int64_t incc);
int32_t tnh_mulvv(int64_t N, const float *src1, int64_t src1Offset,
                  int64_t inca, const float *src2, int64_t src2Offset,
                  int64_t incb, float *dst, int64_t dstOffset, int64_t incc);
/* TNNCuda.fmavv (nncuda.pas:937, an empty method in the reference): dst =
 * src1 * src2 + src3, a multiply then an add. */
int32_t tnh_fmavv(int64_t N, const float *src1, int64_t src1Offset,
                  int64_t inca, const float *src2, int64_t src2Offset,
                  int64_t incb, const float *src3, int64_t src3Offset,
                  int64_t incc, float *dst, int64_t dstOffset, int64_t incd);
/* TNNCuda.power (nncuda.pas:966): y = x^a, evaluated in double and stored as
 * single (TTensor.power's Math.Power, ntensors.pas:8507). */
int32_t tnh_power(int64_t N, const float *x, int64_t xOffset, int64_t incx,
                  float a, float *y, int64_t yOffset, int64_t incy);
/* TNNCuda.fmavss (nncuda.pas:1290; called by TYoloLayer.forwardGPU for
 * scale_x_y != 1, nyololayer.pas:1099): dst[offset + i] = src[offset + i] *
 * scalar + bias, a multiply then an add (sfmavss, ntensors.pas:3355). */
int32_t tnh_fmavss(int64_t N, const float *src, int64_t offset, float scalar,
                   float bias, float *dst);
/* TNNCuda.crossEntropyLogistic (nncuda.pas:1005): error = -t log(max(p,eps))
 * - (1-t) log(max(1-p,eps)), delta = t - p, in single precision. */
int32_t tnh_cross_entropy_logistic(int64_t N, const float *pred,
                                   const float *truth, float *delta,
                                   float *error);
/* TNNCuda.costL2 (nncuda.pas:1540): r = truth - pred, delta = r, error = r*r */
int32_t tnh_cost_l2(int64_t N, const float *pred, const float *truth,
                    float *delta, float *error);
/* TNNCuda.inverseSqrt (nncuda.pas:1563): dst[i*stride + offset] =
 * 1 / sqrt(max(src[i*stride + offset], 1e-6)); alpha is unused, as in
 * TNNCuda's kernel. */
int32_t tnh_inverse_sqrt(int64_t N, float alpha, const float *src, float *dst,
                         int64_t stride, int64_t offset);
/* TNNCuda.activateArraySWISH (nncuda.pas:544): s = 1/(1 + exp(-x)),
 * outSigmoid = s, out = x*s (x, outSigmoid and out at + offset). */
int32_t tnh_activate_swish(int64_t N, const float *x, int64_t offset,
                           float *outSigmoid, float *out);
/* TNNCuda.forwardDropout (nncuda.pas:1512): rnd[i] = a uniform [0, 1) draw,
 * dst[i] = rnd[i] < probability ? 0 : src[i]*scale.  TNNCuda draws a seed
 * on the host per call; here the caller passes it: element i takes the top
 * 24 bits of splitmix64(seed + i), so a call is reproducible. */
int32_t tnh_dropout_fwd(int64_t N, const float *src, float probability,
                        float scale, int64_t seed, float *rnd, float *dst);
/* TNNCuda.backwardDropout (nncuda.pas:1527): dst = rnd < probability ? 0 :
 * src*scale, with the forward's rnd. */
int32_t tnh_dropout_bwd(int64_t N, const float *src, float probability,
                        float scale, const float *rnd, float *dst);

/* ---- training direction (config-3 step: conv-BN-leaky, pooling,
 *      connected, softmax cross-entropy, SGD) --------------------------- */
/* TNNCuda.meansAndVars (nncuda.pas:1308) with the CPU semantics of
 * TTensor.MeansAndVars (ntensors.pas:9102-9180): src (+offset) viewed as
 * [groups][dstSize][block], block = srcSize/(dstSize*groups);
 * means[i] = sum/(groups*block), vars[i] = sum (x-mean)^2/(groups*block-1). */
int32_t tnh_means_vars(int64_t srcSize, int64_t dstSize, int64_t groups,
                       const float *src, int64_t offset, float *means,
                       float *vars);
/* TNNCuda.means (nncuda.pas:1330, called by TBaseLayer.batchNormGPU at
 * nbaselayer.pas:583): the means of tnh_means_vars alone, the same bits. */
int32_t tnh_means(int64_t srcSize, int64_t dstSize, int64_t groups,
                  const float *src, int64_t offset, float *means);
/* TNNCuda.variances (nncuda.pas:1350, nbaselayer.pas:584): vars[i] =
 * sum (x - means[i])^2 / (groups*block - 1) about the means passed in, the
 * unbiased divisor of the CPU path (ntensors.pas:9102-9180; TNNCuda's `vars`
 * kernel divides by groups*block).  With the means of tnh_means the result
 * equals tnh_means_vars' variances bit for bit. */
int32_t tnh_variances(int64_t srcSize, int64_t dstSize, int64_t groups,
                      const float *src, int64_t offset, const float *means,
                      float *vars);
/* No reference counterpart: tnh_means_vars followed by the rolling-statistics
 * update of TBaseLayer.batchNorm in training (nbaselayer.pas:351-355:
 * rolling.Multiply(1 - momentum), then rolling.axpy(momentum, stat)), in
 * one call: rollingMeans[i] = fma(momentum, means[i], (1 - momentum) *
 * rollingMeans[i]), likewise the variances; bit-identical to tnh_means_vars,
 * tnh_scale and tnh_axpy in sequence.  The rolling buffers may both be NULL. */
int32_t tnh_bn_statistics(int64_t srcSize, int64_t dstSize, int64_t groups,
                          const float *src, int64_t offset, float *means,
                          float *vars, float *rollingMeans, float *rollingVars,
                          float momentum);
/* TNNCuda.meansAndVarsDelta (nncuda.pas:1398) / sMeanAndVarianceDelta
 * (ntensors.pas:8831-8898): mean_delta[i] = sum(delta) * -1/sqrt(max(var,
 * 1e-6)); variance_delta[i] = sum(delta*(x-mean)) * -0.5 *
 * max(var, 1e-6)^-1.5.  delta and x share the offset. */
int32_t tnh_means_vars_delta(int64_t srcSize, int64_t dstSize, int64_t groups,
                             const float *delta, const float *x,
                             int64_t offset, const float *mean,
                             const float *variance, float *mean_delta,
                             float *variance_delta);
/* TNNCuda.normalizeDelta (nncuda.pas:1421) / sNormalizeDelta
 * (ntensors.pas:8900-8960): delta = delta/sqrt(max(var,1e-6)) +
 * ((x-mean)*(2*variance_delta/bs) + mean_delta/bs), bs = block*groups. */
int32_t tnh_normalize_delta(int64_t deltaSize, int64_t meanSize,
                            int64_t groups, float *delta, const float *x,
                            int64_t offset, const float *mean,
                            const float *variance, const float *mean_delta,
                            const float *variance_delta);
/* TNNCuda.addDots (nncuda.pas:1448) / TTensor.addDots (ntensors.pas:7783):
 * dst[i] += sum over (group, block) of src1*src2. */
int32_t tnh_add_dots(int64_t N, int64_t dstSize, int64_t groups,
                     const float *src1, const float *src2, int64_t srcOffset,
                     float *dst);
/* No reference counterpart: the first three steps of batchNormBack
 * (nbaselayer.pas:372-392) in one pass over delta, viewed as
 * [groups][dstSize][block]: delta *= act'(output) (TNNCuda.DeriveArray),
 * scaleUpdates[i] += sum x_norm * delta (addDots), delta *= scales[i]
 * (forwardScale); the same operations per element and the same fixed
 * summation order as those three calls, so the results equal theirs bit for
 * bit.  act: TNH_AC_LINEAR, TNH_AC_LEAKY or TNH_AC_LOGISTIC. */
int32_t tnh_bn_backward_scale(int64_t N, int64_t dstSize, int64_t groups,
                              const float *output, int32_t act,
                              const float *xNorm, const float *scales,
                              float *delta, float *scaleUpdates);
/* No reference counterpart: batchNormBackGPU (nbaselayer.pas:662-712) with
 * the layer's activation derivative before it, in two launches instead of
 * six: one pass doing tnh_bn_backward_scale's work (delta *= act'(output),
 * scaleUpdates += sum x_norm*delta, delta *= scales) and taking
 * tnh_means_vars_delta's sums of the new delta, then tnh_normalize_delta
 * with the mean / variance deltas and the dgamma total formed inside it
 * (four launches when a workgroup would hold more than 16 channel rows).
 * The same operations in the same order as those calls, so the same bits; x
 * is the pre-normalization output, mean / variance the forward's
 * statistics.  xNorm may be NULL (here and in the _maxpool / _avgpool
 * forms): the first pass then forms x_norm from x, mean and variance as
 * tnh_bn_forward forms it (the same bits; the forward need not store it).
 * output may be NULL too when biases is given: act(scales * x_norm +
 * biases) is formed again in the same pass (biases is read only then). */
int32_t tnh_bn_backward(int64_t N, int64_t dstSize, int64_t groups,
                        const float *output, int32_t act, const float *xNorm,
                        const float *x, const float *scales, const float *mean,
                        const float *variance, float *delta,
                        float *scaleUpdates, float *mean_delta,
                        float *variance_delta,
                        const float *biases);
/* No reference counterpart: TMaxPoolLayer.backward (2x2, stride 2) into the
 * zeroed delta of the layer below it, then tnh_bn_backward, with the
 * scatter formed inside tnh_bn_backward's first pass: the same bits as
 * tnh_maxpool_bwd(poolDelta) into a zeroed delta followed by
 * tnh_bn_backward.  delta [groups][dstSize][h][w] is written in full (its
 * contents are not read); h and w even, N = groups*dstSize*h*w < 2^31;
 * poolIndexes must be those that tnh_bn_forward_maxpool or tnh_maxpool_fwd
 * (size 2, stride 2) last wrote over this geometry, else TNH_ERR_ARG. */
int32_t tnh_bn_backward_maxpool(int64_t N, int64_t dstSize, int64_t groups,
                                int64_t h, int64_t w,
                                const int64_t *poolIndexes,
                                const float *poolDelta, const float *output,
                                int32_t act, const float *xNorm,
                                const float *x, const float *scales,
                                const float *mean, const float *variance,
                                float *delta, float *scaleUpdates,
                                float *mean_delta, float *variance_delta,
                                const float *biases);
/* No reference counterpart: TAvgPoolLayer.backward (deltaIn += avgDelta /
 * hw, navgpoollayer.pas:86-100) into the zeroed delta of the layer below it,
 * then tnh_bn_backward, the average pool's spread formed inside
 * tnh_bn_backward's first pass: the same bits as the two calls.  avgDelta
 * [groups][dstSize]; delta is written in full (its contents are not read);
 * N < 2^31. */
int32_t tnh_bn_backward_avgpool(int64_t N, int64_t dstSize, int64_t groups,
                                const float *avgDelta, const float *output,
                                int32_t act, const float *xNorm,
                                const float *x, const float *scales,
                                const float *mean, const float *variance,
                                float *delta, float *scaleUpdates,
                                float *mean_delta, float *variance_delta,
                                const float *biases);
/* TNNCuda.softmaxBatch (nncuda.pas:1056) / softmax (nsoftmaxlayer.pas:81):
 * per (batch, group) row of N values (stride apart): e = exp((x-max)/temp),
 * out = e / sum(e). */
int32_t tnh_softmax_batch(int64_t N, const float *input, int64_t iOffset,
                          int64_t batch, int64_t batchSize, int64_t groups,
                          int64_t groupSize, int64_t stride, float temp,
                          float *output, int64_t oOffset);
/* TNNCuda.crossEntropySoftmax (nncuda.pas:1075) / softmaxCrossEntropy
 * (nsoftmaxlayer.pas:123): error = t != 0 ? -ln(max(p, 1e-6)) : 0;
 * delta = t - p. */
int32_t tnh_cross_entropy_softmax(int64_t N, const float *pred,
                                  const float *truth, float *delta,
                                  float *error);
/* No reference counterpart: the tail of a classifier whose last conv block
 * is followed by TAvgPoolLayer, TConnectedLayer and TSoftmaxLayer with
 * cross-entropy (the config-3 network), forward in one launch (one
 * workgroup per image): avg[b][f] = mean of x[b][f][0 .. hw) (the wave tree of
 * tnh_avgpool_fwd), logits = 0 + sdot(avg_b, W_c) + bias[c] (gemm NT with
 * beta 0 in sdot_avx2's 8-lane order, ntensors.pas:1233-1306, then
 * forwardBias), prob = softmaxBatch of the logits (nsoftmaxlayer.pas:81-105),
 * delta and error of softmaxCrossEntropy (nsoftmaxlayer.pas:123-137).
 * weights [classes][F]; F <= 8192, classes <= 1024.  x NULL: avg holds the
 * averages already (tnh_bn_forward_avgpool wrote them). */
int32_t tnh_softmax_head_forward(int64_t batch, int64_t F, int64_t hw,
                                 int64_t classes, const float *x, float *avg,
                                 const float *weights, const float *biases,
                                 const float *truth, float *logits,
                                 float *prob, float *delta, float *error);
/* No reference counterpart: the backward of the same tail in one launch:
 * delta = clamp(delta, -clampAlpha, clampAlpha) (TConnectedLayer.backward,
 * nconnectedlayer.pas:255), biasUpdates += sum over images of delta
 * (addSums), weightUpdates[c][f] = fma chain over the images of delta[b][c] *
 * avg[b][f] (gemm TN, beta 1, saxpy_avx2's order), avgDelta[b][f] = fma chain
 * over the classes from +0 (gemm NN), deltaIn[b][f][p] += avgDelta[b][f] / hw
 * (TAvgPoolLayer.backward, navgpoollayer.pas:86-100).  deltaIn NULL: that
 * last step is left out (tnh_bn_backward_avgpool takes avgDelta instead). */
int32_t tnh_softmax_head_backward(int64_t batch, int64_t F, int64_t hw,
                                  int64_t classes, float clampAlpha,
                                  float *delta, const float *avg,
                                  const float *weights, float *weightUpdates,
                                  float *biasUpdates, float *avgDelta,
                                  float *deltaIn);
/* TNNCuda.clamp (nncuda.pas:1551): dst = max(min(src, alpha), -alpha) at
 * offset + i*stride (TTensor.Clamp(-1, 1), nconnectedlayer.pas:255). */
int32_t tnh_clamp(int64_t N, float alpha, const float *src, float *dst,
                  int64_t stride, int64_t offset);
/* TAvgPoolLayer.forward (navgpoollayer.pas:60-84; the reference has no GPU
 * version): out[b][c] = sum(in[b][c]) / (h*w). */
int32_t tnh_avgpool_fwd(int64_t batch, int64_t c, int64_t h, int64_t w,
                        const float *input, float *output);
/* TAvgPoolLayer.backward (navgpoollayer.pas:86-100):
 * deltaIn[b][c][k] += delta[b][c] / (h*w). */
int32_t tnh_avgpool_bwd(int64_t batch, int64_t c, int64_t h, int64_t w,
                        const float *delta, float *deltaIn);
/* T*Layer.update weight part (nConvolutionLayer.pas:684-691,
 * nconnectedlayer.pas:344-353), fused: weightUpdates =
 * fma(-decay*batch, weights, weightUpdates); weights = fma(lr/batch,
 * weightUpdates, weights); weightUpdates *= momentum. */
int32_t tnh_sgd_update(int64_t N, float learningRate, int64_t batch,
                       float momentum, float decay, float *weights,
                       float *weightUpdates);
/* No reference counterpart: tnh_sgd_update (the same bits) whose pass also
 * writes each updated weight of nPack <= 8 conv layers of the arena (layer l:
 * [packF][packC][taps] at element packOffset[l]) to its tap-major copy
 * packTap[l] and, when packFlip[l] is not NULL, its flipped copy, as
 * tnh_conv2d_pack_weights_dgrad would after the update: a training step's
 * repacks ride on the update's pass instead of a launch per layer.  The same
 * launch then runs tnh_param_update(nParams, learningRate, batch, momentum,
 * params, paramUpdates) (the biases and scales; nParams 0: none). */
int32_t tnh_sgd_update_pack(int64_t N, float learningRate, int64_t batch,
                            float momentum, float decay, float *weights,
                            float *weightUpdates, int32_t nPack,
                            const int64_t *packOffset, const int64_t *packF,
                            const int64_t *packC, const int64_t *packTaps,
                            float *const *packTap, float *const *packFlip,
                            int64_t nParams, float *params,
                            float *paramUpdates);
/* No reference counterpart: tnh_sgd_update_pack whose layer l may also carry
 * packNPieces[l] > 0 weight-gradient pieces from tnh_conv2d_wgrad_pieces at
 * packPieces[l]: the pass first adds their sum to the layer's weight updates
 * exactly as tnh_conv2d_wgrad with alpha = beta = 1 would have (the same
 * bits), so a training step's weight-gradient reductions ride on the update's
 * pass.  packPieces / packNPieces may be NULL (no pieces anywhere). */
int32_t tnh_sgd_update_pack_pieces(int64_t N, float learningRate, int64_t batch,
                                   float momentum, float decay, float *weights,
                                   float *weightUpdates, int32_t nPack,
                                   const int64_t *packOffset,
                                   const int64_t *packF, const int64_t *packC,
                                   const int64_t *packTaps,
                                   float *const *packTap,
                                   float *const *packFlip,
                                   const float *const *packPieces,
                                   const int32_t *packNPieces, int64_t nParams,
                                   float *params, float *paramUpdates);
/* bias / scale part of the same updates (nConvolutionLayer.pas:694-706):
 * params = fma(lr/batch, paramUpdates, params); paramUpdates *= momentum. */
int32_t tnh_param_update(int64_t N, float learningRate, int64_t batch,
                         float momentum, float *params, float *paramUpdates);
/* Weight gradient of conv backward: replaces the per-image loop
 * `for b: gemm(NoTrans, Trans, F, C*k*k, OH*OW, 1, delta_b, col_b, 1, dW)`
 * (nConvolutionLayer.pas:644-650) with one launch:
 *   C = beta*C + alpha * sum_b A_b * B_b^T,
 *   A_b = A + aOff + b*strideA  ([M][L], row stride lda),
 *   B_b = B + bOff + b*strideB  ([N][L], row stride ldb). */
int32_t tnh_sgemm_nt_batch_reduce(int64_t M, int64_t N, int64_t L,
                                  float alpha, const float *A, int64_t aOff,
                                  int64_t lda, int64_t strideA, const float *B,
                                  int64_t bOff, int64_t ldb, int64_t strideB,
                                  float beta, float *C, int64_t cOff,
                                  int64_t ldc, int64_t batch);
/* No reference counterpart: the weight-gradient step of
 * TConvolutionalLayer.backwardGPU (nConvolutionLayer.pas:1203-1232: im2col of
 * every image of the input, then gemmStridedBatched(NoTrans, Trans, F,
 * C*kh*kw, OH*OW, 1, delta_b, col_b, beta = 1, dW) summed over the batch)
 * in one call whose GEMM gathers the column matrix from the input:
 *   dW = beta*dW + alpha * sum_b delta_b * im2col(x_b)^T,
 * x_b = x + b*xBatchStride ([C][H][W]), delta_b = delta + b*deltaBatchStride
 * ([F][OH*OW]), dW [F][C*kh*kw] in the reference weight order.  Geometry as
 * tnh_im2col (padding, stride, dilation).  When OH*OW % 32 == 0, OW % 4 == 0
 * and OW divides 32 or is a multiple of it, one launch (plus the split-K sum) does
 * it, bit for bit equal to tnh_im2col_batched followed by
 * tnh_sgemm_nt_batch_reduce; otherwise it runs im2col and the product image
 * by image in the stream's workspace. */
int32_t tnh_conv2d_wgrad(int64_t batch, int64_t C, int64_t H, int64_t W,
                         int64_t F, int64_t kh, int64_t kw, int64_t padH,
                         int64_t padW, int64_t strideY, int64_t strideX,
                         int64_t dilY, int64_t dilX, const float *x,
                         int64_t xBatchStride, const float *delta,
                         int64_t deltaBatchStride, float alpha, float beta,
                         float *dW);
/* No reference counterpart: tnh_conv2d_wgrad's product (one launch, the
 * single-launch geometry only, else TNH_ERR_UNSUPPORTED) without its sum:
 * the split's raw sums go to pieces ([*nPieces][F][C*kh*kw], piecesFloats
 * floats available) for tnh_sgd_update_pack_pieces to add to dW with
 * alpha = beta = 1.  pieces NULL: only *nPieces is set (the count depends
 * on the geometry and the device's CU count, not on the data).  Refused
 * (TNH_ERR_UNSUPPORTED) for fewer than 8192 weights cut into several pieces,
 * which tnh_conv2d_wgrad sums a wave per weight in another order.  The pieces
 * live in the caller's memory, so several layers' products can wait for one
 * update. */
int32_t tnh_conv2d_wgrad_pieces(int64_t batch, int64_t C, int64_t H, int64_t W,
                                int64_t F, int64_t kh, int64_t kw,
                                int64_t padH, int64_t padW, int64_t strideY,
                                int64_t strideX, int64_t dilY, int64_t dilX,
                                const float *x, int64_t xBatchStride,
                                const float *delta, int64_t deltaBatchStride,
                                float *pieces, int64_t piecesFloats,
                                int32_t *nPieces);

#ifdef __cplusplus
}
#endif
#endif
