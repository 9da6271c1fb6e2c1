unit nnhip;
{ HIP backend object of Tensorium's fp32 convolution path on MI355X (gfx950).

  TNNHip<T> has the surface of TNNCuda<T> (source/nncuda.pas:35-200): the
  same method names, argument order and meaning, so the layers' GPU hooks
  (forwardGPU / backwardGPU, nConvolutionLayer.pas:1022-1290 and the pool,
  upsample, concat, batch-norm hooks) switch `cuda.` for `hip.` unchanged.
  Every method forwards to one call of libtensorium_hip.so's C ABI
  (include/tensorium_hip.h); a non-zero status raises ETNHError with the
  library's message, where nncuda.pas's SAFE_CALL asserts (:237-275).

  T is Single: the library computes in fp32 (the reference's TSingleTensor).
  Buffers are (device pointer, element offset) pairs as in TNNCuda; the
  library never frees or keeps them.  Work is asynchronous and in order on
  one stream; readBuffer / writeBuffer block and finish() waits, as in
  TNNCuda.

  Every TNNCuda method has a kernel here except its CUDA run-time
  compilation (compileToCUBIN, loadCUBIN, compileFile, loadCUBinFile),
  which raises ETNHError: the kernels are compiled ahead of time for
  gfx950, so there is no source to compile at run time. }

{$mode delphi}{$Z4}{$H+}{$POINTERMATH ON}

interface

uses SysUtils;

const
  libtnh = 'libtensorium_hip.so';

  TNH_OK = 0;
  TNH_WEIGHTS_REFERENCE = 0;   // [F][C][kh][kw], the reference storage (nConvolutionLayer.pas:206)
  TNH_WEIGHTS_TAP_MAJOR = 1;   // [F][kh][kw][C], from packConvWeights

  // TActivationType ordinals (ntypes.pas:66) the kernels take
  TNH_AC_LOGISTIC = 0;
  TNH_AC_LINEAR   = 4;
  TNH_AC_LEAKY    = 9;

type
  PSingle   = ^Single;
  PPSingle  = ^PSingle;
  PInt64    = ^Int64;
  PLongInt  = ^LongInt;
  PPointer  = ^Pointer;
  ETNHError = class(Exception);

// --- C ABI of libtensorium_hip.so (include/tensorium_hip.h) -----------------
function tnh_init(device: LongInt): LongInt; cdecl; external libtnh;
function tnh_finalize: LongInt; cdecl; external libtnh;
function tnh_device_count(count: PLongInt): LongInt; cdecl; external libtnh;
function tnh_synchronize: LongInt; cdecl; external libtnh;
function tnh_last_error: PAnsiChar; cdecl; external libtnh;
function tnh_get_stream(stream: PPointer): LongInt; cdecl; external libtnh;
function tnh_set_stream(stream: Pointer): LongInt; cdecl; external libtnh;
function tnh_reset_stream: LongInt; cdecl; external libtnh;
function tnh_cu_count(count: PLongInt): LongInt; cdecl; external libtnh;
function tnh_set_deterministic(enable: LongInt): LongInt; cdecl; external libtnh;
function tnh_graph_begin: LongInt; cdecl; external libtnh;
function tnh_graph_end(graphExec: PPointer): LongInt; cdecl; external libtnh;
function tnh_graph_launch(graphExec: Pointer): LongInt; cdecl; external libtnh;
function tnh_graph_destroy(graphExec: Pointer): LongInt; cdecl; external libtnh;
function tnh_malloc(bytes: Int64; ptr: PPointer): LongInt; cdecl; external libtnh;
function tnh_free(ptr: Pointer): LongInt; cdecl; external libtnh;
function tnh_h2d(dst, src: Pointer; bytes: Int64): LongInt; cdecl; external libtnh;
function tnh_d2h(dst, src: Pointer; bytes: Int64): LongInt; cdecl; external libtnh;
function tnh_event_create(ev: PPointer): LongInt; cdecl; external libtnh;
function tnh_event_destroy(ev: Pointer): LongInt; cdecl; external libtnh;
function tnh_event_record(ev: Pointer): LongInt; cdecl; external libtnh;
function tnh_stream_wait_event(ev: Pointer): LongInt; cdecl; external libtnh;
function tnh_stream_create(stream: PPointer): LongInt; cdecl; external libtnh;
function tnh_stream_destroy(stream: Pointer): LongInt; cdecl; external libtnh;
function tnh_event_elapsed_ms(start, stop: Pointer; ms: PSingle): LongInt; cdecl; external libtnh;
function tnh_sgemm(transA, transB: LongInt; M, N, K: Int64; alpha: Single; A: PSingle; aOff, lda: Int64;
  B: PSingle; bOff, ldb: Int64; beta: Single; C: PSingle; cOff, ldc: Int64): LongInt; cdecl; external libtnh;
function tnh_sgemm_strided_batched(transA, transB: LongInt; M, N, K: Int64; alpha: Single; A: PSingle;
  aOff, lda, strideA: Int64; B: PSingle; bOff, ldb, strideB: Int64; beta: Single; C: PSingle;
  cOff, ldc, strideC, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_sgemm_set_autotune(enable, forcedConfig: LongInt): LongInt; cdecl; external libtnh;
function tnh_im2col(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX: Int64; im: PSingle; imOff: Int64; col: PSingle;
  colOff: Int64): LongInt; cdecl; external libtnh;
function tnh_im2col_batched(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX: Int64; im: PSingle; imOff, imStride: Int64;
  col: PSingle; colOff, colStride, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_col2im(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX: Int64; col: PSingle; colOff: Int64; im: PSingle;
  imOff: Int64): LongInt; cdecl; external libtnh;
function tnh_col2im_batched(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX: Int64; col: PSingle;
  colOff, colStride: Int64; im: PSingle; imOff, imStride, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_conv2d_fwd(batch, C, H, W, F, kh, kw, pH, pW, sY, sX: Int64; x: PSingle; xOff, xBatchStride: Int64;
  weights: PSingle; wOff: Int64; weightLayout: LongInt; bias: PSingle; biasOff: Int64; act: LongInt;
  residual: PSingle; rOff, rBatchStride: Int64; output: PSingle; outOff, outBatchStride: Int64): LongInt; cdecl;
  external libtnh;
function tnh_conv2d_out_dims(H, W, kh, kw, pH, pW, sY, sX: Int64; OH, OW: PInt64): LongInt; cdecl; external libtnh;
function tnh_conv2d_fwd_nhwc(batch, C, H, W, F, kh, kw, pH, pW, sY, sX: Int64; x: PSingle; xOff, xPix: Int64;
  weights: PSingle; wOff: Int64; bias: PSingle; biasOff: Int64; act: LongInt; residual: PSingle;
  rOff, rPix: Int64; output: PSingle; outOff, outPix: Int64): LongInt; cdecl; external libtnh;
function tnh_conv2d_fwd_nhwc_noalloc(batch, C, H, W, F, kh, kw, pH, pW, sY, sX: Int64; x: PSingle;
  xOff, xPix: Int64; weights: PSingle; wOff: Int64; bias: PSingle; biasOff: Int64; act: LongInt;
  residual: PSingle; rOff, rPix: Int64; output: PSingle; outOff, outPix: Int64): LongInt; cdecl;
  external libtnh;
function tnh_conv2d_fwd_nhwc_upsample(batch, C, H, W, F, kh, kw, pH, pW, sY, sX: Int64; x: PSingle;
  xOff, xPix: Int64; weights: PSingle; wOff: Int64; bias: PSingle; biasOff: Int64; act: LongInt;
  upStride: Int64; upScale: Single; output: PSingle; outOff, outPix: Int64): LongInt; cdecl; external libtnh;
function tnh_conv2d_fwd_nhwc_yolo(batch, C, H, W, F, kh, kw, pH, pW, sY, sX: Int64; x: PSingle;
  xOff, xPix: Int64; weights: PSingle; wOff: Int64; bias: PSingle; biasOff: Int64; act: LongInt;
  output: PSingle; outOff, outPix, n, classes: Int64; yoloOut: PSingle; yoloOff: Int64): LongInt; cdecl;
  external libtnh;
function tnh_conv2d_noalloc_scratch_bytes(bytes: PInt64): LongInt; cdecl; external libtnh;
function tnh_conv2d_pack_weights(F, C, kh, kw: Int64; src, dst: PSingle): LongInt; cdecl; external libtnh;
function tnh_conv2d_pack_weights_dgrad(F, C, kh, kw: Int64; src, tapMajor, flipped: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_conv2d_set_autotune(enable, forcedConfig: LongInt): LongInt; cdecl; external libtnh;
function tnh_forward_bias(dstSize: Int64; dst: PSingle; offset, srcSize: Int64; src: PSingle;
  incb, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_forward_scale(dstSize: Int64; dst: PSingle; offset, scaleSize: Int64; scale: PSingle;
  incb, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_backward_bias(dstSize: Int64; dst: PSingle; srcSize: Int64; src: PSingle;
  srcOffset, incb, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_activate(N: Int64; x: PSingle; offset: Int64; act: LongInt): LongInt; cdecl; external libtnh;
function tnh_derive(N: Int64; x: PSingle; offset: Int64; act: LongInt; delta: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_addvv(N: Int64; src1: PSingle; src1Offset, inca: Int64; src2: PSingle; src2Offset, incb: Int64;
  dst: PSingle; dstOffset, incc: Int64): LongInt; cdecl; external libtnh;
function tnh_axpy(N: Int64; a: Single; x: PSingle; xOffset, incx: Int64; y: PSingle;
  yOffset, incy: Int64): LongInt; cdecl; external libtnh;
function tnh_scale(N: Int64; a: Single; x: PSingle; stride: Int64): LongInt; cdecl; external libtnh;
function tnh_fill(N: Int64; x: PSingle; offset: Int64; val: Single; stride: Int64): LongInt; cdecl; external libtnh;
function tnh_copy(N: Int64; src: PSingle; srcOffset, inca: Int64; dst: PSingle; dstOffset, incb: Int64): LongInt;
  cdecl; external libtnh;
function tnh_route(batch: Int64; n: LongInt; srcs: PPSingle; sizes: PInt64; dst: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_maxpool_fwd(batch, outC, outH, outW: Int64; input: PSingle;
  c, h, w, strideX, strideY, padding, kernelSize: Int64; indexes: PInt64; output: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_maxpool_bwd(batch, outC, outH, outW: Int64; output: PSingle; indexes: PInt64;
  delta: PSingle): LongInt; cdecl; external libtnh;
function tnh_maxpool_bwd_geom(batch, outC, outH, outW: Int64; output: PSingle; indexes: PInt64; delta: PSingle;
  h, w, strideX, strideY, padding, kernelSize: Int64): LongInt; cdecl; external libtnh;
function tnh_upsample(batch, channels, h, w: Int64; input: PSingle; stride: Int64; isForward: LongInt;
  scale: Single; output: PSingle; zeroIn: LongInt): LongInt; cdecl; external libtnh;
function tnh_upsample_nhwc(batch, channels, h, w, stride: Int64; scale: Single; input: PSingle;
  inOff, inPix: Int64; output: PSingle; outOff, outPix: Int64): LongInt; cdecl; external libtnh;
function tnh_maxpool_fwd_nhwc(batch, channels, h, w, outH, outW, strideX, strideY, padding, kernelSize: Int64;
  input: PSingle; inOff, inPix: Int64; output: PSingle; outOff, outPix: Int64): LongInt; cdecl; external libtnh;
function tnh_yolo_fwd(batch, n, classes, h, w: Int64; input, output: PSingle): LongInt; cdecl; external libtnh;
function tnh_yolo_fwd_nhwc(batch, n, classes, h, w: Int64; input: PSingle; inOff, inPix: Int64;
  output: PSingle): LongInt; cdecl; external libtnh;
function tnh_copy_channels(pixels, C: Int64; src: PSingle; srcOff, srcPix: Int64; dst: PSingle;
  dstOff, dstPix: Int64): LongInt; cdecl; external libtnh;
function tnh_yolo_detections(batch: Int64; nHeads: LongInt; heads: PPSingle; hw: PInt64; n, classes: Int64;
  anchors: PSingle; netW, netH, imgW, imgH: Int64; thresh: Single; relative, letter: LongInt; capacity: Int64;
  boxes, objectness, prob: PSingle; counts: PLongInt): LongInt; cdecl; external libtnh;
function tnh_yolo_nms_sort(batch, classes, capacity: Int64; boxes, prob: PSingle; counts: PLongInt;
  thresh: Single): LongInt; cdecl; external libtnh;
function tnh_normalize(srcSize, dstSize, groups: Int64; means: PSingle; meansStride: Int64; vars: PSingle;
  varsStride: Int64; dst: PSingle; dstOffset: Int64): LongInt; cdecl; external libtnh;
function tnh_bn_normalize(dstSize: Int64; x: PSingle; offset, N: Int64; mean, variance: PSingle;
  batch: Int64): LongInt; cdecl; external libtnh;
function tnh_forward_scale_add(dstSize: Int64; dst: PSingle; offset, scaleSize: Int64; scales, biases: PSingle;
  incb, batch: Int64): LongInt; cdecl; external libtnh;
function tnh_bn_forward(dstSize, N, batch: Int64; x, xNorm, output, mean, variance, scales, biases: PSingle;
  act: LongInt): LongInt; cdecl; external libtnh;
function tnh_bn_forward_maxpool(batch, N, h, w: Int64; x, xNorm, output, mean, variance, scales, biases: PSingle;
  act: LongInt; pooled: PSingle; indexes: PInt64): LongInt; cdecl; external libtnh;
function tnh_bn_forward_avgpool(batch, N, hw: Int64; x, xNorm, output, mean, variance, scales, biases: PSingle;
  act: LongInt; avg: PSingle): LongInt; cdecl; external libtnh;
function tnh_bn_train_forward_maxpool(batch, N, h, w: Int64; x, xNorm, output, mean, variance, rollMean,
  rollVar: PSingle; momentum: Single; scales, biases: PSingle; act: LongInt; pooled: PSingle;
  indexes: PInt64): LongInt; cdecl; external libtnh;
function tnh_bn_train_forward_avgpool(batch, N, hw: Int64; x, xNorm, output, mean, variance, rollMean,
  rollVar: PSingle; momentum: Single; scales, biases: PSingle; act: LongInt; avg: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_means_vars(srcSize, dstSize, groups: Int64; src: PSingle; offset: Int64;
  means, vars: PSingle): LongInt; cdecl; external libtnh;
function tnh_means(srcSize, dstSize, groups: Int64; src: PSingle; offset: Int64;
  means: PSingle): LongInt; cdecl; external libtnh;
function tnh_bn_backward_scale(N, dstSize, groups: Int64; output: PSingle; act: LongInt; xNorm, scales, delta,
  scaleUpdates: PSingle): LongInt; cdecl; external libtnh;
function tnh_bn_backward(N, dstSize, groups: Int64; output: PSingle; act: LongInt; xNorm, x, scales, mean,
  variance, delta, scaleUpdates, mean_delta, variance_delta, biases: PSingle): LongInt; cdecl; external libtnh;
function tnh_bn_backward_maxpool(N, dstSize, groups, h, w: Int64; poolIndexes: PInt64; poolDelta, output: PSingle;
  act: LongInt; xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta, variance_delta,
  biases: PSingle): LongInt; cdecl; external libtnh;
function tnh_bn_backward_avgpool(N, dstSize, groups: Int64; avgDelta, output: PSingle; act: LongInt; xNorm, x,
  scales, mean, variance, delta, scaleUpdates, mean_delta, variance_delta, biases: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_variances(srcSize, dstSize, groups: Int64; src: PSingle; offset: Int64;
  means, vars: PSingle): LongInt; cdecl; external libtnh;
function tnh_bn_statistics(srcSize, dstSize, groups: Int64; src: PSingle; offset: Int64;
  means, vars, rollingMeans, rollingVars: PSingle; momentum: Single): LongInt; cdecl; external libtnh;
function tnh_means_vars_delta(srcSize, dstSize, groups: Int64; delta, x: PSingle; offset: Int64;
  mean, variance, mean_delta, variance_delta: PSingle): LongInt; cdecl; external libtnh;
function tnh_normalize_delta(deltaSize, meanSize, groups: Int64; delta, x: PSingle; offset: Int64;
  mean, variance, mean_delta, variance_delta: PSingle): LongInt; cdecl; external libtnh;
function tnh_add_dots(N, dstSize, groups: Int64; src1, src2: PSingle; srcOffset: Int64; dst: PSingle): LongInt;
  cdecl; external libtnh;
function tnh_softmax_batch(N: Int64; input: PSingle; iOffset, batch, batchSize, groups, groupSize, stride: Int64;
  temp: Single; output: PSingle; oOffset: Int64): LongInt; cdecl; external libtnh;
function tnh_cross_entropy_softmax(N: Int64; pred, truth, delta, error: PSingle): LongInt; cdecl; external libtnh;
function tnh_softmax_head_forward(batch, F, hw, classes: Int64; x, avg, weights, biases, truth, logits, prob, delta,
  error: PSingle): LongInt; cdecl; external libtnh;
function tnh_softmax_head_backward(batch, F, hw, classes: Int64; clampAlpha: Single; delta, avg, weights,
  weightUpdates, biasUpdates, avgDelta, deltaIn: PSingle): LongInt; cdecl; external libtnh;
function tnh_clamp(N: Int64; alpha: Single; src, dst: PSingle; stride, offset: Int64): LongInt; cdecl;
  external libtnh;
function tnh_subvv(N: Int64; src1: PSingle; src1Offset, inca: Int64; src2: PSingle; src2Offset, incb: Int64;
  dst: PSingle; dstOffset, incc: Int64): LongInt; cdecl; external libtnh;
function tnh_mulvv(N: Int64; src1: PSingle; src1Offset, inca: Int64; src2: PSingle; src2Offset, incb: Int64;
  dst: PSingle; dstOffset, incc: Int64): LongInt; cdecl; external libtnh;
function tnh_fmavv(N: Int64; src1: PSingle; src1Offset, inca: Int64; src2: PSingle; src2Offset, incb: Int64;
  src3: PSingle; src3Offset, incc: Int64; dst: PSingle; dstOffset, incd: Int64): LongInt; cdecl; external libtnh;
function tnh_power(N: Int64; x: PSingle; xOffset, incx: Int64; a: Single; y: PSingle; yOffset, incy: Int64): LongInt;
  cdecl; external libtnh;
function tnh_fmavss(N: Int64; src: PSingle; offset: Int64; scalar, bias: Single; dst: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_cross_entropy_logistic(N: Int64; pred, truth, delta, error: PSingle): LongInt; cdecl; external libtnh;
function tnh_cost_l2(N: Int64; pred, truth, delta, error: PSingle): LongInt; cdecl; external libtnh;
function tnh_inverse_sqrt(N: Int64; alpha: Single; src, dst: PSingle; stride, offset: Int64): LongInt; cdecl;
  external libtnh;
function tnh_activate_swish(N: Int64; x: PSingle; offset: Int64; outSigmoid, output: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_dropout_fwd(N: Int64; src: PSingle; probability, scale: Single; seed: Int64; rnd, dst: PSingle): LongInt;
  cdecl; external libtnh;
function tnh_dropout_bwd(N: Int64; src: PSingle; probability, scale: Single; rnd, dst: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_avgpool_fwd(batch, c, h, w: Int64; input, output: PSingle): LongInt; cdecl; external libtnh;
function tnh_avgpool_bwd(batch, c, h, w: Int64; delta, deltaIn: PSingle): LongInt; cdecl; external libtnh;
function tnh_sgd_update(N: Int64; learningRate: Single; batch: Int64; momentum, decay: Single;
  weights, weightUpdates: PSingle): LongInt; cdecl; external libtnh;
function tnh_sgd_update_pack(N: Int64; learningRate: Single; batch: Int64; momentum, decay: Single;
  weights, weightUpdates: PSingle; nPack: LongInt; packOffset, packF, packC, packTaps: PInt64;
  packTap, packFlip: PPSingle; nParams: Int64; params, paramUpdates: PSingle): LongInt; cdecl; external libtnh;
function tnh_sgd_update_pack_pieces(N: Int64; learningRate: Single; batch: Int64; momentum, decay: Single;
  weights, weightUpdates: PSingle; nPack: LongInt; packOffset, packF, packC, packTaps: PInt64;
  packTap, packFlip, packPieces: PPSingle; packNPieces: PLongInt; nParams: Int64;
  params, paramUpdates: PSingle): LongInt; cdecl; external libtnh;
function tnh_param_update(N: Int64; learningRate: Single; batch: Int64; momentum: Single;
  params, paramUpdates: PSingle): LongInt; cdecl; external libtnh;
function tnh_sgemm_nt_batch_reduce(M, N, L: Int64; alpha: Single; A: PSingle; aOff, lda, strideA: Int64;
  B: PSingle; bOff, ldb, strideB: Int64; beta: Single; C: PSingle; cOff, ldc, batch: Int64): LongInt; cdecl;
  external libtnh;
function tnh_conv2d_wgrad(batch, C, H, W, F, kh, kw, padH, padW, strideY, strideX, dilY, dilX: Int64; x: PSingle;
  xBatchStride: Int64; delta: PSingle; deltaBatchStride: Int64; alpha, beta: Single; dW: PSingle): LongInt; cdecl;
  external libtnh;
function tnh_conv2d_wgrad_pieces(batch, C, H, W, F, kh, kw, padH, padW, strideY, strideX, dilY, dilX: Int64;
  x: PSingle; xBatchStride: Int64; delta: PSingle; deltaBatchStride: Int64; pieces: PSingle; piecesFloats: Int64;
  nPieces: PLongInt): LongInt; cdecl; external libtnh;

// --- the backend object -------------------------------------------------------
type
  TNNHip<T> = class
  type
    TCUMem = ^T;
    PCUMem = ^TCUMem;
  private
    procedure unsupported(const what: string);
  public
    useBLAS: integer;  // kept for source compatibility with TNNCuda; every GEMM runs this library's kernels
    class function deviceCount(): longint;
    constructor Create(deviceIndex: longint = 0);
    destructor Destroy(); override;
    function CompileLog: ansistring;
    function createDeviceBuffer(const N: SizeInt): TCUMem;
    procedure freeDeviceBuffer(cudaMem: TCUMem);
    procedure readBuffer(const cudaMem: TCUMem; const bufferSize: size_t; const buffer: pointer);
    procedure writeBuffer(const cudaMem: TCUMem; const bufferSize: size_t; const buffer: pointer);
    procedure ActivateArray(const N: SizeInt; const x: TCUMem; const offset: SizeInt; const activation: longint);
    procedure activateArraySWISH(const N: SizeInt; const x: TCUMem; const offset: SizeInt;
      const output_sigmoid, output: TCUMem);
    procedure DeriveArray(const N: SizeInt; const x: TCUMem; const offset: SizeInt; const activation: longint;
      delta: TCUMem);
    procedure forwardBias(const dstSize: SizeInt; const dst: TCUMem; const offset: SizeInt; const srcSize: SizeInt;
      const src: TCUMem; const incb: SizeInt; const batch: SizeInt);
    procedure backwardBias(const dstSize: SizeInt; const dst: TCUMem; const srcSize: SizeInt; const src: TCUMem;
      const srcOffset: SizeInt; const incb: SizeInt; const batch: SizeInt);
    procedure gemm(const transA, transB: boolean; const M, N, K: SizeInt; const ALPHA: T; const A: TCUMem;
      const aOffset: SizeInt; const lda: SizeInt; const B: TCUMem; const bOffset: SizeInt; const ldb: SizeInt;
      const BETA: T; const C: TCUMem; const cOffset: SizeInt; const ldc: SizeInt);
    procedure gemmBatched(const transA, transB: boolean; const M, N, K: SizeInt; const ALPHA: T; const A: PCUMem;
      const aOffset: SizeInt; const lda: SizeInt; const B: PCUMem; const bOffset: SizeInt; const ldb: SizeInt;
      const BETA: T; const C: PCUMem; const cOffset: SizeInt; const ldc: SizeInt; const batchCount: SizeInt);
    procedure gemmStridedBatched(const transA, transB: boolean; const M, N, K: SizeInt; const ALPHA: T; A: TCUMem;
      const aOffset: SizeInt; const lda: SizeInt; const strideA: SizeInt; B: TCUMem; const bOffset: SizeInt;
      const ldb: SizeInt; const strideB: SizeInt; const BETA: T; C: TCUMem; const cOffset: SizeInt;
      const ldc: SizeInt; const strideC: SizeInt; const batchCount: SizeInt);
    procedure addvv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
      const src2Offset, incb: SizeInt; dst: TCUMem; const dstOffset, incc: SizeInt);
    procedure subvv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
      const src2Offset, incb: SizeInt; dst: TCUMem; const dstOffset, incc: SizeInt);
    procedure mulvv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
      const src2Offset, incb: SizeInt; dst: TCUMem; const dstOffset, incc: SizeInt);
    procedure fmavv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
      const src2Offset, incb: SizeInt; const src3: TCUMem; const src3Offset, incc: SizeInt; dst: TCUMem;
      const dstOffset, incd: SizeInt);
    procedure axpy(const N: SizeInt; const a: T; const x: TCUMem; const xOffset: SizeInt; const incx: SizeInt;
      const y: TCUMem; const yOffset: SizeInt; const incy: SizeInt);
    procedure power(const N: SizeInt; const x: TCUMem; const xOffset: SizeInt; const incx: SizeInt; const a: T;
      const y: TCUMem; const yOffset: SizeInt; const incy: SizeInt);
    procedure scale(const N: SizeInt; const a: T; const x: TCUMem; const stride: SizeInt);
    procedure crossEntropyLogistic(const N: SizeInt; const pred, truth: TCUMem; delta, error: TCUMem);
    procedure fill(const N: SizeInt; const x: TCUMem; const offset: SizeInt; const val: T; const stride: SizeInt);
    procedure copy(const N: SizeInt; const src: TCUMem; const srcOffset, inca: SizeInt; const dst: TCUMem;
      const dstOffset, incb: SizeInt);
    procedure softmaxBatch(const N: SizeInt; const input: TCUMem; const iOffset: SizeInt;
      const batch, batch_size, groups, group_size, stride: SizeInt; const temp: T; const output: TCUMem;
      const oOffset: SizeInt);
    procedure crossEntropySoftmax(const N: SizeInt; const pred, truth: TCUMem; delta, error: TCUMem);
    procedure forwardMaxPool(const aBatch, outC, outH, outW: SizeInt; const input: TCUMem; const c, h, w: SizeInt;
      const stride_x, stride_y, padding, kernelSize: SizeInt; indexes, output: TCUMem);
    // the library remembers the geometry of the forwardMaxPool call that
    // wrote `indexes` and gathers in the CPU order
    procedure backwardMaxPool(const aBatch, outC, outH, outW: SizeInt; output: TCUMem; const indexes, delta: TCUMem);
    procedure im2col(const aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
      strideY, strideX, dilationY, dilationX: SizeInt; const im: TCUMem; const imOffset: SizeInt;
      const col: TCUMem; const colOffset: SizeInt);
    procedure col2im(const aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
      strideY, strideX, dilationY, dilationX: SizeInt; const col: TCUMem; const colOffset: SizeInt;
      const im: TCUMem; const imOffset: SizeInt);
    procedure upSample(const aBatch, aChannels, outHeight, outWidth: SizeInt; const &in: TCUMem;
      const stride: SizeInt; const isForward: longint; const scale: T; const &out: TCUMem; const zeroIn: integer = 0);
    procedure fmavss(const N: SizeInt; const src: TCUMem; const offset: SizeInt; const scalar, bias: T; dst: TCUMem);
    procedure meansAndVars(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
      means, vars: TCUMem);
    procedure means(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
      means: TCUMem);
    procedure variances(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
      means, vars: TCUMem);
    procedure normalize(const srcSize, dstSize, groups: SizeInt; means: TCUMem; const meansStride: SizeInt;
      vars: TCUMem; const varsStride: SizeInt; dst: TCUMem; const dstOffset: SizeInt);
    procedure meansAndVarsDelta(const srcSize, dstSize, groups: SizeInt; delta, x: TCUMem; const offset: SizeInt;
      mean, variance, mean_delta, variance_delta: TCUMem);
    procedure normalizeDelta(const deltaSize, meanSize, groups: SizeInt; const delta, x: TCUMem;
      const offset: SizeInt; mean, variance, mean_delta, variance_delta: TCUMem);
    procedure addDots(const N, dstSize, groups: SizeInt; const src1, src2: TCUMem; const srcOffset: SizeInt;
      dst: TCUMem);
    procedure forwardScale(const dstSize: SizeInt; const dst: TCUMem; const offset: SizeInt;
      const scaleSize: SizeInt; const scale: TCUMem; const incb: SizeInt; const batch: SizeInt);
    procedure forwardScaleAdd(const dstSize: SizeInt; const dst: TCUMem; const offset: SizeInt;
      const scaleSize: SizeInt; const scales, biases: TCUMem; const incb: SizeInt; const batch: SizeInt);
    procedure forwardDropout(const N: SizeInt; const src: TCUMem; const probability, scale: T; rnd: TCUMem;
      dst: TCUMem);
    procedure backwardDropout(const N: SizeInt; const src: TCUMem; const probability, scale: T; const rnd: TCUMem;
      dst: TCUMem);
    procedure costL2(const N: SizeInt; const pred, truth, delta, error: TCUMem);
    procedure clamp(const N: SizeInt; const alpha: T; const src, dst: TCUMem; const stride: SizeInt = 1;
      offset: SizeInt = 0);
    procedure inverseSqrt(const N: SizeInt; const alpha: T; const src, dst: TCUMem; const stride: SizeInt = 1;
      offset: SizeInt = 0);
    procedure finish();
    function compileToCUBIN(const code, name: ansistring; const headers: TArray<PAnsiChar> = nil;
      const includeNames: TArray<PAnsiChar> = nil): RawByteString;
    procedure loadCUBIN(const cubin: RawByteString);
    function compileFile(const filename: ansistring): RawByteString;
    procedure loadCUBinFile(const filename: ansistring);

    // --- no TNNCuda counterpart: the convolution path's fused and layout calls
    // one fused conv + bias + activation (+ shortcut): replaces the im2col /
    // gemmStridedBatched / forwardBias / ActivateArray sequence of forwardGPU
    procedure conv2dForward(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX: SizeInt;
      const input: TCUMem; const inOffset, inBatchStride: SizeInt; const weights: TCUMem;
      const weightLayout: longint; const biases: TCUMem; const activation: longint; const residual: TCUMem;
      const resOffset, resBatchStride: SizeInt; const output: TCUMem; const outOffset, outBatchStride: SizeInt);
    procedure conv2dForwardNHWC(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX: SizeInt;
      const input: TCUMem; const inOffset, inPix: SizeInt; const weights, biases: TCUMem; const activation: longint;
      const residual: TCUMem; const resOffset, resPix: SizeInt; const output: TCUMem; const outOffset, outPix: SizeInt;
      const noAlloc: boolean = false);
    // the convolution stores the upsampled image (tnh_upsample_nhwc) instead of its own output
    procedure conv2dForwardNHWCUpsample(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
      strideX: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const weights, biases: TCUMem;
      const activation: longint; const upStride: SizeInt; const upScale: T; const output: TCUMem;
      const outOffset, outPix: SizeInt);
    // the convolution also writes the yolo head (tnh_yolo_fwd_nhwc) to the NCHW tensor yoloOut
    procedure conv2dForwardNHWCYolo(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
      strideX: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const weights, biases: TCUMem;
      const activation: longint; const output: TCUMem; const outOffset, outPix: SizeInt; const n, classes: SizeInt;
      const yoloOut: TCUMem);
    procedure packConvWeights(const filters, c, kernelH, kernelW: SizeInt; const src, dst: TCUMem);
    // the forward's tap-major copy (nil: skipped) and the data gradient's flipped [C][kh][kw][F] copy
    procedure packConvWeightsDgrad(const filters, c, kernelH, kernelW: SizeInt; const src, tapMajor, flipped: TCUMem);
    procedure route(const batch: SizeInt; const srcs: array of TCUMem; const sizes: array of Int64; const dst: TCUMem);
    procedure copyChannels(const pixels, channels: SizeInt; const src: TCUMem; const srcOffset, srcPix: SizeInt;
      const dst: TCUMem; const dstOffset, dstPix: SizeInt);
    procedure upSampleNHWC(const batch, channels, h, w, stride: SizeInt; const scale: T; const input: TCUMem;
      const inOffset, inPix: SizeInt; const output: TCUMem; const outOffset, outPix: SizeInt);
    procedure forwardMaxPoolNHWC(const batch, channels, h, w, outH, outW, strideX, strideY, padding,
      kernelSize: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const output: TCUMem;
      const outOffset, outPix: SizeInt);
    procedure yoloForward(const batch, n, classes, h, w: SizeInt; const input, output: TCUMem);
    procedure yoloForwardNHWC(const batch, n, classes, h, w: SizeInt; const input: TCUMem;
      const inOffset, inPix: SizeInt; const output: TCUMem);
    procedure yoloDetections(const batch: SizeInt; const heads: array of TCUMem; const hw: array of Int64;
      const n, classes: SizeInt; const anchors: PSingle; const netW, netH, imgW, imgH: SizeInt; const thresh: T;
      const relative, letter: boolean; const capacity: SizeInt; const boxes, objectness, prob: TCUMem;
      const counts: PLongInt);
    procedure yoloNmsSort(const batch, classes, capacity: SizeInt; const boxes, prob: TCUMem; const counts: PLongInt;
      const thresh: T);
    procedure blockNormalize(const dstSize: SizeInt; const dst: TCUMem; const offset, N: SizeInt;
      const mean, variance: TCUMem; const batch: SizeInt);
    procedure bnForward(const dstSize, N, batch: SizeInt; const x, xNorm, output, mean, variance, scales,
      biases: TCUMem; const activation: longint);
    // avgpool + connected + softmax cross-entropy, forward and backward, one launch each
    procedure softmaxHeadForward(const batch, F, hw, classes: SizeInt; const x, avg, weights, biases, truth, logits,
      prob, delta, error: TCUMem);
    procedure softmaxHeadBackward(const batch, F, hw, classes: SizeInt; const clampAlpha: T; const delta, avg,
      weights, weightUpdates, biasUpdates, avgDelta, deltaIn: TCUMem);
    // bnForward, then the 2x2 / stride 2 maxpool of its output, in one pass
    procedure bnForwardMaxPool(const batch, N, h, w: SizeInt; const x, xNorm, output, mean, variance, scales,
      biases: TCUMem; const activation: longint; const pooled, indexes: TCUMem);
    // bnForward, then the average of each output plane (hw <= 64), in one pass
    procedure bnForwardAvgPool(const batch, N, hw: SizeInt; const x, xNorm, output, mean, variance, scales,
      biases: TCUMem; const activation: longint; const avg: TCUMem);
    // bnStatistics then bnForwardMaxPool / bnForwardAvgPool, three launches each
    procedure bnTrainForwardMaxPool(const batch, N, h, w: SizeInt; const x, xNorm, output, mean, variance, rollMean,
      rollVar: TCUMem; const momentum: T; const scales, biases: TCUMem; const activation: longint;
      const pooled, indexes: TCUMem);
    procedure bnTrainForwardAvgPool(const batch, N, hw: SizeInt; const x, xNorm, output, mean, variance, rollMean,
      rollVar: TCUMem; const momentum: T; const scales, biases: TCUMem; const activation: longint;
      const avg: TCUMem);
    procedure bnStatistics(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
      means, vars, rollingMeans, rollingVars: TCUMem; const momentum: T);
    // DeriveArray + addDots + forwardScale of batchNormBack in one pass
    procedure bnBackwardScale(const N, dstSize, groups: SizeInt; const output: TCUMem; const activation: longint;
      const xNorm, scales, delta, scaleUpdates: TCUMem);
    // batchNormBackGPU with the activation derivative before it, in four launches
    // (xNorm nil: formed from x, mean, variance; output nil: formed from x_norm, scales and biases)
    procedure bnBackward(const N, dstSize, groups: SizeInt; const output: TCUMem; const activation: longint;
      const xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta, variance_delta: TCUMem;
      const biases: TCUMem = nil);
    // backwardMaxPool (2x2, stride 2) into a zeroed delta, then bnBackward; delta is written in full
    procedure bnBackwardMaxPool(const N, dstSize, groups, h, w: SizeInt; const poolIndexes, poolDelta,
      output: TCUMem; const activation: longint; const xNorm, x, scales, mean, variance, delta, scaleUpdates,
      mean_delta, variance_delta: TCUMem; const biases: TCUMem = nil);
    // avgPoolBackward into a zeroed delta, then bnBackward; delta is written in full
    procedure bnBackwardAvgPool(const N, dstSize, groups: SizeInt; const avgDelta, output: TCUMem;
      const activation: longint; const xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta,
      variance_delta: TCUMem; const biases: TCUMem = nil);
    procedure avgPoolForward(const batch, c, h, w: SizeInt; const input, output: TCUMem);
    procedure avgPoolBackward(const batch, c, h, w: SizeInt; const delta, deltaIn: TCUMem);
    procedure sgdUpdate(const N: SizeInt; const learningRate: T; const batch: SizeInt; const momentum, decay: T;
      weights, weightUpdates: TCUMem);
    // sgdUpdate whose pass also refreshes the packed copies of conv layers in the arena (flip[l] may be nil),
    // then paramUpdate of nParams biases / scales in the same launch
    procedure sgdUpdatePack(const N: SizeInt; const learningRate: T; const batch: SizeInt; const momentum, decay: T;
      weights, weightUpdates: TCUMem; const offsets, F, C, taps: array of Int64; const tapMajor,
      flipped: array of TCUMem; const nParams: SizeInt = 0; params: TCUMem = nil; paramUpdates: TCUMem = nil);
    procedure paramUpdate(const N: SizeInt; const learningRate: T; const batch: SizeInt; const momentum: T;
      params, paramUpdates: TCUMem);
    procedure gemmNTBatchReduce(const M, N, L: SizeInt; const ALPHA: T; const A: TCUMem;
      const aOffset, lda, strideA: SizeInt; const B: TCUMem; const bOffset, ldb, strideB: SizeInt; const BETA: T;
      const C: TCUMem; const cOffset, ldc, batch: SizeInt);
    // backwardGPU's im2col + gemmStridedBatched weight gradient in one call (the im2col in the GEMM's loader)
    procedure convWeightGradient(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX,
      dilY, dilX: SizeInt; const input: TCUMem; const inBatchStride: SizeInt; const delta: TCUMem;
      const deltaBatchStride: SizeInt; const ALPHA, BETA: T; const dW: TCUMem);
    // the same product's split sums into pieces (nil: only counted); returns the number of pieces
    function convWeightGradientPieces(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
      strideX, dilY, dilX: SizeInt; const input: TCUMem; const inBatchStride: SizeInt; const delta: TCUMem;
      const deltaBatchStride: SizeInt; const pieces: TCUMem = nil; const piecesFloats: SizeInt = 0): longint;
    // sgdUpdatePack adding each layer's pieces (count 0: none) to its weight updates first
    procedure sgdUpdatePackPieces(const N: SizeInt; const learningRate: T; const batch: SizeInt;
      const momentum, decay: T; weights, weightUpdates: TCUMem; const offsets, F, C, taps: array of Int64;
      const tapMajor, flipped, pieces: array of TCUMem; const nPieces: array of longint; const nParams: SizeInt;
      params, paramUpdates: TCUMem);
    procedure setDeterministic(const enable: boolean);
    procedure setConvAutotune(const enable: boolean; const forcedConfig: longint = -1);
    procedure setSgemmAutotune(const enable: boolean; const forcedConfig: longint = -1);
    function cuCount: longint;
  end;

implementation

procedure check(st: LongInt);
begin
  if st <> TNH_OK then raise ETNHError.Create(string(tnh_last_error()));
end;

function S(const v): Single; inline;  // a T = Single argument as the ABI's float
begin
  result := Single(v);
end;

procedure TNNHip<T>.unsupported(const what: string);
begin
  raise ETNHError.Create('TNNHip.' + what + ': not provided by libtensorium_hip (outside the fp32 convolution path)');
end;

class function TNNHip<T>.deviceCount(): longint;
begin
  if tnh_device_count(@result) <> TNH_OK then result := 0;
end;

constructor TNNHip<T>.Create(deviceIndex: longint);
begin
  if SizeOf(T) <> SizeOf(Single) then raise ETNHError.Create('TNNHip: only T = Single is supported');
  check(tnh_init(deviceIndex));
end;

destructor TNNHip<T>.Destroy();
begin
  tnh_finalize();
  inherited;
end;

function TNNHip<T>.CompileLog: ansistring;
begin
  result := '';  // kernels are compiled ahead of time; nothing is compiled at run time
end;

function TNNHip<T>.createDeviceBuffer(const N: SizeInt): TCUMem;
var p: Pointer;
begin
  check(tnh_malloc(N * SizeOf(T), @p));
  result := p;
end;

procedure TNNHip<T>.freeDeviceBuffer(cudaMem: TCUMem);
begin
  check(tnh_free(cudaMem));
end;

procedure TNNHip<T>.readBuffer(const cudaMem: TCUMem; const bufferSize: size_t; const buffer: pointer);
begin
  check(tnh_d2h(buffer, cudaMem, bufferSize));
end;

procedure TNNHip<T>.writeBuffer(const cudaMem: TCUMem; const bufferSize: size_t; const buffer: pointer);
begin
  check(tnh_h2d(cudaMem, buffer, bufferSize));
end;

procedure TNNHip<T>.ActivateArray(const N: SizeInt; const x: TCUMem; const offset: SizeInt; const activation: longint);
begin
  check(tnh_activate(N, PSingle(x), offset, activation));
end;

procedure TNNHip<T>.activateArraySWISH(const N: SizeInt; const x: TCUMem; const offset: SizeInt;
  const output_sigmoid, output: TCUMem);
begin
  check(tnh_activate_swish(N, PSingle(x), offset, PSingle(output_sigmoid), PSingle(output)));
end;

procedure TNNHip<T>.DeriveArray(const N: SizeInt; const x: TCUMem; const offset: SizeInt; const activation: longint;
  delta: TCUMem);
begin
  check(tnh_derive(N, PSingle(x), offset, activation, PSingle(delta)));
end;

procedure TNNHip<T>.forwardBias(const dstSize: SizeInt; const dst: TCUMem; const offset: SizeInt;
  const srcSize: SizeInt; const src: TCUMem; const incb: SizeInt; const batch: SizeInt);
begin
  check(tnh_forward_bias(dstSize, PSingle(dst), offset, srcSize, PSingle(src), incb, batch));
end;

procedure TNNHip<T>.backwardBias(const dstSize: SizeInt; const dst: TCUMem; const srcSize: SizeInt;
  const src: TCUMem; const srcOffset: SizeInt; const incb: SizeInt; const batch: SizeInt);
begin
  check(tnh_backward_bias(dstSize, PSingle(dst), srcSize, PSingle(src), srcOffset, incb, batch));
end;

procedure TNNHip<T>.gemm(const transA, transB: boolean; const M, N, K: SizeInt; const ALPHA: T; const A: TCUMem;
  const aOffset: SizeInt; const lda: SizeInt; const B: TCUMem; const bOffset: SizeInt; const ldb: SizeInt;
  const BETA: T; const C: TCUMem; const cOffset: SizeInt; const ldc: SizeInt);
begin
  check(tnh_sgemm(ord(transA), ord(transB), M, N, K, S(ALPHA), PSingle(A), aOffset, lda, PSingle(B), bOffset, ldb,
    S(BETA), PSingle(C), cOffset, ldc));
end;

// A, B, C: host arrays of batchCount device pointers; one GEMM per entry
procedure TNNHip<T>.gemmBatched(const transA, transB: boolean; const M, N, K: SizeInt; const ALPHA: T;
  const A: PCUMem; const aOffset: SizeInt; const lda: SizeInt; const B: PCUMem; const bOffset: SizeInt;
  const ldb: SizeInt; const BETA: T; const C: PCUMem; const cOffset: SizeInt; const ldc: SizeInt;
  const batchCount: SizeInt);
var i: SizeInt;
begin
  for i := 0 to batchCount - 1 do
    check(tnh_sgemm(ord(transA), ord(transB), M, N, K, S(ALPHA), PSingle(A[i]), aOffset, lda, PSingle(B[i]),
      bOffset, ldb, S(BETA), PSingle(C[i]), cOffset, ldc));
end;

procedure TNNHip<T>.gemmStridedBatched(const transA, transB: boolean; const M, N, K: SizeInt; const ALPHA: T;
  A: TCUMem; const aOffset: SizeInt; const lda: SizeInt; const strideA: SizeInt; B: TCUMem; const bOffset: SizeInt;
  const ldb: SizeInt; const strideB: SizeInt; const BETA: T; C: TCUMem; const cOffset: SizeInt; const ldc: SizeInt;
  const strideC: SizeInt; const batchCount: SizeInt);
begin
  check(tnh_sgemm_strided_batched(ord(transA), ord(transB), M, N, K, S(ALPHA), PSingle(A), aOffset, lda, strideA,
    PSingle(B), bOffset, ldb, strideB, S(BETA), PSingle(C), cOffset, ldc, strideC, batchCount));
end;

procedure TNNHip<T>.addvv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
  const src2Offset, incb: SizeInt; dst: TCUMem; const dstOffset, incc: SizeInt);
begin
  check(tnh_addvv(N, PSingle(src1), src1Offset, inca, PSingle(src2), src2Offset, incb, PSingle(dst), dstOffset,
    incc));
end;

procedure TNNHip<T>.subvv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
  const src2Offset, incb: SizeInt; dst: TCUMem; const dstOffset, incc: SizeInt);
begin
  check(tnh_subvv(N, PSingle(src1), src1Offset, inca, PSingle(src2), src2Offset, incb, PSingle(dst), dstOffset,
    incc));
end;

procedure TNNHip<T>.mulvv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
  const src2Offset, incb: SizeInt; dst: TCUMem; const dstOffset, incc: SizeInt);
begin
  check(tnh_mulvv(N, PSingle(src1), src1Offset, inca, PSingle(src2), src2Offset, incb, PSingle(dst), dstOffset,
    incc));
end;

procedure TNNHip<T>.fmavv(const N: SizeInt; const src1: TCUMem; const src1Offset, inca: SizeInt; const src2: TCUMem;
  const src2Offset, incb: SizeInt; const src3: TCUMem; const src3Offset, incc: SizeInt; dst: TCUMem;
  const dstOffset, incd: SizeInt);
begin
  check(tnh_fmavv(N, PSingle(src1), src1Offset, inca, PSingle(src2), src2Offset, incb, PSingle(src3), src3Offset,
    incc, PSingle(dst), dstOffset, incd));
end;

procedure TNNHip<T>.axpy(const N: SizeInt; const a: T; const x: TCUMem; const xOffset: SizeInt; const incx: SizeInt;
  const y: TCUMem; const yOffset: SizeInt; const incy: SizeInt);
begin
  check(tnh_axpy(N, S(a), PSingle(x), xOffset, incx, PSingle(y), yOffset, incy));
end;

procedure TNNHip<T>.power(const N: SizeInt; const x: TCUMem; const xOffset: SizeInt; const incx: SizeInt;
  const a: T; const y: TCUMem; const yOffset: SizeInt; const incy: SizeInt);
begin
  check(tnh_power(N, PSingle(x), xOffset, incx, S(a), PSingle(y), yOffset, incy));
end;

procedure TNNHip<T>.scale(const N: SizeInt; const a: T; const x: TCUMem; const stride: SizeInt);
begin
  check(tnh_scale(N, S(a), PSingle(x), stride));
end;

procedure TNNHip<T>.crossEntropyLogistic(const N: SizeInt; const pred, truth: TCUMem; delta, error: TCUMem);
begin
  check(tnh_cross_entropy_logistic(N, PSingle(pred), PSingle(truth), PSingle(delta), PSingle(error)));
end;

procedure TNNHip<T>.fill(const N: SizeInt; const x: TCUMem; const offset: SizeInt; const val: T;
  const stride: SizeInt);
begin
  check(tnh_fill(N, PSingle(x), offset, S(val), stride));
end;

procedure TNNHip<T>.copy(const N: SizeInt; const src: TCUMem; const srcOffset, inca: SizeInt; const dst: TCUMem;
  const dstOffset, incb: SizeInt);
begin
  check(tnh_copy(N, PSingle(src), srcOffset, inca, PSingle(dst), dstOffset, incb));
end;

procedure TNNHip<T>.softmaxBatch(const N: SizeInt; const input: TCUMem; const iOffset: SizeInt;
  const batch, batch_size, groups, group_size, stride: SizeInt; const temp: T; const output: TCUMem;
  const oOffset: SizeInt);
begin
  check(tnh_softmax_batch(N, PSingle(input), iOffset, batch, batch_size, groups, group_size, stride, S(temp),
    PSingle(output), oOffset));
end;

procedure TNNHip<T>.crossEntropySoftmax(const N: SizeInt; const pred, truth: TCUMem; delta, error: TCUMem);
begin
  check(tnh_cross_entropy_softmax(N, PSingle(pred), PSingle(truth), PSingle(delta), PSingle(error)));
end;

procedure TNNHip<T>.forwardMaxPool(const aBatch, outC, outH, outW: SizeInt; const input: TCUMem;
  const c, h, w: SizeInt; const stride_x, stride_y, padding, kernelSize: SizeInt; indexes, output: TCUMem);
begin
  check(tnh_maxpool_fwd(aBatch, outC, outH, outW, PSingle(input), c, h, w, stride_x, stride_y, padding, kernelSize,
    PInt64(indexes), PSingle(output)));
end;

procedure TNNHip<T>.backwardMaxPool(const aBatch, outC, outH, outW: SizeInt; output: TCUMem;
  const indexes, delta: TCUMem);
begin
  check(tnh_maxpool_bwd(aBatch, outC, outH, outW, PSingle(output), PInt64(indexes), PSingle(delta)));
end;

procedure TNNHip<T>.im2col(const aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
  strideY, strideX, dilationY, dilationX: SizeInt; const im: TCUMem; const imOffset: SizeInt; const col: TCUMem;
  const colOffset: SizeInt);
begin
  check(tnh_im2col(aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideY, strideX,
    dilationY, dilationX, PSingle(im), imOffset, PSingle(col), colOffset));
end;

procedure TNNHip<T>.col2im(const aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
  strideY, strideX, dilationY, dilationX: SizeInt; const col: TCUMem; const colOffset: SizeInt; const im: TCUMem;
  const imOffset: SizeInt);
begin
  check(tnh_col2im(aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideY, strideX,
    dilationY, dilationX, PSingle(col), colOffset, PSingle(im), imOffset));
end;

procedure TNNHip<T>.upSample(const aBatch, aChannels, outHeight, outWidth: SizeInt; const &in: TCUMem;
  const stride: SizeInt; const isForward: longint; const scale: T; const &out: TCUMem; const zeroIn: integer);
begin
  check(tnh_upsample(aBatch, aChannels, outHeight, outWidth, PSingle(&in), stride, isForward, S(scale),
    PSingle(&out), zeroIn));
end;

procedure TNNHip<T>.fmavss(const N: SizeInt; const src: TCUMem; const offset: SizeInt; const scalar, bias: T;
  dst: TCUMem);
begin
  check(tnh_fmavss(N, PSingle(src), offset, S(scalar), S(bias), PSingle(dst)));
end;

procedure TNNHip<T>.meansAndVars(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
  means, vars: TCUMem);
begin
  check(tnh_means_vars(srcSize, dstSize, groups, PSingle(src), offset, PSingle(means), PSingle(vars)));
end;

procedure TNNHip<T>.means(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
  means: TCUMem);
begin
  check(tnh_means(srcSize, dstSize, groups, PSingle(src), offset, PSingle(means)));
end;

procedure TNNHip<T>.variances(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
  means, vars: TCUMem);
begin
  check(tnh_variances(srcSize, dstSize, groups, PSingle(src), offset, PSingle(means), PSingle(vars)));
end;

procedure TNNHip<T>.normalize(const srcSize, dstSize, groups: SizeInt; means: TCUMem; const meansStride: SizeInt;
  vars: TCUMem; const varsStride: SizeInt; dst: TCUMem; const dstOffset: SizeInt);
begin
  check(tnh_normalize(srcSize, dstSize, groups, PSingle(means), meansStride, PSingle(vars), varsStride, PSingle(dst),
    dstOffset));
end;

procedure TNNHip<T>.meansAndVarsDelta(const srcSize, dstSize, groups: SizeInt; delta, x: TCUMem;
  const offset: SizeInt; mean, variance, mean_delta, variance_delta: TCUMem);
begin
  check(tnh_means_vars_delta(srcSize, dstSize, groups, PSingle(delta), PSingle(x), offset, PSingle(mean),
    PSingle(variance), PSingle(mean_delta), PSingle(variance_delta)));
end;

procedure TNNHip<T>.normalizeDelta(const deltaSize, meanSize, groups: SizeInt; const delta, x: TCUMem;
  const offset: SizeInt; mean, variance, mean_delta, variance_delta: TCUMem);
begin
  check(tnh_normalize_delta(deltaSize, meanSize, groups, PSingle(delta), PSingle(x), offset, PSingle(mean),
    PSingle(variance), PSingle(mean_delta), PSingle(variance_delta)));
end;

procedure TNNHip<T>.addDots(const N, dstSize, groups: SizeInt; const src1, src2: TCUMem; const srcOffset: SizeInt;
  dst: TCUMem);
begin
  check(tnh_add_dots(N, dstSize, groups, PSingle(src1), PSingle(src2), srcOffset, PSingle(dst)));
end;

procedure TNNHip<T>.forwardScale(const dstSize: SizeInt; const dst: TCUMem; const offset: SizeInt;
  const scaleSize: SizeInt; const scale: TCUMem; const incb: SizeInt; const batch: SizeInt);
begin
  check(tnh_forward_scale(dstSize, PSingle(dst), offset, scaleSize, PSingle(scale), incb, batch));
end;

procedure TNNHip<T>.forwardScaleAdd(const dstSize: SizeInt; const dst: TCUMem; const offset: SizeInt;
  const scaleSize: SizeInt; const scales, biases: TCUMem; const incb: SizeInt; const batch: SizeInt);
begin
  check(tnh_forward_scale_add(dstSize, PSingle(dst), offset, scaleSize, PSingle(scales), PSingle(biases), incb,
    batch));
end;

procedure TNNHip<T>.forwardDropout(const N: SizeInt; const src: TCUMem; const probability, scale: T; rnd: TCUMem;
  dst: TCUMem);
begin
  // a fresh seed per call, drawn on the host as TNNCuda does (nncuda.pas:1521)
  check(tnh_dropout_fwd(N, PSingle(src), S(probability), S(scale), random($10000000), PSingle(rnd), PSingle(dst)));
end;

procedure TNNHip<T>.backwardDropout(const N: SizeInt; const src: TCUMem; const probability, scale: T;
  const rnd: TCUMem; dst: TCUMem);
begin
  check(tnh_dropout_bwd(N, PSingle(src), S(probability), S(scale), PSingle(rnd), PSingle(dst)));
end;

procedure TNNHip<T>.costL2(const N: SizeInt; const pred, truth, delta, error: TCUMem);
begin
  check(tnh_cost_l2(N, PSingle(pred), PSingle(truth), PSingle(delta), PSingle(error)));
end;

procedure TNNHip<T>.clamp(const N: SizeInt; const alpha: T; const src, dst: TCUMem; const stride: SizeInt;
  offset: SizeInt);
begin
  check(tnh_clamp(N, S(alpha), PSingle(src), PSingle(dst), stride, offset));
end;

procedure TNNHip<T>.inverseSqrt(const N: SizeInt; const alpha: T; const src, dst: TCUMem; const stride: SizeInt;
  offset: SizeInt);
begin
  check(tnh_inverse_sqrt(N, S(alpha), PSingle(src), PSingle(dst), stride, offset));
end;

procedure TNNHip<T>.finish();
begin
  check(tnh_synchronize());
end;

function TNNHip<T>.compileToCUBIN(const code, name: ansistring; const headers: TArray<PAnsiChar>;
  const includeNames: TArray<PAnsiChar>): RawByteString;
begin
  result := '';
  unsupported('compileToCUBIN (kernels are compiled ahead of time for gfx950)');
end;

procedure TNNHip<T>.loadCUBIN(const cubin: RawByteString);
begin
  unsupported('loadCUBIN (kernels are compiled ahead of time for gfx950)');
end;

function TNNHip<T>.compileFile(const filename: ansistring): RawByteString;
begin
  result := '';
  unsupported('compileFile (kernels are compiled ahead of time for gfx950)');
end;

procedure TNNHip<T>.loadCUBinFile(const filename: ansistring);
begin
  unsupported('loadCUBinFile (kernels are compiled ahead of time for gfx950)');
end;

procedure TNNHip<T>.conv2dForward(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
  strideX: SizeInt; const input: TCUMem; const inOffset, inBatchStride: SizeInt; const weights: TCUMem;
  const weightLayout: longint; const biases: TCUMem; const activation: longint; const residual: TCUMem;
  const resOffset, resBatchStride: SizeInt; const output: TCUMem; const outOffset, outBatchStride: SizeInt);
begin
  check(tnh_conv2d_fwd(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX, PSingle(input),
    inOffset, inBatchStride, PSingle(weights), 0, weightLayout, PSingle(biases), 0, activation, PSingle(residual),
    resOffset, resBatchStride, PSingle(output), outOffset, outBatchStride));
end;

procedure TNNHip<T>.conv2dForwardNHWC(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
  strideX: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const weights, biases: TCUMem;
  const activation: longint; const residual: TCUMem; const resOffset, resPix: SizeInt; const output: TCUMem;
  const outOffset, outPix: SizeInt; const noAlloc: boolean);
begin
  if noAlloc then
    check(tnh_conv2d_fwd_nhwc_noalloc(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX,
      PSingle(input), inOffset, inPix, PSingle(weights), 0, PSingle(biases), 0, activation, PSingle(residual),
      resOffset, resPix, PSingle(output), outOffset, outPix))
  else
    check(tnh_conv2d_fwd_nhwc(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX,
      PSingle(input), inOffset, inPix, PSingle(weights), 0, PSingle(biases), 0, activation, PSingle(residual),
      resOffset, resPix, PSingle(output), outOffset, outPix));
end;

procedure TNNHip<T>.conv2dForwardNHWCUpsample(const batch, c, h, w, filters, kernelH, kernelW, padH, padW,
  strideY, strideX: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const weights, biases: TCUMem;
  const activation: longint; const upStride: SizeInt; const upScale: T; const output: TCUMem;
  const outOffset, outPix: SizeInt);
begin
  check(tnh_conv2d_fwd_nhwc_upsample(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX,
    PSingle(input), inOffset, inPix, PSingle(weights), 0, PSingle(biases), 0, activation, upStride, S(upScale),
    PSingle(output), outOffset, outPix));
end;

procedure TNNHip<T>.conv2dForwardNHWCYolo(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
  strideX: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const weights, biases: TCUMem;
  const activation: longint; const output: TCUMem; const outOffset, outPix: SizeInt; const n, classes: SizeInt;
  const yoloOut: TCUMem);
begin
  check(tnh_conv2d_fwd_nhwc_yolo(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX,
    PSingle(input), inOffset, inPix, PSingle(weights), 0, PSingle(biases), 0, activation, PSingle(output),
    outOffset, outPix, n, classes, PSingle(yoloOut), 0));
end;

procedure TNNHip<T>.packConvWeights(const filters, c, kernelH, kernelW: SizeInt; const src, dst: TCUMem);
begin
  check(tnh_conv2d_pack_weights(filters, c, kernelH, kernelW, PSingle(src), PSingle(dst)));
end;

procedure TNNHip<T>.packConvWeightsDgrad(const filters, c, kernelH, kernelW: SizeInt;
  const src, tapMajor, flipped: TCUMem);
begin
  check(tnh_conv2d_pack_weights_dgrad(filters, c, kernelH, kernelW, PSingle(src), PSingle(tapMajor),
    PSingle(flipped)));
end;

procedure TNNHip<T>.route(const batch: SizeInt; const srcs: array of TCUMem; const sizes: array of Int64;
  const dst: TCUMem);
var p: array of PSingle; i: integer;
begin
  SetLength(p, Length(srcs));
  for i := 0 to High(srcs) do p[i] := PSingle(srcs[i]);
  check(tnh_route(batch, Length(srcs), @p[0], @sizes[0], PSingle(dst)));
end;

procedure TNNHip<T>.copyChannels(const pixels, channels: SizeInt; const src: TCUMem; const srcOffset,
  srcPix: SizeInt; const dst: TCUMem; const dstOffset, dstPix: SizeInt);
begin
  check(tnh_copy_channels(pixels, channels, PSingle(src), srcOffset, srcPix, PSingle(dst), dstOffset, dstPix));
end;

procedure TNNHip<T>.upSampleNHWC(const batch, channels, h, w, stride: SizeInt; const scale: T; const input: TCUMem;
  const inOffset, inPix: SizeInt; const output: TCUMem; const outOffset, outPix: SizeInt);
begin
  check(tnh_upsample_nhwc(batch, channels, h, w, stride, S(scale), PSingle(input), inOffset, inPix, PSingle(output),
    outOffset, outPix));
end;

procedure TNNHip<T>.forwardMaxPoolNHWC(const batch, channels, h, w, outH, outW, strideX, strideY, padding,
  kernelSize: SizeInt; const input: TCUMem; const inOffset, inPix: SizeInt; const output: TCUMem;
  const outOffset, outPix: SizeInt);
begin
  check(tnh_maxpool_fwd_nhwc(batch, channels, h, w, outH, outW, strideX, strideY, padding, kernelSize,
    PSingle(input), inOffset, inPix, PSingle(output), outOffset, outPix));
end;

procedure TNNHip<T>.yoloForward(const batch, n, classes, h, w: SizeInt; const input, output: TCUMem);
begin
  check(tnh_yolo_fwd(batch, n, classes, h, w, PSingle(input), PSingle(output)));
end;

procedure TNNHip<T>.yoloForwardNHWC(const batch, n, classes, h, w: SizeInt; const input: TCUMem;
  const inOffset, inPix: SizeInt; const output: TCUMem);
begin
  check(tnh_yolo_fwd_nhwc(batch, n, classes, h, w, PSingle(input), inOffset, inPix, PSingle(output)));
end;

procedure TNNHip<T>.yoloDetections(const batch: SizeInt; const heads: array of TCUMem; const hw: array of Int64;
  const n, classes: SizeInt; const anchors: PSingle; const netW, netH, imgW, imgH: SizeInt; const thresh: T;
  const relative, letter: boolean; const capacity: SizeInt; const boxes, objectness, prob: TCUMem;
  const counts: PLongInt);
var p: array of PSingle; i: integer;
begin
  SetLength(p, Length(heads));
  for i := 0 to High(heads) do p[i] := PSingle(heads[i]);
  check(tnh_yolo_detections(batch, Length(heads), @p[0], @hw[0], n, classes, anchors, netW, netH, imgW, imgH,
    S(thresh), ord(relative), ord(letter), capacity, PSingle(boxes), PSingle(objectness), PSingle(prob), counts));
end;

procedure TNNHip<T>.yoloNmsSort(const batch, classes, capacity: SizeInt; const boxes, prob: TCUMem;
  const counts: PLongInt; const thresh: T);
begin
  check(tnh_yolo_nms_sort(batch, classes, capacity, PSingle(boxes), PSingle(prob), counts, S(thresh)));
end;

procedure TNNHip<T>.blockNormalize(const dstSize: SizeInt; const dst: TCUMem; const offset, N: SizeInt;
  const mean, variance: TCUMem; const batch: SizeInt);
begin
  check(tnh_bn_normalize(dstSize, PSingle(dst), offset, N, PSingle(mean), PSingle(variance), batch));
end;

procedure TNNHip<T>.softmaxHeadForward(const batch, F, hw, classes: SizeInt; const x, avg, weights, biases, truth,
  logits, prob, delta, error: TCUMem);
begin
  check(tnh_softmax_head_forward(batch, F, hw, classes, PSingle(x), PSingle(avg), PSingle(weights), PSingle(biases),
    PSingle(truth), PSingle(logits), PSingle(prob), PSingle(delta), PSingle(error)));
end;

procedure TNNHip<T>.softmaxHeadBackward(const batch, F, hw, classes: SizeInt; const clampAlpha: T; const delta, avg,
  weights, weightUpdates, biasUpdates, avgDelta, deltaIn: TCUMem);
begin
  check(tnh_softmax_head_backward(batch, F, hw, classes, S(clampAlpha), PSingle(delta), PSingle(avg),
    PSingle(weights), PSingle(weightUpdates), PSingle(biasUpdates), PSingle(avgDelta), PSingle(deltaIn)));
end;

procedure TNNHip<T>.bnTrainForwardMaxPool(const batch, N, h, w: SizeInt; const x, xNorm, output, mean, variance,
  rollMean, rollVar: TCUMem; const momentum: T; const scales, biases: TCUMem; const activation: longint;
  const pooled, indexes: TCUMem);
begin
  check(tnh_bn_train_forward_maxpool(batch, N, h, w, PSingle(x), PSingle(xNorm), PSingle(output), PSingle(mean),
    PSingle(variance), PSingle(rollMean), PSingle(rollVar), momentum, PSingle(scales), PSingle(biases), activation,
    PSingle(pooled), PInt64(indexes)));
end;

procedure TNNHip<T>.bnTrainForwardAvgPool(const batch, N, hw: SizeInt; const x, xNorm, output, mean, variance,
  rollMean, rollVar: TCUMem; const momentum: T; const scales, biases: TCUMem; const activation: longint;
  const avg: TCUMem);
begin
  check(tnh_bn_train_forward_avgpool(batch, N, hw, PSingle(x), PSingle(xNorm), PSingle(output), PSingle(mean),
    PSingle(variance), PSingle(rollMean), PSingle(rollVar), momentum, PSingle(scales), PSingle(biases), activation,
    PSingle(avg)));
end;

procedure TNNHip<T>.bnForwardAvgPool(const batch, N, hw: SizeInt; const x, xNorm, output, mean, variance, scales,
  biases: TCUMem; const activation: longint; const avg: TCUMem);
begin
  check(tnh_bn_forward_avgpool(batch, N, hw, PSingle(x), PSingle(xNorm), PSingle(output), PSingle(mean),
    PSingle(variance), PSingle(scales), PSingle(biases), activation, PSingle(avg)));
end;

procedure TNNHip<T>.bnForwardMaxPool(const batch, N, h, w: SizeInt; const x, xNorm, output, mean, variance,
  scales, biases: TCUMem; const activation: longint; const pooled, indexes: TCUMem);
begin
  check(tnh_bn_forward_maxpool(batch, N, h, w, PSingle(x), PSingle(xNorm), PSingle(output), PSingle(mean),
    PSingle(variance), PSingle(scales), PSingle(biases), activation, PSingle(pooled), PInt64(indexes)));
end;

procedure TNNHip<T>.bnForward(const dstSize, N, batch: SizeInt; const x, xNorm, output, mean, variance, scales,
  biases: TCUMem; const activation: longint);
begin
  check(tnh_bn_forward(dstSize, N, batch, PSingle(x), PSingle(xNorm), PSingle(output), PSingle(mean),
    PSingle(variance), PSingle(scales), PSingle(biases), activation));
end;

procedure TNNHip<T>.bnStatistics(const srcSize, dstSize, groups: SizeInt; const src: TCUMem; const offset: SizeInt;
  means, vars, rollingMeans, rollingVars: TCUMem; const momentum: T);
begin
  check(tnh_bn_statistics(srcSize, dstSize, groups, PSingle(src), offset, PSingle(means), PSingle(vars),
    PSingle(rollingMeans), PSingle(rollingVars), S(momentum)));
end;

procedure TNNHip<T>.bnBackward(const N, dstSize, groups: SizeInt; const output: TCUMem; const activation: longint;
  const xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta, variance_delta: TCUMem;
  const biases: TCUMem);
begin
  check(tnh_bn_backward(N, dstSize, groups, PSingle(output), activation, PSingle(xNorm), PSingle(x), PSingle(scales),
    PSingle(mean), PSingle(variance), PSingle(delta), PSingle(scaleUpdates), PSingle(mean_delta),
    PSingle(variance_delta), PSingle(biases)));
end;

procedure TNNHip<T>.bnBackwardMaxPool(const N, dstSize, groups, h, w: SizeInt; const poolIndexes, poolDelta,
  output: TCUMem; const activation: longint; const xNorm, x, scales, mean, variance, delta, scaleUpdates,
  mean_delta, variance_delta: TCUMem; const biases: TCUMem);
begin
  check(tnh_bn_backward_maxpool(N, dstSize, groups, h, w, PInt64(poolIndexes), PSingle(poolDelta), PSingle(output),
    activation, PSingle(xNorm), PSingle(x), PSingle(scales), PSingle(mean), PSingle(variance), PSingle(delta),
    PSingle(scaleUpdates), PSingle(mean_delta), PSingle(variance_delta), PSingle(biases)));
end;

procedure TNNHip<T>.bnBackwardAvgPool(const N, dstSize, groups: SizeInt; const avgDelta, output: TCUMem;
  const activation: longint; const xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta,
  variance_delta: TCUMem; const biases: TCUMem);
begin
  check(tnh_bn_backward_avgpool(N, dstSize, groups, PSingle(avgDelta), PSingle(output), activation, PSingle(xNorm),
    PSingle(x), PSingle(scales), PSingle(mean), PSingle(variance), PSingle(delta), PSingle(scaleUpdates),
    PSingle(mean_delta), PSingle(variance_delta), PSingle(biases)));
end;

procedure TNNHip<T>.bnBackwardScale(const N, dstSize, groups: SizeInt; const output: TCUMem;
  const activation: longint; const xNorm, scales, delta, scaleUpdates: TCUMem);
begin
  check(tnh_bn_backward_scale(N, dstSize, groups, PSingle(output), activation, PSingle(xNorm), PSingle(scales),
    PSingle(delta), PSingle(scaleUpdates)));
end;

procedure TNNHip<T>.avgPoolForward(const batch, c, h, w: SizeInt; const input, output: TCUMem);
begin
  check(tnh_avgpool_fwd(batch, c, h, w, PSingle(input), PSingle(output)));
end;

procedure TNNHip<T>.avgPoolBackward(const batch, c, h, w: SizeInt; const delta, deltaIn: TCUMem);
begin
  check(tnh_avgpool_bwd(batch, c, h, w, PSingle(delta), PSingle(deltaIn)));
end;

procedure TNNHip<T>.sgdUpdate(const N: SizeInt; const learningRate: T; const batch: SizeInt;
  const momentum, decay: T; weights, weightUpdates: TCUMem);
begin
  check(tnh_sgd_update(N, S(learningRate), batch, S(momentum), S(decay), PSingle(weights), PSingle(weightUpdates)));
end;

procedure TNNHip<T>.sgdUpdatePack(const N: SizeInt; const learningRate: T; const batch: SizeInt;
  const momentum, decay: T; weights, weightUpdates: TCUMem; const offsets, F, C, taps: array of Int64;
  const tapMajor, flipped: array of TCUMem; const nParams: SizeInt; params: TCUMem; paramUpdates: TCUMem);
var
  tp, fl: array of PSingle;
  i: SizeInt;
begin
  if Length(offsets) = 0 then begin  // no layer table: @offsets[0] would not exist
    check(tnh_sgd_update_pack(N, S(learningRate), batch, S(momentum), S(decay), PSingle(weights),
      PSingle(weightUpdates), 0, nil, nil, nil, nil, nil, nil, nParams, PSingle(params), PSingle(paramUpdates)));
    exit
  end;
  SetLength(tp, Length(tapMajor));
  SetLength(fl, Length(flipped));
  for i := 0 to High(tapMajor) do tp[i] := PSingle(tapMajor[i]);
  for i := 0 to High(flipped) do fl[i] := PSingle(flipped[i]);
  check(tnh_sgd_update_pack(N, S(learningRate), batch, S(momentum), S(decay), PSingle(weights),
    PSingle(weightUpdates), Length(offsets), @offsets[0], @F[0], @C[0], @taps[0], @tp[0], @fl[0], nParams,
    PSingle(params), PSingle(paramUpdates)));
end;

procedure TNNHip<T>.paramUpdate(const N: SizeInt; const learningRate: T; const batch: SizeInt; const momentum: T;
  params, paramUpdates: TCUMem);
begin
  check(tnh_param_update(N, S(learningRate), batch, S(momentum), PSingle(params), PSingle(paramUpdates)));
end;

procedure TNNHip<T>.gemmNTBatchReduce(const M, N, L: SizeInt; const ALPHA: T; const A: TCUMem;
  const aOffset, lda, strideA: SizeInt; const B: TCUMem; const bOffset, ldb, strideB: SizeInt; const BETA: T;
  const C: TCUMem; const cOffset, ldc, batch: SizeInt);
begin
  check(tnh_sgemm_nt_batch_reduce(M, N, L, S(ALPHA), PSingle(A), aOffset, lda, strideA, PSingle(B), bOffset, ldb,
    strideB, S(BETA), PSingle(C), cOffset, ldc, batch));
end;

procedure TNNHip<T>.convWeightGradient(const batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY,
  strideX, dilY, dilX: SizeInt; const input: TCUMem; const inBatchStride: SizeInt; const delta: TCUMem;
  const deltaBatchStride: SizeInt; const ALPHA, BETA: T; const dW: TCUMem);
begin
  check(tnh_conv2d_wgrad(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX, dilY, dilX,
    PSingle(input), inBatchStride, PSingle(delta), deltaBatchStride, S(ALPHA), S(BETA), PSingle(dW)));
end;

function TNNHip<T>.convWeightGradientPieces(const batch, c, h, w, filters, kernelH, kernelW, padH, padW,
  strideY, strideX, dilY, dilX: SizeInt; const input: TCUMem; const inBatchStride: SizeInt; const delta: TCUMem;
  const deltaBatchStride: SizeInt; const pieces: TCUMem; const piecesFloats: SizeInt): longint;
var
  n: longint;
begin
  n := 0;
  check(tnh_conv2d_wgrad_pieces(batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX, dilY,
    dilX, PSingle(input), inBatchStride, PSingle(delta), deltaBatchStride, PSingle(pieces), piecesFloats, @n));
  result := n;
end;

procedure TNNHip<T>.sgdUpdatePackPieces(const N: SizeInt; const learningRate: T; const batch: SizeInt;
  const momentum, decay: T; weights, weightUpdates: TCUMem; const offsets, F, C, taps: array of Int64;
  const tapMajor, flipped, pieces: array of TCUMem; const nPieces: array of longint; const nParams: SizeInt;
  params, paramUpdates: TCUMem);
var
  tp, fl, pc: array of PSingle;
  i: SizeInt;
begin
  if Length(offsets) = 0 then begin
    sgdUpdatePack(N, learningRate, batch, momentum, decay, weights, weightUpdates, offsets, F, C, taps, tapMajor,
      flipped, nParams, params, paramUpdates);
    exit
  end;
  SetLength(tp, Length(tapMajor));
  SetLength(fl, Length(flipped));
  SetLength(pc, Length(pieces));
  for i := 0 to High(tapMajor) do tp[i] := PSingle(tapMajor[i]);
  for i := 0 to High(flipped) do fl[i] := PSingle(flipped[i]);
  for i := 0 to High(pieces) do pc[i] := PSingle(pieces[i]);
  check(tnh_sgd_update_pack_pieces(N, S(learningRate), batch, S(momentum), S(decay), PSingle(weights),
    PSingle(weightUpdates), Length(offsets), @offsets[0], @F[0], @C[0], @taps[0], @tp[0], @fl[0], @pc[0],
    @nPieces[0], nParams, PSingle(params), PSingle(paramUpdates)));
end;

procedure TNNHip<T>.setDeterministic(const enable: boolean);
begin
  check(tnh_set_deterministic(ord(enable)));
end;

procedure TNNHip<T>.setConvAutotune(const enable: boolean; const forcedConfig: longint);
begin
  check(tnh_conv2d_set_autotune(ord(enable), forcedConfig));
end;

procedure TNNHip<T>.setSgemmAutotune(const enable: boolean; const forcedConfig: longint);
begin
  check(tnh_sgemm_set_autotune(ord(enable), forcedConfig));
end;

function TNNHip<T>.cuCount: longint;
begin
  check(tnh_cu_count(@result));
end;

end.
