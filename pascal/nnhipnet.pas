unit nnhipnet;
{ Channels-last inference forward of a whole TNNet on TNNHip.

  The per-layer forwardGPU hooks keep the reference's NCHW tensors and run
  one layer at a time (TNNet.forward, source/nnet.pas:275-317).  This unit is
  the faster alternative a USE_HIP build can take for inference: it plans
  device storage for the whole network once and then runs it with fused,
  channels-last launches:
    - activations live as [B][h][w][C] device buffers; a multi-input route
      (TConcatLayer) gets one [B][h][w][sum C] buffer and each input's
      producer writes straight into its channel slice (outOffset = channel
      offset, outPix = sum C), so the route itself launches nothing;
    - a convolution followed by a linear shortcut (TAddLayer with one input)
      that only it feeds adds the shortcut input in its epilogue
      (residual) and writes the shortcut's storage;
    - a convolution read only by an upsample stores the upsampled image
      (conv2dForwardNHWCUpsample); one read only by a yolo layer also writes
      the yolo head (conv2dForwardNHWCYolo);
    - layer 0 reads the NCHW input image (inPix = 0) and the yolo layers
      write their own NCHW output tensors (TYoloLayer.output.devData), so
      the input upload and TNNet.Detections (nnet.pas:584-680) stay as they
      are.
  3x3 weights are repacked tap-major once per plan (packConvWeights); call
  repack after the weights change (update, load).  Construct the plan after
  fuseBatchNorm (nnet.pas:268-273): batch-normalized convolutions are not
  planned.

  The Python class darknet.Network(layout="nhwc") (tensorium_amd/darknet.py)
  runs the same plan and is what the tests check against the CPU oracle. }

{$mode delphi}{$H+}

interface

uses SysUtils, ntensors, nbaselayer, nnet, nConvolutionLayer, naddlayer, nconcatlayer, nupsamplelayer,
  nMaxPoolLayer, nyololayer, nnhip;

type
  ENHWCPlan = class(Exception);

  // where a layer's output lives: pixel (b, y, x) channel k at
  // buf + offset + ((b*h + y)*w + x)*pix + k
  TNHWCSlot = record
    buf: TCUMem;
    offset, pix: SizeInt;
  end;

  // a route input that could not be written in place: copied into the
  // route buffer at channel offset `offset`
  TRouteCopy = record
    src, offset: SizeInt;
  end;

  TNHWCForward = class
  private
    hip: TNNHip<Single>;
    net: TNNet;
    batch: SizeInt;
    slot: TArray<TNHWCSlot>;
    hasSlot: TArray<boolean>;
    packed: TArray<TCUMem>;
    shortcutFused, upFused, yoloFused: TArray<boolean>;
    copies: TArray<TArray<TRouteCopy>>;
    allocated: TArray<TCUMem>;
    function routeCopy(const src, offset: SizeInt): TRouteCopy;
    function layerCount: SizeInt;
    function consumers(const i: SizeInt): TArray<SizeInt>;
    function ownerOf(const i: SizeInt): SizeInt;
    function store(const i: SizeInt): TNHWCSlot;
    function newBuffer(const floats: SizeInt): TCUMem;
    procedure planFusions;
    procedure planStorage;
    procedure scaleXY(const L: TYoloLayer);
  public
    // aNet after fuseBatchNorm; aBatch images per forward
    constructor Create(const aNet: TNNet; const aHip: TNNHip<Single>; const aBatch: SizeInt);
    destructor Destroy; override;
    // tap-major copies of the 3x3 weights (again after the weights change)
    procedure repack;
    // input: the NCHW image batch on the device; the yolo layers' outputs
    // hold the heads afterwards
    procedure forward(const input: TCUMem);
  end;

implementation

function TNHWCForward.routeCopy(const src, offset: SizeInt): TRouteCopy;
begin
  result.src := src;
  result.offset := offset
end;

function TNHWCForward.layerCount: SizeInt;
begin
  result := length(net.layers)
end;

function TNHWCForward.consumers(const i: SizeInt): TArray<SizeInt>;
var
  j, k: SizeInt;
  L: TBaseLayer;
begin
  result := nil;
  for j := i + 1 to layerCount - 1 do begin
    L := net.layers[j];
    if L is TConcatLayer then begin
      for k := 0 to high(TConcatLayer(L).inputLayers) do
        if TConcatLayer(L).inputLayers[k] = i then begin
          result := result + [j];
          break
        end
    end
    else if (j = i + 1) or ((L is TAddLayer) and (TAddLayer(L).inputLayers[0] = i)) then
      result := result + [j]
  end
end;

function TNHWCForward.ownerOf(const i: SizeInt): SizeInt;
var
  L: TBaseLayer;
begin
  L := net.layers[i];
  if (L is TConcatLayer) and (length(TConcatLayer(L).inputLayers) = 1) then
    exit(ownerOf(TConcatLayer(L).inputLayers[0]));
  if shortcutFused[i] then
    exit(i + 1);
  result := i
end;

function TNHWCForward.store(const i: SizeInt): TNHWCSlot;
var
  o: SizeInt;
begin
  o := ownerOf(i);
  if not hasSlot[o] then
    raise ENHWCPlan.CreateFmt('layer %d has no channels-last storage', [i]);
  result := slot[o]
end;

function TNHWCForward.newBuffer(const floats: SizeInt): TCUMem;
begin
  result := hip.createDeviceBuffer(floats * SizeOf(Single));
  allocated := allocated + [result]
end;

procedure TNHWCForward.planFusions;
var
  i: SizeInt;
  L, nxt: TBaseLayer;
  use: TArray<SizeInt>;
begin
  for i := 0 to layerCount - 2 do begin
    L := net.layers[i];
    if not (L is TConvolutionalLayer) then continue;
    use := consumers(i);
    if (length(use) <> 1) or (use[0] <> i + 1) then continue;
    nxt := net.layers[i + 1];
    if (nxt is TAddLayer) and (length(TAddLayer(nxt).inputLayers) = 1) and (nxt.ActivationType = acLINEAR)
      and (TAddLayer(nxt).inputLayers[0] <> i) then
      shortcutFused[i] := true
    else if i > 0 then begin
      if nxt is TUpSampleLayer then upFused[i] := true
      else if nxt is TYoloLayer then yoloFused[i] := true
    end
  end
end;

procedure TNHWCForward.planStorage;
var
  i, k, o, off, total: SizeInt;
  L: TBaseLayer;
  R: TConcatLayer;
  buf: TCUMem;
  s: TNHWCSlot;
begin
  // route buffers first: their inputs' producers write into the slices
  for i := 0 to layerCount - 1 do begin
    L := net.layers[i];
    if not (L is TConcatLayer) then continue;
    R := TConcatLayer(L);
    if length(R.inputLayers) < 2 then continue;
    total := R.outC;
    buf := newBuffer(batch * R.outH * R.outW * total);
    s.buf := buf; s.offset := 0; s.pix := total;
    slot[i] := s; hasSlot[i] := true;
    off := 0;
    for k := 0 to high(R.inputLayers) do begin
      o := ownerOf(R.inputLayers[k]);
      if not hasSlot[o] and ((net.layers[o] is TConvolutionalLayer) or (net.layers[o] is TAddLayer)
        or (net.layers[o] is TUpSampleLayer) or (net.layers[o] is TMaxPoolLayer)) then begin
        s.buf := buf; s.offset := off; s.pix := total;
        slot[o] := s; hasSlot[o] := true
      end
      else
        copies[i] := copies[i] + [routeCopy(R.inputLayers[k], off)];
      inc(off, TBaseImageLayer(net.layers[R.inputLayers[k]]).outC)
    end
  end;
  // everything else that stores an output: its own [B][h][w][C] buffer
  for i := 0 to layerCount - 1 do begin
    L := net.layers[i];
    if L is TYoloLayer then continue;  // writes its own NCHW output tensor
    if ((L is TConcatLayer) and (length(TConcatLayer(L).inputLayers) = 1)) or shortcutFused[i] or hasSlot[i]
      or upFused[i] then continue;
    // (no `with` here: TBaseLayer has a Batch field of its own)
    s.buf := newBuffer(batch * TBaseImageLayer(L).outH * TBaseImageLayer(L).outW * TBaseImageLayer(L).outC);
    s.offset := 0;
    s.pix := TBaseImageLayer(L).outC;
    slot[i] := s; hasSlot[i] := true
  end
end;

constructor TNHWCForward.Create(const aNet: TNNet; const aHip: TNNHip<Single>; const aBatch: SizeInt);
var
  i, n: SizeInt;
  L: TBaseLayer;
  C: TConvolutionalLayer;
begin
  inherited Create;
  net := aNet;
  hip := aHip;
  batch := aBatch;
  n := layerCount;
  if (n = 0) or not (net.layers[0] is TConvolutionalLayer) then
    raise ENHWCPlan.Create('a channels-last network starts with a convolution');
  for i := 0 to n - 1 do begin
    L := net.layers[i];
    if L is TConvolutionalLayer then begin
      C := TConvolutionalLayer(L);
      if C.isBatchNormalized then
        raise ENHWCPlan.CreateFmt('layer %d: call fuseBatchNorm before planning', [i]);
      if (C.Dilation <> 1) or not (C.kernelSize in [1, 3]) then
        raise ENHWCPlan.CreateFmt('layer %d: channels-last convolutions are 1x1 or 3x3, dilation 1', [i]);
      if (i = 0) and ((C.kernelSize <> 3) or (C.c > 4)) then
        raise ENHWCPlan.Create('layer 0 must be a 3x3 convolution on <= 4 channels (it reads the NCHW image)');
      if (i > 0) and (C.c mod 4 <> 0) then
        raise ENHWCPlan.CreateFmt('layer %d: channels-last convolutions need C %% 4 = 0', [i]);
    end
    else if L is TMaxPoolLayer then begin
      if TMaxPoolLayer(L).maxPoolDepth <> 0 then
        raise ENHWCPlan.CreateFmt('layer %d: maxpool_depth runs NCHW (forwardGPU)', [i])
    end
    else if not ((L is TAddLayer) or (L is TConcatLayer) or (L is TUpSampleLayer) or (L is TYoloLayer)) then
      raise ENHWCPlan.CreateFmt('layer %d (%s) has no channels-last form', [i, L.LayerTypeStr])
  end;
  setLength(slot, n);
  setLength(hasSlot, n);
  setLength(packed, n);
  setLength(shortcutFused, n);
  setLength(upFused, n);
  setLength(yoloFused, n);
  setLength(copies, n);
  planFusions;
  planStorage;
  repack
end;

destructor TNHWCForward.Destroy;
var
  i: SizeInt;
begin
  for i := 0 to high(allocated) do
    hip.freeDeviceBuffer(allocated[i]);
  inherited Destroy
end;

procedure TNHWCForward.repack;
var
  i: SizeInt;
  C: TConvolutionalLayer;
begin
  for i := 0 to layerCount - 1 do begin
    if not (net.layers[i] is TConvolutionalLayer) then continue;
    C := TConvolutionalLayer(net.layers[i]);
    if not C.weights.wasGPU() then C.weights.pushToDevice;
    if not C.biases.wasGPU() then C.biases.pushToDevice;
    if C.kernelSize = 1 then continue;  // [F][C] is tap-major already
    if not assigned(packed[i]) then
      packed[i] := newBuffer(C.weights.size());
    hip.packConvWeights(C.filters, C.c, C.kernelSize, C.kernelSize, C.weights.devData, packed[i])
  end
end;

procedure TNHWCForward.scaleXY(const L: TYoloLayer);
var
  b, a: SizeInt;
begin
  // TYoloLayer.forwardGPU's scale_x_y step (nyololayer.pas:1098-1099)
  if L.scaleXY = 1 then exit;
  for b := 0 to batch - 1 do
    for a := 0 to L.n - 1 do
      hip.fmavss(2 * L.outH * L.outW, L.output.devData, (b * L.n + a) * (L.classes + 5) * L.outH * L.outW,
        L.scaleXY, 0.5 * (1 - L.scaleXY), L.output.devData)
end;

procedure TNHWCForward.forward(const input: TCUMem);
var
  i, k: SizeInt;
  L: TBaseLayer;
  C: TConvolutionalLayer;
  src, dst, res, cs: TNHWCSlot;
  w: TCUMem;
  inPix: SizeInt;
  U: TUpSampleLayer;
  Y: TYoloLayer;
  M: TMaxPoolLayer;
  A: TAddLayer;
begin
  for i := 0 to layerCount - 1 do begin
    L := net.layers[i];
    if L is TConvolutionalLayer then begin
      C := TConvolutionalLayer(L);
      if i = 0 then begin
        src.buf := input; src.offset := 0; inPix := 0  // NCHW image
      end
      else begin
        src := store(i - 1); inPix := src.pix
      end;
      if assigned(packed[i]) then w := packed[i] else w := C.weights.devData;
      if upFused[i] then begin
        U := TUpSampleLayer(net.layers[i + 1]);
        dst := store(i + 1);
        hip.conv2dForwardNHWCUpsample(batch, C.c, C.h, C.w, C.filters, C.kernelSize, C.kernelSize, C.Padding,
          C.Padding, C.stride_y, C.stride_x, src.buf, src.offset, inPix, w, C.biases.devData,
          longint(C.ActivationType), U.stride, U.scale, dst.buf, dst.offset, dst.pix)
      end
      else if yoloFused[i] then begin
        Y := TYoloLayer(net.layers[i + 1]);
        dst := store(i);
        Y.output.setCUDA;
        hip.conv2dForwardNHWCYolo(batch, C.c, C.h, C.w, C.filters, C.kernelSize, C.kernelSize, C.Padding,
          C.Padding, C.stride_y, C.stride_x, src.buf, src.offset, inPix, w, C.biases.devData,
          longint(C.ActivationType), dst.buf, dst.offset, dst.pix, Y.n, Y.classes, Y.output.devData)
      end
      else begin
        dst := store(i);
        if shortcutFused[i] then
          res := store(TAddLayer(net.layers[i + 1]).inputLayers[0])
        else begin
          res.buf := nil; res.offset := 0; res.pix := 0
        end;
        hip.conv2dForwardNHWC(batch, C.c, C.h, C.w, C.filters, C.kernelSize, C.kernelSize, C.Padding, C.Padding,
          C.stride_y, C.stride_x, src.buf, src.offset, inPix, w, C.biases.devData, longint(C.ActivationType),
          res.buf, res.offset, res.pix, dst.buf, dst.offset, dst.pix)
      end
    end
    else if L is TAddLayer then begin
      if shortcutFused[i - 1] then continue;
      A := TAddLayer(L);
      src := store(i - 1); res := store(A.inputLayers[0]); dst := store(i);
      if (src.pix <> A.outC) or (res.pix <> A.outC) or (dst.pix <> A.outC) then
        raise ENHWCPlan.CreateFmt('layer %d: an unfused shortcut needs whole buffers', [i]);
      hip.addvv(batch * A.outputs, src.buf, 0, 1, res.buf, 0, 1, dst.buf, 0, 1);
      hip.ActivateArray(batch * A.outputs, dst.buf, 0, longint(A.ActivationType))
    end
    else if L is TConcatLayer then begin
      if length(TConcatLayer(L).inputLayers) < 2 then continue;  // an alias of its input
      dst := store(i);
      for k := 0 to high(copies[i]) do begin
        cs := store(copies[i][k].src);
        hip.copyChannels(batch * TConcatLayer(L).outH * TConcatLayer(L).outW,
          TBaseImageLayer(net.layers[copies[i][k].src]).outC, cs.buf, cs.offset, cs.pix, dst.buf,
          dst.offset + copies[i][k].offset, dst.pix)
      end
    end
    else if L is TUpSampleLayer then begin
      if upFused[i - 1] then continue;
      U := TUpSampleLayer(L);
      src := store(i - 1); dst := store(i);
      hip.upSampleNHWC(batch, U.c, U.h, U.w, U.stride, U.scale, src.buf, src.offset, src.pix, dst.buf, dst.offset,
        dst.pix)
    end
    else if L is TMaxPoolLayer then begin
      M := TMaxPoolLayer(L);
      src := store(i - 1); dst := store(i);
      hip.forwardMaxPoolNHWC(batch, M.c, M.h, M.w, M.outH, M.outW, M.stride_x, M.stride_y, M.Padding, M.kernelSize,
        src.buf, src.offset, src.pix, dst.buf, dst.offset, dst.pix)
    end
    else if L is TYoloLayer then begin
      Y := TYoloLayer(L);
      if not yoloFused[i - 1] then begin
        src := store(i - 1);
        Y.output.setCUDA;
        hip.yoloForwardNHWC(batch, Y.n, Y.classes, Y.h, Y.w, src.buf, src.offset, src.pix, Y.output.devData)
      end;
      scaleXY(Y)
    end
  end
end;

end.
