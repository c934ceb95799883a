"""Seeded synthetic models in the `.engine` format.

The YOLOv8 graph emitted here follows the node pattern of an Ultralytics
static ONNX export (opset 18, BN folded into the conv bias) after the
reference converter's rewrites (pdefa/tools/onnx_to_engine.py:200-268 turns
Split into Slice nodes with constant starts/ends/axes; :580-590 appends the
Transpose perm as a weight; constants become F32 weights):

  Conv block      Conv(k, s, p=k//2, bias) -> Sigmoid -> Mul
  C2f             Conv1x1 -> Slice x2 -> [Conv3x3 -> Conv3x3 (+ Add)] x n
                  -> Concat(axis 1) -> Conv1x1
  SPPF            Conv1x1 -> MaxPool(k5 s1 p2) x3 -> Concat -> Conv1x1
  FPN/PAN         Resize(scales [1,1,2,2], nearest) -> Concat
  Detect level    cv2: Conv3x3 -> Conv3x3 -> Conv1x1(64)
                  cv3: Conv3x3 -> Conv3x3 -> Conv1x1(nc)
                  -> Concat(axis 1) -> Reshape [1, 64+nc, -1]
  head            Concat(axis 2) -> Slice(64 | nc)
                  box: Reshape [1,4,16,A] -> Transpose [0,2,1,3] -> Softmax(1)
                       -> Conv1x1(16->1, w = arange(16)) -> Reshape [1,4,A]
                       -> Slice(2 | 2) -> anchors - lt, anchors + rb
                       -> (x1y1 + x2y2) / 2, x2y2 - x1y1 -> Concat -> Mul(strides)
                  cls: Sigmoid
                  out: Concat(axis 1) -> [1, 4+nc, A]

Architecture constants follow the public YOLOv8 model definition: backbone
Conv(64,3,2) Conv(128,3,2) C2f(128)x3 Conv(256,3,2) C2f(256)x6 Conv(512,3,2)
C2f(512)x6 Conv(1024,3,2) C2f(1024)x3 SPPF(1024); head Upsample Concat(P4)
C2f(512)x3 Upsample Concat(P3) C2f(256)x3 Conv(256,3,2) Concat C2f(512)x3
Conv(512,3,2) Concat C2f(1024)x3 Detect; widths scaled by the width multiple
and capped at max_channels, repeats by the depth multiple.
"""
from __future__ import annotations

import math
from typing import List, Optional, Tuple

import numpy as np

from .engine_format import OP, EngineModel, Node, TensorInfo, write_engine

SCALES = {
    # depth multiple, width multiple, max channels
    "n": (0.33, 0.25, 1024),
    "s": (0.33, 0.50, 1024),
    "m": (0.67, 0.75, 768),
    "l": (1.00, 1.00, 512),
    "x": (1.00, 1.25, 512),
}


class GraphBuilder:
    """Emits engine nodes the way the reference converter numbers them:
    weights as -1000-w, the graph input as -1, intermediates from 0 upward."""

    def __init__(self) -> None:
        self.weights: List[np.ndarray] = []
        self.wnames: List[str] = []
        self.nodes: List[Node] = []
        self.n_inter = 0

    def const(self, name: str, arr) -> int:
        a = np.asarray(arr)
        # int64 / int32 constants keep their type (written as I64 / I32)
        a = a if a.dtype in (np.int64, np.int32) else a.astype(np.float32)
        self.weights.append(np.ascontiguousarray(a))
        self.wnames.append(name)
        return -1000 - (len(self.weights) - 1)

    def node(self, op: str, name: str, inputs: List[int], n_out: int = 1, **params):
        outs = list(range(self.n_inter, self.n_inter + n_out))
        self.n_inter += n_out
        self.nodes.append(Node(OP[op], name, list(inputs), outs, params))
        return outs[0] if n_out == 1 else outs

    def model(self, in_shape, out_shape, outputs: List[int]) -> EngineModel:
        """out_shape: the output's shape, or with several outputs a list of
        shapes (the second and later ones may be None)."""
        shapes = out_shape if len(outputs) > 1 else [out_shape]
        infos = [TensorInfo(f"output{i}", list(sh) if sh is not None else []) for i, sh in enumerate(shapes)]
        infos += [TensorInfo(f"output{i}", []) for i in range(len(infos), len(outputs))]
        return EngineModel(self.weights, self.wnames, self.nodes, [-1], outputs,
                           [TensorInfo("images", list(in_shape))], infos)


def make_divisible(x: float, d: int = 8) -> int:
    return int(math.ceil(x / d) * d)


def kaiming_uniform(rng: np.random.Generator, shape) -> np.ndarray:
    fan_in = int(np.prod(shape[1:]))
    bound = math.sqrt(6.0 / fan_in)
    return rng.uniform(-bound, bound, size=shape).astype(np.float32)


class _Yolo:
    def __init__(self, b: GraphBuilder, rng: np.random.Generator, cls_bias: float):
        self.b, self.rng, self.cls_bias = b, rng, cls_bias

    def conv_raw(self, x, cin, cout, k, s, name, bias_value=None, gain=1.0):
        w = kaiming_uniform(self.rng, (cout, cin, k, k)) * np.float32(gain)
        if bias_value is None:
            bias = self.rng.uniform(-0.1, 0.1, size=cout).astype(np.float32)
        else:
            bias = np.full(cout, bias_value, np.float32)
        wi = self.b.const(f"{name}.weight", w)
        bi = self.b.const(f"{name}.bias", bias)
        p = k // 2
        return self.b.node("Conv", f"/{name}/Conv", [x, wi, bi], stride_h=s, stride_w=s,
                           pad_h=p, pad_w=p, dil_h=1, dil_w=1, groups=1)

    def conv(self, x, cin, cout, k, s, name):
        y = self.conv_raw(x, cin, cout, k, s, f"{name}/conv")
        sg = self.b.node("Sigmoid", f"/{name}/act/Sigmoid", [y])
        return self.b.node("Mul", f"/{name}/act/Mul", [y, sg])

    def slice(self, x, start, end, axis, name):
        s = self.b.const(f"{name}_start::const", [start])
        e = self.b.const(f"{name}_end::const", [end])
        a = self.b.const(f"{name}_axes::const", [axis])
        return self.b.node("Slice", name, [x, s, e, a])

    def c2f(self, x, cin, cout, n, shortcut, name):
        c = int(cout * 0.5)
        y = self.conv(x, cin, 2 * c, 1, 1, f"{name}/cv1")
        parts = [self.slice(y, 0, c, 1, f"/{name}/Split_slice_0"),
                 self.slice(y, c, 2 * c, 1, f"/{name}/Split_slice_1")]
        for i in range(n):
            h = self.conv(parts[-1], c, c, 3, 1, f"{name}/m.{i}/cv1")
            h = self.conv(h, c, c, 3, 1, f"{name}/m.{i}/cv2")
            if shortcut:
                h = self.b.node("Add", f"/{name}/m.{i}/add", [parts[-1], h])
            parts.append(h)
        cat = self.b.node("Concat", f"/{name}/Concat", parts, axis=1)
        return self.conv(cat, (2 + n) * c, cout, 1, 1, f"{name}/cv2")

    def sppf(self, x, cin, cout, name):
        c_ = cin // 2
        y = self.conv(x, cin, c_, 1, 1, f"{name}/cv1")
        ys = [y]
        for i in range(3):
            ys.append(self.b.node("MaxPool", f"/{name}/m/MaxPool_{i}", [ys[-1]], kernel_h=5,
                                  kernel_w=5, stride_h=1, stride_w=1, pad_h=2, pad_w=2))
        cat = self.b.node("Concat", f"/{name}/Concat", ys, axis=1)
        return self.conv(cat, 4 * c_, cout, 1, 1, f"{name}/cv2")

    def upsample(self, x, name):
        sc = self.b.const(f"{name}/scales::const", [1.0, 1.0, 2.0, 2.0])
        return self.b.node("Resize", f"/{name}/Resize", [x, sc])


# Class-head gain and bias per scale.  The random-weight class logits of
# the unscaled head are tightly clustered (spread ~0.01), so the gain spreads
# them out: at 300 the best-class scores of the synthetic images are sparse
# enough above 0.25 that thresholds with no score within 1e-2 exist (a parity
# test's detection lists then cannot flip on a tolerance-sized difference);
# the bias puts 15 to 150 candidates above 0.25 on each synthetic image (the
# spread of the logits grows with model width, hence a lower bias for wider
# models).
CLS_GAIN = 300.0
CLS_BIAS = {"n": -50.0, "s": -50.0, "m": -66.0, "l": -66.0, "x": -66.0}


def build_yolov8(scale: str = "n", seed: int = 0, nc: int = 80, imgsz=640,
                 cls_bias: Optional[float] = None, cls_gain: float = CLS_GAIN) -> EngineModel:
    """YOLOv8{scale} detection graph with seeded random weights (BN folded),
    for square imgsz x imgsz inputs or, with imgsz = (h, w), h x w inputs
    (both multiples of 32).

    The class head's last conv has its Kaiming weights scaled by cls_gain and
    a constant bias cls_bias (default CLS_BIAS[scale]), so that a random-weight
    model still yields candidates above 0.25 on a synthetic image (the
    unscaled head scores every anchor near sigmoid(cls_bias))."""
    if cls_bias is None:
        cls_bias = CLS_BIAS[scale]
    ih, iw = (imgsz, imgsz) if isinstance(imgsz, int) else (int(imgsz[0]), int(imgsz[1]))
    depth, width, max_ch = SCALES[scale]
    ch = lambda c: make_divisible(min(c, max_ch) * width, 8)
    rep = lambda n: max(round(n * depth), 1)
    rng = np.random.default_rng(seed)
    b = GraphBuilder()
    y = _Yolo(b, rng, cls_bias)
    x = -1
    c0, c1, c2, c3, c4 = ch(64), ch(128), ch(256), ch(512), ch(1024)
    x = y.conv(x, 3, c0, 3, 2, "model.0")
    x = y.conv(x, c0, c1, 3, 2, "model.1")
    x = y.c2f(x, c1, c1, rep(3), True, "model.2")
    x = y.conv(x, c1, c2, 3, 2, "model.3")
    p3 = y.c2f(x, c2, c2, rep(6), True, "model.4")
    x = y.conv(p3, c2, c3, 3, 2, "model.5")
    p4 = y.c2f(x, c3, c3, rep(6), True, "model.6")
    x = y.conv(p4, c3, c4, 3, 2, "model.7")
    x = y.c2f(x, c4, c4, rep(3), True, "model.8")
    p5 = y.sppf(x, c4, c4, "model.9")
    x = y.upsample(p5, "model.10")
    x = b.node("Concat", "/model.11/Concat", [x, p4], axis=1)
    h12 = y.c2f(x, c4 + c3, c3, rep(3), False, "model.12")
    x = y.upsample(h12, "model.13")
    x = b.node("Concat", "/model.14/Concat", [x, p3], axis=1)
    h15 = y.c2f(x, c3 + c2, c2, rep(3), False, "model.15")
    x = y.conv(h15, c2, c2, 3, 2, "model.16")
    x = b.node("Concat", "/model.17/Concat", [x, h12], axis=1)
    h18 = y.c2f(x, c2 + c3, c3, rep(3), False, "model.18")
    x = y.conv(h18, c3, c3, 3, 2, "model.19")
    x = b.node("Concat", "/model.20/Concat", [x, p5], axis=1)
    h21 = y.c2f(x, c3 + c4, c4, rep(3), False, "model.21")

    # Detect head (reg_max 16)
    feats = [(h15, c2, 8), (h18, c3, 16), (h21, c4, 32)]
    reg = 16
    no = nc + 4 * reg
    cb = max(16, c2 // 4, 4 * reg)
    cc = max(c2, min(nc, 100))
    flat = []
    anchors, strides = [], []
    for i, (f, cin, s) in enumerate(feats):
        n = f"model.22"
        a = y.conv(f, cin, cb, 3, 1, f"{n}/cv2.{i}/cv2.{i}.0")
        a = y.conv(a, cb, cb, 3, 1, f"{n}/cv2.{i}/cv2.{i}.1")
        a = y.conv_raw(a, cb, 4 * reg, 1, 1, f"{n}/cv2.{i}/cv2.{i}.2", bias_value=1.0)
        c = y.conv(f, cin, cc, 3, 1, f"{n}/cv3.{i}/cv3.{i}.0")
        c = y.conv(c, cc, cc, 3, 1, f"{n}/cv3.{i}/cv3.{i}.1")
        c = y.conv_raw(c, cc, nc, 1, 1, f"{n}/cv3.{i}/cv3.{i}.2", bias_value=cls_bias, gain=cls_gain)
        cat = b.node("Concat", f"/{n}/Concat_{i}", [a, c], axis=1)
        shp = b.const(f"/{n}/Reshape_{i}/shape::const", [1, no, -1])
        flat.append(b.node("Reshape", f"/{n}/Reshape_{i}", [cat, shp]))
        fh, fw = ih // s, iw // s
        gy, gx = np.meshgrid(np.arange(fh, dtype=np.float32) + 0.5, np.arange(fw, dtype=np.float32) + 0.5,
                             indexing="ij")
        anchors.append(np.stack([gx.ravel(), gy.ravel()], 0))
        strides.append(np.full(fh * fw, s, np.float32))
    n_anchor = sum(a.shape[1] for a in anchors)
    xcat = b.node("Concat", "/model.22/Concat_3", flat, axis=2)
    box = y.slice(xcat, 0, 4 * reg, 1, "/model.22/Split_slice_0")
    cls = y.slice(xcat, 4 * reg, no, 1, "/model.22/Split_slice_1")
    shp = b.const("/model.22/dfl/Reshape/shape::const", [1, 4, reg, n_anchor])
    t = b.node("Reshape", "/model.22/dfl/Reshape", [box, shp])
    perm = b.const("/model.22/dfl/Transpose::perm", [0, 2, 1, 3])
    t = b.node("Transpose", "/model.22/dfl/Transpose", [t, perm])
    t = b.node("Softmax", "/model.22/dfl/Softmax", [t], axis=1)
    dflw = b.const("model.22.dfl.conv.weight",
                   np.arange(reg, dtype=np.float32).reshape(1, reg, 1, 1))
    t = b.node("Conv", "/model.22/dfl/conv/Conv", [t, dflw], stride_h=1, stride_w=1,
               pad_h=0, pad_w=0, dil_h=1, dil_w=1, groups=1)
    shp = b.const("/model.22/dfl/Reshape_1/shape::const", [1, 4, n_anchor])
    dist = b.node("Reshape", "/model.22/dfl/Reshape_1", [t, shp])
    lt = y.slice(dist, 0, 2, 1, "/model.22/Split_1_slice_0")
    rb = y.slice(dist, 2, 4, 1, "/model.22/Split_1_slice_1")
    anc = b.const("/model.22/anchors::const", np.concatenate(anchors, 1)[None])
    x1y1 = b.node("Sub", "/model.22/Sub", [anc, lt])
    x2y2 = b.node("Add", "/model.22/Add", [anc, rb])
    ssum = b.node("Add", "/model.22/Add_1", [x1y1, x2y2])
    two = b.const("/model.22/Constant_two::const", np.array(2.0, np.float32))
    cxy = b.node("Div", "/model.22/Div", [ssum, two])
    wh = b.node("Sub", "/model.22/Sub_1", [x2y2, x1y1])
    dbox = b.node("Concat", "/model.22/Concat_4", [cxy, wh], axis=1)
    strd = b.const("/model.22/strides::const", np.concatenate(strides)[None])
    dbox = b.node("Mul", "/model.22/Mul_2", [dbox, strd])
    sig = b.node("Sigmoid", "/model.22/Sigmoid", [cls])
    out = b.node("Concat", "/model.22/Concat_5", [dbox, sig], axis=1)
    return b.model([1, 3, ih, iw], [1, 4 + nc, n_anchor], [out])


def build_single_conv(cin: int, cout: int, k: int, stride: int, hw: int, seed: int = 7,
                      silu: bool = True, groups: int = 1, act: Optional[str] = None,
                      leaky_slope: float = 0.1, centered: bool = False) -> Tuple[EngineModel, np.ndarray]:
    """One Conv2d(k, stride, pad k//2, groups) + bias (+ SiLU as Sigmoid*Mul)
    graph.

    act: instead of the SiLU, one single-consumer activation node after the
    conv ("Relu", "LeakyRelu" with leaky_slope, "Sigmoid" or "Tanh"), which
    the reference session fuses into the conv (session_fusion.inc:85-107).
    centered: the input is U[-1,1) instead of U[0,1) (pre-activations of
    both signs).

    Returns the model and its seeded input x of shape [1,cin,hw,hw].
    Seed stream: x, then W [cout, cin/groups, k, k] (Kaiming-uniform, bound
    sqrt(6/fan_in)), then b ~ U[-0.1, 0.1]."""
    rng = np.random.default_rng(seed)
    x = rng.random((1, cin, hw, hw), dtype=np.float32)
    if centered:
        x = (x * np.float32(2.0) - np.float32(1.0)).astype(np.float32)
    w = kaiming_uniform(rng, (cout, cin // groups, k, k))
    bias = rng.uniform(-0.1, 0.1, size=cout).astype(np.float32)
    b = GraphBuilder()
    wi, bi = b.const("conv.weight", w), b.const("conv.bias", bias)
    p = k // 2
    y = b.node("Conv", "/conv/Conv", [-1, wi, bi], stride_h=stride, stride_w=stride,
               pad_h=p, pad_w=p, dil_h=1, dil_w=1, groups=groups)
    if act is not None:
        params = {"leaky_slope": leaky_slope} if act == "LeakyRelu" else {}
        y = b.node(act, f"/act/{act}", [y], **params)
    elif silu:
        sg = b.node("Sigmoid", "/act/Sigmoid", [y])
        y = b.node("Mul", "/act/Mul", [y, sg])
    ho = (hw + 2 * p - k) // stride + 1
    return b.model([1, cin, hw, hw], [1, cout, ho, ho], [y]), x


def build_scdown(cin: int, cout: int, hw: int, n: int = 1, seed: int = 11) -> Tuple[EngineModel, np.ndarray]:
    """YOLOv10's SCDown block: a 1x1 Conv-SiLU to cout channels, then a 3x3
    stride-2 depthwise Conv (groups = cout, no activation), and a grouped 3x3
    Conv-SiLU (groups = cout / 8) whose output is added to the depthwise one.
    Returns the model and its seeded input x ~ U[0,1) of shape [n,cin,hw,hw]."""
    rng = np.random.default_rng(seed)
    x = rng.random((n, cin, hw, hw), dtype=np.float32)
    b = GraphBuilder()

    def conv(name, src, ci, co, k, stride, groups, silu):
        w = b.const(name + ".weight", kaiming_uniform(rng, (co, ci // groups, k, k)))
        bias = b.const(name + ".bias", rng.uniform(-0.1, 0.1, size=co).astype(np.float32))
        y = b.node("Conv", f"/{name}/conv/Conv", [src, w, bias], stride_h=stride, stride_w=stride, pad_h=k // 2,
                   pad_w=k // 2, dil_h=1, dil_w=1, groups=groups)
        if silu:
            y = b.node("Mul", f"/{name}/act/Mul", [y, b.node("Sigmoid", f"/{name}/act/Sigmoid", [y])])
        return y

    y1 = conv("cv1", -1, cin, cout, 1, 1, 1, True)
    y2 = conv("cv2", y1, cout, cout, 3, 2, cout, False)
    y3 = conv("cv3", y2, cout, cout, 3, 1, cout // 8, True)
    out = b.node("Add", "/add/Add", [y2, y3])
    ho = (hw - 1) // 2 + 1
    return b.model([n, cin, hw, hw], [n, cout, ho, ho], [out]), x


def build_topk_head(anchors: int = 8400, nc: int = 80, k: int = 300, seed: int = 9,
                    k_dtype=np.int64) -> Tuple[EngineModel, np.ndarray]:
    """A YOLOv10-style selection of the best anchors from a [1, 4 + nc, A]
    head: Transpose to [1, A, 4 + nc], Slice boxes [1, A, 4] and scores
    [1, A, nc], TopK(k, axis 1) of the scores (values and indices), the
    indices of the first four classes gather the boxes (GatherElements,
    axis 1), and Concat(boxes, values of those classes) -> [1, k, 8]; the
    indices [1, k, nc] are a second (I32) output.  k is an int64 constant.
    Returns the model and a seeded head input (scores distinct)."""
    rng = np.random.default_rng(seed)
    x = np.empty((1, 4 + nc, anchors), np.float32)
    x[0, :4] = rng.uniform(0, 640, (4, anchors)).astype(np.float32)
    x[0, 4:] = rng.permutation(nc * anchors).reshape(nc, anchors).astype(np.float32) / np.float32(nc * anchors)
    b = GraphBuilder()
    perm = b.const("/head/perm", np.array([0, 2, 1], np.float32))
    t = b.node("Transpose", "/head/Transpose", [-1, perm])
    def sl(name, src, start, end):
        return b.node("Slice", name, [src, b.const(name + "/starts", np.array([start], np.float32)),
                                      b.const(name + "/ends", np.array([end], np.float32)),
                                      b.const(name + "/axes", np.array([2], np.float32))])
    boxes = sl("/head/boxes", t, 0, 4)
    scores = sl("/head/scores", t, 4, 4 + nc)
    kk = b.const("/head/k", np.array([k], k_dtype))
    vals, idx = b.node("TopK", "/head/TopK", [scores, kk], n_out=2, axis=1)
    idx4 = sl("/head/idx4", idx, 0, 4)
    got = b.node("GatherElements", "/head/GatherElements", [boxes, idx4], axis=1)
    v4 = sl("/head/vals4", vals, 0, 4)
    out = b.node("Concat", "/head/Concat", [got, v4], axis=2)
    return b.model([1, 4 + nc, anchors], [[1, k, 8], [1, k, nc]], [out, idx]), x


def build_topk_gather(shape, axis: int, k: int, gather_idx=None, seed: int = 4) -> Tuple[EngineModel, np.ndarray]:
    """TopK(k, axis) of a seeded input with distinct values (values and
    indices as outputs 0 and 1) and, with `gather_idx` (an int64 array of
    the input's rank), GatherElements(input, gather_idx constant, axis) as
    output 2.  Returns the model and the input."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    x = (rng.permutation(n).astype(np.float32) / np.float32(n) - np.float32(0.5)).reshape(shape)
    b = GraphBuilder()
    vals, idx = b.node("TopK", "/t/TopK", [-1, b.const("/t/k", np.array([k], np.int64))], n_out=2, axis=axis)
    outs = [vals, idx]
    if gather_idx is not None:
        outs.append(b.node("GatherElements", "/t/GatherElements",
                           [-1, b.const("/t/idx", np.asarray(gather_idx, np.int64))], axis=axis))
    return b.model(list(shape), [None] * len(outs), outs), x


def build_eltwise_chain(n: int, c: int, h: int, w: int, seed: int = 6) -> Tuple[EngineModel, np.ndarray]:
    """A chain of elementwise nodes over an [n, c, h, w] input: Add of a
    per-channel constant, Mul by a per-pixel constant, Sub of a scalar, Div
    by a full-shape constant, then Sigmoid, Relu, LeakyRelu (slope 0.1) and
    Tanh, each node feeding the next (broadcast along every kind of dim)."""
    rng = np.random.default_rng(seed)
    b = GraphBuilder()
    pc = b.const("per_channel", rng.uniform(-1, 1, (1, c, 1, 1)))
    pp = b.const("per_pixel", rng.uniform(0.5, 1.5, (1, 1, h, w)))
    sc = b.const("scalar", rng.uniform(-1, 1, (1,)))
    full = b.const("full", rng.uniform(0.5, 2.0, (1, c, h, w)))
    y = b.node("Add", "/add", [-1, pc])
    y = b.node("Mul", "/mul", [y, pp])
    y = b.node("Sub", "/sub", [y, sc])
    y = b.node("Div", "/div", [y, full])
    y = b.node("Sigmoid", "/sigmoid", [y])
    y = b.node("Sub", "/center", [y, b.const("half", [0.5])])
    y = b.node("Relu", "/relu", [y])
    y = b.node("LeakyRelu", "/leaky", [b.node("Sub", "/shift", [y, b.const("q", [0.25])])], leaky_slope=0.1)
    y = b.node("Tanh", "/tanh", [y])
    x = rng.uniform(-3, 3, (n, c, h, w)).astype(np.float32)
    return b.model([n, c, h, w], [n, c, h, w], [y]), x


def build_pool_chain(n: int, c: int, h: int, w: int, k: int, seed: int = 5) -> Tuple[EngineModel, np.ndarray]:
    """SPPF's pooling part on its own: three chained MaxPool(k, stride 1,
    pad k//2) and the channel Concat of the input and the three results.
    Returns the model and its seeded input x ~ N(0,1) of shape [n,c,h,w]."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, c, h, w), dtype=np.float32)
    b = GraphBuilder()
    ys = [-1]
    for i in range(3):
        ys.append(b.node("MaxPool", f"/m/MaxPool_{i}", [ys[-1]], kernel_h=k, kernel_w=k, stride_h=1, stride_w=1,
                         pad_h=k // 2, pad_w=k // 2))
    cat = b.node("Concat", "/Concat", ys, axis=1)
    return b.model([n, c, h, w], [n, 4 * c, h, w], [cat]), x


def build_sppf(n: int, c: int, h: int, w: int, k: int = 5, seed: int = 8) -> Tuple[EngineModel, np.ndarray]:
    """The YOLOv8 SPPF block on its own (Conv1x1 -> three chained
    MaxPool(k, stride 1, pad k//2) -> Concat of the four -> Conv1x1, both
    convs with SiLU): the pools then run over channels-last conv outputs, as
    in the network.  Returns the model and a seeded input ~ U[0, 1)."""
    rng = np.random.default_rng(seed)
    b = GraphBuilder()
    y = _Yolo(b, rng, 0.0).sppf(-1, c, c, "sppf")
    x = rng.uniform(0.0, 1.0, (n, c, h, w)).astype(np.float32)
    return b.model([n, c, h, w], [n, c, h, w], [y]), x


def build_conv3x3_epilogue(cin: int, cout: int, hw: int, mode: str, side: int = 3,
                           seed: int = 21) -> Tuple[EngineModel, np.ndarray]:
    """A 3x3 stride-1 conv (+ SiLU) whose output either takes a residual or
    lands inside a concat, for the output paths of the conv epilogues.

    mode "add": Add(Conv1x1(x, cin->cout), Conv3x3(x, cin->cout)); the Add
    becomes the 3x3 conv's residual.  mode "concat": Concat(Conv1x1(x,
    cin->side), Conv3x3(x, cin->cout)) on channels; the 3x3 conv writes at
    channel offset `side` of the (channels-last) concat buffer.  Either
    result feeds a final Conv1x1 to 8 channels, the graph output, so that
    the 3x3 conv's output stays an inner channels-last tensor.  Returns the
    model and a seeded input ~ U[0, 1) of shape [1, cin, hw, hw]."""
    rng = np.random.default_rng(seed)
    b = GraphBuilder()
    yb = _Yolo(b, rng, 0.0)
    if mode == "add":
        a = yb.conv(-1, cin, cout, 1, 1, "side")
        c = yb.conv(-1, cin, cout, 3, 1, "main")
        out = b.node("Add", "/add", [a, c])
        oc = cout
    elif mode == "concat":
        a = yb.conv(-1, cin, side, 1, 1, "side")
        c = yb.conv(-1, cin, cout, 3, 1, "main")
        out = b.node("Concat", "/cat", [a, c], axis=1)
        oc = side + cout
    else:
        raise ValueError(mode)
    out = yb.conv(out, oc, 8, 1, 1, "head")
    x = rng.uniform(0.0, 1.0, (1, cin, hw, hw)).astype(np.float32)
    return b.model([1, cin, hw, hw], [1, 8, hw, hw], [out]), x


def build_tiny(seed: int = 3) -> EngineModel:
    """A small stand-in for the reference tests' tiny.engine (a 64x64
    Conv -> AvgPool -> Linear to 4 outputs, pdefa/tests/README.md:13-39, not
    shipped): one Conv(3 -> 4, 64x64 kernel, no padding) + bias over the
    whole [1,3,64,64] image, i.e. a linear map to 4 values, then Reshape to
    [1,4].  Same input/output shapes, built from ops on this path."""
    rng = np.random.default_rng(seed)
    w = kaiming_uniform(rng, (4, 3, 64, 64))
    bias = rng.uniform(-0.1, 0.1, size=4).astype(np.float32)
    b = GraphBuilder()
    wi, bi = b.const("fc.weight", w), b.const("fc.bias", bias)
    y = b.node("Conv", "/fc/Conv", [-1, wi, bi], stride_h=1, stride_w=1, pad_h=0, pad_w=0, dil_h=1, dil_w=1,
               groups=1)
    shp = b.const("/fc/Reshape/shape::const", [1, 4])
    y = b.node("Reshape", "/fc/Reshape", [y, shp])
    return b.model([1, 3, 64, 64], [1, 4], [y])


# Source image sizes for the batch-8 workload: aspect cycle 16:9, 4:3, 1:1.
ASPECT_SIZES = [(1280, 720), (1024, 768), (800, 800)]


def synth_image(seed: int, w: int = 1280, h: int = 720) -> np.ndarray:
    """A synthetic RGB8 image, pixels ~ U[0, 255], shape [h, w, 3] uint8."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, 256, size=(h, w, 3), dtype=np.uint8)


def letterbox(img: np.ndarray, target_w: int = 640, target_h: int = 640,
              scale: float = 1.0 / 255.0, pad_value: float = 114.0 / 255.0):
    """Bilinear letterbox to an NCHW float32 [1,3,th,tw] tensor.

    Restates imageloader/src/preprocess.cpp:15-144: ratio = min(tw/w, th/h),
    scaled size = clamp(round(src*ratio), 1, target), centred pads (integer
    halves), sample positions s = d * (1/ratio) truncated to int, x0/y0
    clamped to src-2, bilinear weights with the scale folded into the row
    weights, and the pad value written raw (not scaled).  The blend rounds as
    the reference's own build computes it (imageloader/CMakeLists.txt:41
    compiles with -mfma and GCC contracts (p00 w0 + p10 w1) into
    fma(p00, w0, p10 w1), and so on).
    Returns (tensor, meta dict)."""
    h, w = img.shape[:2]
    ch = 1 if img.ndim == 2 else img.shape[2]
    if img.ndim == 2:
        img = img[:, :, None]
    ratio = np.float32(min(np.float32(target_w) / np.float32(w),
                           np.float32(target_h) / np.float32(h)))
    # std::round rounds halves away from zero (numpy's round is half-to-even)
    sw = int(np.clip(int(np.floor(np.float32(w) * ratio + np.float32(0.5))), 1, target_w))
    sh = int(np.clip(int(np.floor(np.float32(h) * ratio + np.float32(0.5))), 1, target_h))
    px, py = (target_w - sw) // 2, (target_h - sh) // 2
    out = np.full((3, target_h, target_w), np.float32(pad_value), np.float32)
    inv = np.float32(1.0) / ratio
    sx = np.arange(sw, dtype=np.float32) * inv
    x0 = sx.astype(np.int64)
    if w > 1:
        x0 = np.minimum(x0, w - 2)
    x1 = np.where(x0 + 1 < w, x0 + 1, x0)
    fx = (sx - x0.astype(np.float32)).astype(np.float32)
    sy = np.arange(sh, dtype=np.float32) * inv
    y0 = sy.astype(np.int64)
    if h > 1:
        y0 = np.minimum(y0, h - 2)
    y1 = np.where(y0 + 1 < h, y0 + 1, y0)
    fy = (sy - y0.astype(np.float32)).astype(np.float32)
    ns = np.float32(scale)
    wy0 = ((np.float32(1) - fy) * ns)[:, None]
    wy1 = (fy * ns)[:, None]
    w0 = (np.float32(1) - fx)[None, :]
    w1 = fx[None, :]
    src = img.astype(np.float32)
    chans = [0, 0, 0] if ch == 1 else [0, 1, 2]

    def fma(a, b, c):
        # one rounding of a * b + c: the exact value fits the 64-bit
        # significand of long double for these operands (8-bit pixels and
        # float32 weights)
        return (a.astype(np.longdouble) * b + c).astype(np.float32)

    for c in range(3):
        p = src[:, :, chans[c]]
        # the reference's GCC build computes a * b + c * d as fma(a, b, c * d)
        r0 = fma(p[y0][:, x0], w0, (p[y0][:, x1] * w1).astype(np.float32))
        r1 = fma(p[y1][:, x0], w0, (p[y1][:, x1] * w1).astype(np.float32))
        out[c, py:py + sh, px:px + sw] = fma(r0, wy0, (r1 * wy1).astype(np.float32))
    meta = dict(target_w=target_w, target_h=target_h, orig_w=w, orig_h=h, pad_x=px,
                pad_y=py, scaled_w=sw, scaled_h=sh, ratio=float(ratio))
    return out[None], meta


def yolo_inputs(batch: int, imgsz=640) -> Tuple[np.ndarray, list]:
    """Letterboxed synthetic inputs: image i has seed i and the i-th size of the
    16:9 / 4:3 / 1:1 cycle; pad 114/255, scale 1/255.  imgsz: the square side,
    or (h, w)."""
    th, tw = (imgsz, imgsz) if isinstance(imgsz, int) else (int(imgsz[0]), int(imgsz[1]))
    xs, metas = [], []
    for i in range(batch):
        w, h = ASPECT_SIZES[i % len(ASPECT_SIZES)]
        t, m = letterbox(synth_image(i, w, h), tw, th)
        xs.append(t)
        metas.append(m)
    return np.concatenate(xs, 0), metas


def save(model: EngineModel, path: str) -> str:
    write_engine(path, model)
    return path
