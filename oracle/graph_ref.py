"""CPU oracle for the conv/GEMM hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker; the product never routes through
it.

A float64 numpy restatement of what the reference engine computes for an
`.engine` graph on the YOLOv8 path.  The reference keeps activations NHWC and
remaps ONNX axes by heuristics (PDEFA1.0/src/core/session_parts/*.inc); the
results it realises for the traced YOLOv8 pattern are the ONNX operator
semantics, which is what this module evaluates in NCHW:

  Conv      session_ops_nn.inc:2-65 -> ops::conv2d (conv2d.cpp:484-651);
            output size (H + 2p - ((k-1)d + 1)) / s + 1 (conv2d.cpp:442-446);
            fused activation codes 1 relu, 2 leaky, 3 sigmoid, 4 tanh, 5 silu
            (session_fusion.inc:33-107, conv2d.hpp:16-24), as the reference's
            kernel for the conv evaluates them (reference_conv_path,
            fused_activation); groups > 1 per group (depthwise
            conv2d.cpp:576-586, grouped 342-392)
  MaxPool   session_ops_nn.inc:267-347 -> pooling.cpp:35-101 (padding never wins)
  Resize    session_ops_shape.inc:96-202: nearest, target = in * scale
            (+0.5 truncation), source index floor(out * in/out)
  Concat    session_ops_shape.inc:66-93
  Slice     session_ops_shape.inc:754-889 (clamped starts/ends, steps)
  Reshape   session_ops_shape.inc:512-726 (0 copies a dim, -1 infers)
  Transpose session_ops_shape.inc:946-1096
  Softmax   session_ops_math.inc:223-318 (max-subtracted exp, / sum)
  Add/Sub/Mul/Div  session_ops_math.inc:4-220 (numpy broadcasting)
  TopK      session_ops_math.inc:321-395 (values, then indices)
  GatherElements  session_ops_math.inc:397-432
  Sigmoid   activation_avx2.cpp:110-121 (1 / (1 + e^-x)); Relu, LeakyRelu,
            Tanh, SiLU: session_ops_nn.inc:210-231 -> activation.cpp:28-70

Pins (tests/test_oracle.py): the compiled reference (oracle/_ref) on the same
`.engine` files and inputs; closed-form conv known answers from
PDEFA1.0/examples/test_conv2d.cpp:13-148; brute-force direct loops on tiny
shapes; silu(1) = 0.7311 (pdefa/tests/test_ops_extra.py:26-30).
"""
from __future__ import annotations

import numpy as np

from pdefa_amd.engine_format import EngineModel, OP_NAME


def conv2d(x, w, b=None, stride=(1, 1), pad=(0, 0), dil=(1, 1), act=0, slope=0.01, groups=1):
    """NCHW conv, float64 accumulation; w is [Cout, Cin/groups, KH, KW].

    groups > 1 (conv2d.cpp:576-597: the depthwise kernel when groups == Cin ==
    Cout, else engine_conv2d_grouped_gemm, conv2d.cpp:342-392): group g
    convolves input channels [g*Cin/groups, ...) with weight rows
    [g*Cout/groups, ...) into the same output channel range."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    if groups > 1:
        c, co = x.shape[1], w.shape[0]
        if c % groups or co % groups or w.shape[1] * groups != c:
            raise ValueError(f"conv: {c} -> {co} channels do not split into {groups} groups")
        cg, og = c // groups, co // groups
        parts = [conv2d(x[:, g * cg:(g + 1) * cg], w[g * og:(g + 1) * og],
                        None if b is None else np.asarray(b)[g * og:(g + 1) * og], stride, pad, dil)
                 for g in range(groups)]
        return activation(np.concatenate(parts, axis=1), act, slope)
    n, c, h, wd = x.shape
    co, ci, kh, kw = w.shape
    if ci != c:
        raise ValueError(f"conv: input has {c} channels, weight expects {ci}")
    sh, sw = stride
    ph, pw = pad
    dh, dw = dil
    ho = (h + 2 * ph - ((kh - 1) * dh + 1)) // sh + 1
    wo = (wd + 2 * pw - ((kw - 1) * dw + 1)) // sw + 1
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    wm = w.reshape(co, ci * kh * kw).T
    out = np.empty((n, co, ho, wo), np.float64)
    for i in range(n):
        cols = np.empty((ci, kh, kw, ho, wo), np.float64)
        for a in range(kh):
            for bb in range(kw):
                y0, x0 = a * dh, bb * dw
                cols[:, a, bb] = xp[i, :, y0:y0 + sh * (ho - 1) + 1:sh, x0:x0 + sw * (wo - 1) + 1:sw]
        cols = cols.reshape(ci * kh * kw, ho * wo).T
        out[i] = (cols @ wm).T.reshape(co, ho, wo)
    if b is not None:
        out += np.asarray(b, np.float64)[None, :, None, None]
    return activation(out, act, slope)


def activation(x, act, slope=0.01):
    """The plain functions behind the fused codes (conv2d.cpp:131-139,
    conv2d_gemm.cpp:55-64): 1 relu, 2 leaky relu, 3 sigmoid, 4 tanh, 5 silu."""
    if act == 0:
        return x
    if act == 1:
        return np.maximum(x, 0)
    if act == 2:
        return np.where(x > 0, x, x * slope)
    if act == 3:
        return 1.0 / (1.0 + np.exp(-x))
    if act == 4:
        return np.tanh(x)
    if act == 5:
        return x / (1.0 + np.exp(-x))
    raise ValueError(f"activation code {act}")


def gelu_tanh(x):
    """Tanh-form GELU, 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3)))
    (conv2d_winograd.cpp:108-111, conv2d_avx2.cpp:109-112)."""
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x * x * x)))


def reference_conv_path(cin, kh, kw, stride, pad, dil, groups):
    """The kernel the reference conv dispatcher (PDEFA1.0/src/ops/conv2d.cpp:484-651)
    sends a conv to, as far as it changes the fused activations: "direct"
    (groups 1, Cin <= 16, KH, KW <= 7 and not a plain 1x1 with stride 1 and
    no padding; conv2d.cpp:599-611), "winograd" (3x3, stride 1, dilation 1,
    groups 1, Cin <= 512; conv2d.cpp:616-629) or "other" (DFL, depthwise,
    grouped GEMM, GEMM)."""
    if groups != 1:
        return "other"
    pure_1x1 = (kh == 1 and kw == 1 and tuple(pad) == (0, 0) and tuple(stride) == (1, 1)
                and tuple(dil) == (1, 1))
    if not pure_1x1 and cin <= 16 and kh <= 7 and kw <= 7:
        return "direct"
    if kh == 3 and kw == 3 and tuple(stride) == (1, 1) and tuple(dil) == (1, 1) and cin <= 512:
        return "winograd"
    return "other"


def fused_activation(y, act, path, slope=0.01, compat_silu=True):
    """A fused code as the reference's kernel on `path` evaluates it:
    code 3 on the direct kernel is 1 / (1 + v) (conv2d_avx2.cpp:99-103),
    code 4 on the direct and Winograd kernels is tanh-form GELU
    (conv2d_avx2.cpp:109-112, conv2d_winograd.cpp:108-111), code 5 on the
    Winograd kernel the polynomial SiLU form (conv2d_winograd.cpp:81-101,
    evaluated in float32; compat_silu=False takes the true SiLU); everything
    else the plain function."""
    if path == "direct" and act == 3:
        return 1.0 / (1.0 + y)
    if path in ("direct", "winograd") and act == 4:
        return gelu_tanh(y)
    if path == "winograd" and act == 5 and compat_silu:
        return silu_winograd_compat(np.asarray(y, np.float32)).astype(np.asarray(y).dtype)
    return activation(y, act, slope)


def silu_winograd_compat(x):
    """The SiLU the reference applies in its Winograd epilogue, restated in
    float32 (PDEFA1.0/src/kernels/simd/avx2/conv2d_winograd.cpp:81-101).

    exp(-x) is formed as 2^n * P(f) with n = round(-x * log2 e) and
    f = -x * log2 e - n, where P is the degree-6 polynomial
    1 + f/2 + c4 f^2 + ... evaluated in f's log2 units; the result differs from
    the true SiLU by up to ~2% of |x|.  Inputs beyond the +/-88.37626 clamp
    return x (large positive) or 0 (large negative)."""
    x = np.asarray(x, np.float32)
    f32 = np.float32
    neg = -x
    fx = neg * f32(1.44269504088896341)
    n = np.where(fx >= 0, np.floor(fx + f32(0.5)), np.ceil(fx - f32(0.5))).astype(np.float32)
    f = (fx - n).astype(np.float32)
    p = np.full_like(f, f32(1.9875691500e-4))
    for c in (1.3981999507e-3, 8.3334519073e-3, 4.1665795894e-2, 1.6666665459e-1,
              5.0000001201e-1, 1.0):
        p = (p * f + f32(c)).astype(np.float32)
    e = np.clip(n, -127, 128).astype(np.int64) + 127
    with np.errstate(over="ignore"):  # n = 128 gives the exponent pattern of +inf, as in the reference
        scale = np.ldexp(np.float32(1.0), (e - 127).astype(np.int32)).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        y = (x / (f32(1.0) + p * scale)).astype(np.float32)
    y = np.where(neg < f32(-88.37626), x, y)
    y = np.where(neg > f32(88.37626), f32(0.0), y)
    return y


def _silu_form_with_n(x, n):
    f32 = np.float32
    fx = (-x) * f32(1.44269504088896341)
    f = (fx - n).astype(np.float32)
    p = np.full_like(f, f32(1.9875691500e-4))
    for c in (1.3981999507e-3, 8.3334519073e-3, 4.1665795894e-2, 1.6666665459e-1,
              5.0000001201e-1, 1.0):
        p = (p * f + f32(c)).astype(np.float32)
    scale = np.ldexp(np.float32(1.0), np.clip(n, -127, 128).astype(np.int32)).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        return (x / (f32(1.0) + p * scale)).astype(np.float32)


def silu_winograd_compat_branches(x, tol=2e-6):
    """Both sides of the compat SiLU's jumps.

    The form is discontinuous where -x log2 e crosses a half-integer (n
    switches while P(f) does not wrap continuously), jumping by ~2% of |x|.
    For inputs within `tol` (relative) of such a point a 1-ulp change in the
    conv result selects the other side, so a checker accepts either value
    there.  Returns (y_low_n, y_high_n, unstable_mask)."""
    x = np.asarray(x, np.float32)
    fx = ((-x) * np.float32(1.44269504088896341)).astype(np.float64)
    lo = np.floor(fx)
    unstable = np.abs(fx - lo - 0.5) <= tol * np.maximum(1.0, np.abs(fx))
    y_lo = _silu_form_with_n(x, lo.astype(np.float32))
    y_hi = _silu_form_with_n(x, (lo + 1).astype(np.float32))
    return y_lo, y_hi, unstable


def winograd_path(cin, kh, kw, stride, dil, groups):
    """True when the reference conv dispatcher routes a conv to its Winograd
    kernel (PDEFA1.0/src/ops/conv2d.cpp:602-631): 3x3, stride 1, dilation 1,
    groups 1, and 16 < Cin <= 512 (Cin <= 16 goes to the direct kernel)."""
    return reference_conv_path(cin, kh, kw, stride, (1, 1), dil, groups) == "winograd"


def conv2d_direct(x, w, b=None, stride=(1, 1), pad=(0, 0)):
    """Brute-force seven-loop conv (pins conv2d on tiny shapes)."""
    n, c, h, wd = x.shape
    co, ci, kh, kw = w.shape
    ho = (h + 2 * pad[0] - kh) // stride[0] + 1
    wo = (wd + 2 * pad[1] - kw) // stride[1] + 1
    out = np.zeros((n, co, ho, wo), np.float64)
    for i in range(n):
        for o in range(co):
            for y in range(ho):
                for xx in range(wo):
                    s = 0.0 if b is None else float(b[o])
                    for k in range(ci):
                        for a in range(kh):
                            for bb in range(kw):
                                iy = y * stride[0] - pad[0] + a
                                ix = xx * stride[1] - pad[1] + bb
                                if 0 <= iy < h and 0 <= ix < wd:
                                    s += float(x[i, k, iy, ix]) * float(w[o, k, a, bb])
                    out[i, o, y, xx] = s
    return out


def maxpool2d(x, k, s, p):
    n, c, h, w = x.shape
    ho = (h + 2 * p[0] - k[0]) // s[0] + 1
    wo = (w + 2 * p[1] - k[1]) // s[1] + 1
    xp = np.pad(x, ((0, 0), (0, 0), (p[0], p[0]), (p[1], p[1])), constant_values=-np.inf)
    out = np.full((n, c, ho, wo), -np.inf, x.dtype)
    for a in range(k[0]):
        for b in range(k[1]):
            out = np.maximum(out, xp[:, :, a:a + s[0] * (ho - 1) + 1:s[0],
                                     b:b + s[1] * (wo - 1) + 1:s[1]])
    return out


def resize_nearest(x, scales):
    n, c, h, w = x.shape
    sh, sw = float(scales[2]), float(scales[3])
    ho = int(np.float32(h) * np.float32(sh) + np.float32(0.5))
    wo = int(np.float32(w) * np.float32(sw) + np.float32(0.5))
    ry = np.float32(h) / np.float32(ho)
    rx = np.float32(w) / np.float32(wo)
    iy = np.minimum((np.arange(ho, dtype=np.float32) * ry).astype(np.int64), h - 1)
    ix = np.minimum((np.arange(wo, dtype=np.float32) * rx).astype(np.int64), w - 1)
    return x[:, :, iy][:, :, :, ix]


def softmax(x, axis):
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def _ints(t):
    return [int(v) for v in np.asarray(t).reshape(-1)]


def slice_(x, starts, ends, axes=None, steps=None):
    idx = [slice(None)] * x.ndim
    axes = list(range(len(starts))) if axes is None else axes
    steps = [1] * len(starts) if steps is None else steps
    for s, e, a, st in zip(starts, ends, axes, steps):
        if a < 0:
            a += x.ndim
        d = x.shape[a]
        s = s + d if s < 0 else s
        e = e + d if e < 0 else e
        s = min(max(s, 0), d)
        e = min(max(e, 0), d)
        idx[a] = slice(s, max(e, s), st)
    return x[tuple(idx)]


def reshape(x, shape):
    shape = list(shape)
    for i, s in enumerate(shape):
        if s == 0:
            shape[i] = x.shape[i]
    return x.reshape(shape)


def _consumers(model, ref):
    """One entry per use of `ref`: a node for each of its inputs that reads
    it, None for each graph output (session_fusion.inc:20-30 counts so)."""
    return [n for n in model.nodes for i in n.inputs if i == ref] + \
        [None for o in model.graph_outputs if o == ref]


_FUSABLE = {"Relu": 1, "LeakyRelu": 2, "Sigmoid": 3, "Tanh": 4}


def _single_act_consumer(model, conv):
    """(node, code) when conv's output has exactly one use and it is a
    one-input ReLU / LeakyReLU / Sigmoid / Tanh (session_fusion.inc:85-107)."""
    out = conv.outputs[0]
    cons = _consumers(model, out)
    if len(cons) != 1 or cons[0] is None:
        return None
    n = cons[0]
    if n.inputs == [out] and n.op_name in _FUSABLE:
        return n, _FUSABLE[n.op_name]
    return None


def _silu_nodes(model, conv):
    """(sigmoid, mul) node names when conv's output feeds exactly a Sigmoid and
    a Mul(conv, sigmoid), the pattern session_fusion.inc:33-81 fuses."""
    out = conv.outputs[0]
    cons = _consumers(model, out)
    if len(cons) != 2 or None in cons:
        return None
    sig = next((n for n in cons if n.op_name == "Sigmoid" and n.inputs == [out]), None)
    if sig is None or len(_consumers(model, sig.outputs[0])) != 1:
        return None
    mul = next((n for n in cons if n.op_name == "Mul" and sorted(n.inputs) ==
                sorted([out, sig.outputs[0]])), None)
    if mul is None:
        return None
    return {sig.name, mul.name}


def _silu_consumer(model, conv):
    names = _silu_nodes(model, conv)
    if names is None:
        return None
    mul = next(n for n in model.nodes if n.name in names and n.op_name == "Mul")
    return mul.outputs[0]


def run_graph(model: EngineModel, inputs, dtype=np.float64, compat_silu=True, flip=None, flip_tol=1e-5,
              flip_elems=None, jump_log=None, jump_tol=1e-6, jump_values=None):
    """Evaluates the graph on `inputs` (list of NCHW arrays); returns outputs
    as float32 arrays in graph_outputs order.  compat_silu=False evaluates the
    true SiLU everywhere.

    flip: optional predicate on a conv node's name.  On the compat-SiLU layers
    it accepts, every element whose pre-activation lies within flip_tol
    (relative, see silu_winograd_compat_branches) of one of the form's jumps
    takes the other side of the jump: the output an fp32 computation gets when
    its rounding lands there on the other side.
    flip_elems: {conv node name: flat indices} -- exactly these compat-SiLU
    activations take the other side of their jump.
    jump_log: optional list that receives (conv node name, flat index,
    relative distance) of every compat-SiLU activation whose pre-activation
    lies within jump_tol of a jump (the candidates for an fp32 conv landing
    on the other side).
    jump_values: optional dict that receives, for each jump_log entry
    (conv node name, flat index), the activation on each side of the jump:
    (the side the rounded float64 pre-activation takes, the other side)."""
    inter = {}
    skip = set()

    def get(ref):
        if ref <= -1000:
            return model.weights[-1000 - ref].astype(dtype)
        if ref < 0:
            return np.asarray(inputs[-1 - ref], dtype)
        return inter[ref]

    for node in model.nodes:
        if node.name in skip:
            continue
        op = OP_NAME.get(node.op)
        ins = node.inputs
        p = node.params
        if op == "Conv":
            b = get(ins[2]) if len(ins) > 2 else None
            groups = max(1, int(p.get("groups", 1)))
            x, w = get(ins[0]), get(ins[1])
            stride, dil = (p["stride_h"], p["stride_w"]), (p["dil_h"], p["dil_w"])
            pad = (p["pad_h"], p["pad_w"])
            y = conv2d(x, w, b, stride, pad, dil, groups=groups)
            path = reference_conv_path(x.shape[1], w.shape[2], w.shape[3], stride, pad, dil, groups)
            slope = float(p.get("leaky_slope", 0.01))
            # Conv -> Sigmoid -> Mul is fused into the conv by the reference
            # session (session_fusion.inc:33-81), a single-consumer
            # ReLU / LeakyReLU / Sigmoid / Tanh too (85-107); on the reference's
            # Winograd and direct kernels some fused codes are other functions
            # (fused_activation).
            silu = _silu_consumer(model, node)
            if silu is not None:
                if compat_silu and path == "winograd":
                    y32 = y.astype(np.float32)
                    straight = silu_winograd_compat(y32)
                    if flip is not None and flip(node.name):
                        y_lo, y_hi, unstable = silu_winograd_compat_branches(y32, tol=flip_tol)
                        other = np.where(straight == y_lo, y_hi, y_lo)
                        straight = np.where(unstable, other, straight)
                    if flip_elems and node.name in flip_elems:
                        idx = np.asarray(flip_elems[node.name], np.int64)
                        y_lo, y_hi, _ = silu_winograd_compat_branches(y32, tol=0.0)
                        flat, lo_f, hi_f = straight.reshape(-1), y_lo.reshape(-1), y_hi.reshape(-1)
                        flat[idx] = np.where(flat[idx] == lo_f[idx], hi_f[idx], lo_f[idx])
                    if jump_log is not None:
                        fx = ((-y32) * np.float32(1.44269504088896341)).astype(np.float64).reshape(-1)
                        dist = np.abs(fx - np.floor(fx) - 0.5) / np.maximum(1.0, np.abs(fx))
                        near = np.flatnonzero(dist <= jump_tol)
                        if jump_values is not None and near.size:
                            y_lo, y_hi, _ = silu_winograd_compat_branches(y32.reshape(-1)[near], tol=0.0)
                            own = silu_winograd_compat(y32.reshape(-1)[near])
                        for j, i in enumerate(near):
                            jump_log.append((node.name, int(i), float(dist[i])))
                            if jump_values is not None:
                                other = y_hi[j] if own[j] == y_lo[j] else y_lo[j]
                                jump_values[(node.name, int(i))] = (float(own[j]), float(other))
                    y = straight.astype(dtype)
                else:
                    y = y / (1.0 + np.exp(-y))
                inter[node.outputs[0]] = y
                inter[silu] = y
                skip.update(_silu_nodes(model, node))
                continue
            single = _single_act_consumer(model, node)
            code = int(p.get("fused_activation", 0))
            if single is not None:
                act_node, code = single
                if code == 2:
                    slope = float(act_node.params.get("leaky_slope", 0.01))
                y = fused_activation(y, code, path, slope, compat_silu)
                inter[node.outputs[0]] = y
                inter[act_node.outputs[0]] = y
                skip.add(act_node.name)
                continue
            y = fused_activation(y, code, path, slope, compat_silu)
        elif op == "Sigmoid":
            y = 1.0 / (1.0 + np.exp(-get(ins[0])))
        elif op in ("Relu", "Tanh", "SiLU"):
            y = activation(get(ins[0]), {"Relu": 1, "Tanh": 4, "SiLU": 5}[op])
        elif op == "LeakyRelu":
            y = activation(get(ins[0]), 2, float(p.get("leaky_slope", 0.01)))
        elif op in ("Add", "Sub", "Mul", "Div"):
            a, b = get(ins[0]), get(ins[1])
            y = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply,
                 "Div": np.divide}[op](a, b)
        elif op == "MaxPool":
            y = maxpool2d(get(ins[0]), (p["kernel_h"], p["kernel_w"]),
                          (p["stride_h"], p["stride_w"]), (p["pad_h"], p["pad_w"]))
        elif op == "Resize":
            scales = None
            for r in ins[1:]:
                t = get(r)
                if t.size == 4:
                    scales = t.reshape(-1)
                    break
            if scales is None:
                raise NotImplementedError("Resize without a 4-element scales input")
            y = resize_nearest(get(ins[0]), scales)
        elif op == "Concat":
            y = np.concatenate([get(r) for r in ins], axis=int(p["axis"]))
        elif op == "Slice":
            axes = _ints(get(ins[3])) if len(ins) > 3 else None
            steps = _ints(get(ins[4])) if len(ins) > 4 else None
            y = slice_(get(ins[0]), _ints(get(ins[1])), _ints(get(ins[2])), axes, steps)
        elif op == "Reshape":
            y = reshape(get(ins[0]), _ints(get(ins[1])))
        elif op == "Transpose":
            y = np.transpose(get(ins[0]), _ints(get(ins[1])))
        elif op == "Softmax":
            y = softmax(get(ins[0]), int(p["axis"]))
        elif op == "TopK":
            # session_ops_math.inc:321-395: the k largest along the axis
            # (k <= 0 or > the axis length: all of it), values then indices;
            # ties go to the lower index here (the reference's partial_sort
            # leaves their order open)
            x = get(ins[0])
            kt = model.weights[-1000 - ins[1]] if ins[1] <= -1000 else get(ins[1])
            kk = int(np.asarray(kt).reshape(-1)[0])
            ax = int(p["axis"])
            ax = ax + x.ndim if ax < 0 else ax
            if x.ndim == 4:
                raise NotImplementedError("TopK on rank-4 tensors (the reference sorts its channels-last storage)")
            n_ax = x.shape[ax]
            if kk <= 0 or kk > n_ax:
                kk = n_ax
            order = np.take(np.argsort(-x, axis=ax, kind="stable"), np.arange(kk), axis=ax)
            if node.outputs[0] >= 0:
                inter[node.outputs[0]] = np.take_along_axis(x, order, axis=ax)
            if len(node.outputs) > 1 and node.outputs[1] >= 0:
                inter[node.outputs[1]] = order.astype(np.float64)
            continue
        elif op == "GatherElements":
            # session_ops_math.inc:397-432: indices truncated toward zero,
            # negative ones from the end, the rest out of range read element 0
            data, idx = get(ins[0]), get(ins[1])
            ax = int(p["axis"])
            ax = ax + data.ndim if ax < 0 else ax
            n_ax = data.shape[ax]
            g = np.trunc(np.asarray(idx, np.float64)).astype(np.int64)
            g = np.where(g < 0, g + n_ax, g)
            g = np.where((g < 0) | (g >= n_ax), 0, g)
            y = np.take_along_axis(data, g, axis=ax)
        elif op in ("Input", "Output"):
            continue
        else:
            raise NotImplementedError(f"oracle: op {node.op} ({op}) in node {node.name}")
        inter[node.outputs[0]] = y
    return [inter[o].astype(np.float32) for o in model.graph_outputs]
