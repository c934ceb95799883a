"""Pins the CPU oracle (oracle/graph_ref.py, oracle/decode_ref.py) before it is
trusted as the checker of the GPU path.

- golden vectors written from the compiled reference engine (tests/golden/);
- the compiled reference itself (oracle/_ref) on fresh cases, when built;
- closed-form convolution answers of PDEFA1.0/examples/test_conv2d.cpp:13-148;
- brute-force direct loops on tiny shapes (catches index/transpose mistakes);
- ONNX-semantics identities for pooling, resize, softmax, slice, reshape;
- letterbox known answers (imageloader/tests/test_preprocess.cpp:27-130).
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import decode_ref, graph_ref, ref_lib
from pdefa_amd import postprocess, yolo_synth as ys

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = dict(atol=1e-3, rtol=1e-3)


def golden(name):
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        return json.load(f)


def check_samples(arr, g, atol=1e-3, rtol=1e-3):
    flat = arr.reshape(-1)
    idx = np.asarray(g["samples"]["index"])
    np.testing.assert_allclose(flat[idx], np.asarray(g["samples"]["value"]), atol=atol, rtol=rtol)
    means = arr.reshape(arr.shape[0], arr.shape[1], -1).astype(np.float64).mean(axis=(0, 2))
    np.testing.assert_allclose(means, np.asarray(g["channel_means"]), atol=atol, rtol=rtol)


# ---------------------------------------------------------------- conv KATs

def test_conv_kat_all_ones():
    y = graph_ref.conv2d(np.ones((1, 1, 5, 5)), np.ones((1, 1, 3, 3)), np.zeros(1))
    assert y.shape == (1, 1, 3, 3) and np.all(y == 9.0)


def test_conv_kat_varied():
    x = np.arange(1, 10, dtype=np.float64).reshape(1, 1, 3, 3)
    y = graph_ref.conv2d(x, np.ones((1, 1, 2, 2)), np.zeros(1))
    assert y.reshape(-1).tolist() == [12.0, 16.0, 24.0, 28.0]


def test_conv_kat_stride_pad():
    y = graph_ref.conv2d(np.ones((1, 1, 4, 4)), np.ones((1, 1, 3, 3)), np.zeros(1), stride=(2, 2), pad=(1, 1))
    assert y.reshape(-1).tolist() == [4.0, 6.0, 6.0, 9.0]


def test_conv_kat_fused_relu():
    y = graph_ref.conv2d(-np.ones((1, 1, 3, 3)), np.ones((1, 1, 2, 2)), np.zeros(1), act=1)
    assert np.all(y == 0.0)


@pytest.mark.parametrize("shape", [(1, 3, 7, 6, 4, 3, 1, 1), (2, 5, 9, 9, 3, 3, 2, 1), (1, 4, 8, 5, 6, 1, 1, 0),
                                   (1, 2, 6, 7, 2, 5, 3, 2)])
def test_conv_matches_brute_force(shape):
    n, ci, h, w, co, k, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal((n, ci, h, w))
    wt = rng.standard_normal((co, ci, k, k))
    b = rng.standard_normal(co)
    np.testing.assert_allclose(graph_ref.conv2d(x, wt, b, (s, s), (p, p)),
                               graph_ref.conv2d_direct(x, wt, b, (s, s), (p, p)), rtol=1e-12, atol=1e-12)


def test_silu_known_values():
    assert abs(graph_ref.activation(np.array([1.0]), 5)[0] - 0.7311) < 1e-3
    assert graph_ref.activation(np.array([0.0]), 5)[0] == 0.0


def test_winograd_form_silu_shape():
    # a faithful SiLU near 0 and for large |x|, ~2% off in between, with jumps
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    y = graph_ref.silu_winograd_compat(x)
    exact = x / (1 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(y - exact)) < 0.05 * np.max(np.abs(x)) + 1e-3
    assert np.max(np.abs(y - exact)) > 1e-3  # not the exact function
    assert graph_ref.silu_winograd_compat(np.array([100.0], np.float32))[0] == 100.0
    assert graph_ref.silu_winograd_compat(np.array([-100.0], np.float32))[0] == 0.0


def test_round_half_away_by_biased_truncation():
    """The device form of the reference's std::round: trunc(x + copysign(
    0.49999997, x)) in float32 equals rounding half away from zero, checked on
    every half-integer tie in the SiLU's range, the floats on either side of
    each, and 2^20 random floats (float64 rounding is the independent side)."""
    f32 = np.float32
    k = np.arange(-130, 131, dtype=np.float64)
    ties = (k + 0.5).astype(np.float32)
    ints = k.astype(np.float32)
    base = np.concatenate([ties, ints, np.float32([0.5, -0.5, 0.49999997, -0.49999997])])
    near = np.concatenate([base, np.nextafter(base, f32(np.inf)), np.nextafter(base, f32(-np.inf))])
    rnd = np.random.default_rng(3).uniform(-128, 128, 1 << 20).astype(np.float32)
    x = np.concatenate([near, rnd])
    got = np.trunc((x + np.copysign(f32(0.49999997), x)).astype(np.float32))
    want = np.trunc(x.astype(np.float64) + np.copysign(0.5, x.astype(np.float64)))
    np.testing.assert_array_equal(got, want)
    # the oracle's own rounding agrees on the ties
    fx_ties = np.where(ties >= 0, np.floor(ties + f32(0.5)), np.ceil(ties - f32(0.5)))
    np.testing.assert_array_equal(fx_ties, np.trunc(ties.astype(np.float64) + np.copysign(0.5, ties)))


def test_winograd_dispatch_rule():
    assert graph_ref.winograd_path(64, 3, 3, (1, 1), (1, 1), 1)
    assert not graph_ref.winograd_path(16, 3, 3, (1, 1), (1, 1), 1)   # direct kernel
    assert not graph_ref.winograd_path(576, 3, 3, (1, 1), (1, 1), 1)  # Cin > 512
    assert not graph_ref.winograd_path(64, 3, 3, (2, 2), (1, 1), 1)
    assert not graph_ref.winograd_path(64, 1, 1, (1, 1), (1, 1), 1)


# ------------------------------------------------------- other op semantics

def test_maxpool_sppf_equivalence():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 3, 11, 9))
    p5 = graph_ref.maxpool2d(x, (5, 5), (1, 1), (2, 2))
    p9 = graph_ref.maxpool2d(x, (9, 9), (1, 1), (4, 4))
    np.testing.assert_array_equal(graph_ref.maxpool2d(p5, (5, 5), (1, 1), (2, 2)), p9)
    # brute force
    ref = np.empty_like(p5)
    for i in range(11):
        for j in range(9):
            ref[..., i, j] = x[..., max(i - 2, 0):i + 3, max(j - 2, 0):j + 3].max(axis=(-1, -2))
    np.testing.assert_array_equal(p5, ref)


def test_resize_nearest_2x():
    x = np.arange(6, dtype=np.float32).reshape(1, 1, 2, 3)
    y = graph_ref.resize_nearest(x, [1, 1, 2, 2])
    np.testing.assert_array_equal(y, x.repeat(2, 2).repeat(2, 3))


def test_softmax_and_slice():
    x = np.random.default_rng(0).standard_normal((2, 16, 3))
    s = graph_ref.softmax(x, 1)
    np.testing.assert_allclose(s.sum(1), 1.0, rtol=1e-12)
    y = graph_ref.slice_(x, [2], [2 ** 31 - 1], [1])
    assert y.shape == (2, 14, 3)
    assert graph_ref.reshape(x, [0, -1]).shape == (2, 48)


# ------------------------------------------------------- golden vectors

@pytest.mark.parametrize("name,args", [("conv3x3_s1_64_160", (64, 64, 3, 1, 160)),
                                       ("conv3x3_s2_64_160", (64, 64, 3, 2, 160)),
                                       ("conv1x1_128_64_160", (128, 64, 1, 1, 160))])
def test_oracle_single_conv_vs_golden(name, args):
    g = golden(name)
    model, x = ys.build_single_conv(*args, seed=7)
    import hashlib
    assert hashlib.sha256(x.tobytes()).hexdigest() == g["input_sha256"]
    out = graph_ref.run_graph(model, [x])[0]
    assert list(out.shape) == g["shape"]
    check_samples(out, g, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("name,args,groups", [("dwconv3x3_s1_64_80", (64, 64, 3, 1, 80), 64),
                                              ("dwconv3x3_s2_96_41", (96, 96, 3, 2, 41), 96),
                                              ("gconv3x3_g4_64_40", (64, 64, 3, 1, 40), 4),
                                              ("gconv3x3_g16_32_40", (32, 32, 3, 1, 40), 16)])
def test_oracle_grouped_conv_vs_golden(name, args, groups):
    """Depthwise and grouped convs against the reference's own results
    (its depthwise kernel and grouped GEMM, conv2d.cpp:576-597)."""
    g = golden(name)
    assert g["groups"] == groups
    model, x = ys.build_single_conv(*args, seed=7, groups=groups)
    import hashlib
    assert hashlib.sha256(x.tobytes()).hexdigest() == g["input_sha256"]
    out = graph_ref.run_graph(model, [x])[0]
    assert list(out.shape) == g["shape"]
    check_samples(out, g, atol=2e-5, rtol=2e-5)


def test_grouped_conv_matches_brute_force():
    """Grouped conv against a seven-loop sum whose input channel is picked
    per output channel: output channel o sums input channels
    (o // (Cout/G)) * Cin/G + j (a wrong group mapping fails here)."""
    rng = np.random.default_rng(5)
    n, c, h, w_, co, g, k, s, p = 2, 6, 7, 6, 9, 3, 3, 2, 1
    x = rng.standard_normal((n, c, h, w_))
    wt = rng.standard_normal((co, c // g, k, k))
    b = rng.standard_normal(co)
    ho, wo = (h + 2 * p - k) // s + 1, (w_ + 2 * p - k) // s + 1
    want = np.zeros((n, co, ho, wo))
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)))
    for i in range(n):
        for o in range(co):
            for y in range(ho):
                for xx in range(wo):
                    acc = b[o]
                    for j in range(c // g):
                        ci = (o // (co // g)) * (c // g) + j
                        for a in range(k):
                            for bb in range(k):
                                acc += xp[i, ci, y * s + a, xx * s + bb] * wt[o, j, a, bb]
                    want[i, o, y, xx] = acc
    np.testing.assert_allclose(graph_ref.conv2d(x, wt, b, (s, s), (p, p), groups=g), want, rtol=1e-12, atol=1e-12)
    # depthwise: every channel on its own
    wd = rng.standard_normal((c, 1, k, k))
    got = graph_ref.conv2d(x, wd, None, (1, 1), (1, 1), groups=c)
    for ci in range(c):
        np.testing.assert_allclose(got[:, ci:ci + 1], graph_ref.conv2d_direct(x[:, ci:ci + 1], wd[ci:ci + 1],
                                                                              None, (1, 1), (1, 1)), atol=1e-12)


@pytest.fixture(scope="module")
def yolov8n_model():
    return ys.build_yolov8("n", seed=0)


@pytest.mark.parametrize("img", [0, 1, 2])
def test_oracle_yolov8n_vs_golden(yolov8n_model, img):
    g = golden(f"yolov8n_640_img{img}")
    x, metas = ys.yolo_inputs(img + 1)
    x = x[img:img + 1]
    import hashlib
    assert hashlib.sha256(x.tobytes()).hexdigest() == g["input_sha256"]
    out = graph_ref.run_graph(yolov8n_model, [x])[0]
    assert list(out.shape) == g["shape"]
    check_samples(out, g)
    assert g["min_score_gap_to_threshold"] >= 1e-2
    dets = decode_ref.decode(out.tolist(), metas[img], g["conf_thres"], g["iou_thres"])
    gd = g["detections"]
    assert [(d["anchor"], d["cls"]) for d in dets] == [(d["anchor"], d["cls"]) for d in gd]
    for a, b in zip(dets, gd):
        for k in ("x1", "y1", "x2", "y2", "conf"):
            assert math.isclose(a[k], b[k], rel_tol=1e-3, abs_tol=1e-3)


def test_sgemm_golden():
    g = golden("sgemm_512")
    rng = np.random.default_rng(42)
    a = rng.standard_normal((512, 512), dtype=np.float32)
    b = rng.standard_normal((512, 512), dtype=np.float32)
    c = a.astype(np.float64) @ b.astype(np.float64)
    idx = np.asarray(g["samples"]["index"])
    np.testing.assert_allclose(c.reshape(-1)[idx], g["samples"]["value"], atol=1e-3, rtol=1e-4)
    np.testing.assert_allclose(c.sum(1), g["row_sums"], atol=1e-2, rtol=1e-4)
    np.testing.assert_allclose(np.eye(4) @ np.arange(16.0).reshape(4, 4), np.arange(16.0).reshape(4, 4))


# ------------------------------------------------------- letterbox

def test_letterbox_known_answers():
    img = np.full((4, 4, 3), 128, np.uint8)
    t, m = ys.letterbox(img, 8, 8, 1 / 255, 0.0)
    assert t.shape == (1, 3, 8, 8) and (m["pad_x"], m["pad_y"], m["scaled_w"], m["scaled_h"]) == (0, 0, 8, 8)
    assert abs(t[0, 0, 0, 0] - 128 / 255) < 0.01
    img = np.full((50, 100, 3), 200, np.uint8)
    t, m = ys.letterbox(img, 100, 100, 1 / 255, 0.0)
    assert (m["scaled_w"], m["scaled_h"], m["pad_x"], m["pad_y"]) == (100, 50, 0, 25)
    assert abs(t.reshape(-1)[50]) < 1e-3 and abs(t.reshape(-1)[50 * 100 + 50] - 200 / 255) < 0.02
    g = np.full((4, 4), 100, np.uint8)
    t, _ = ys.letterbox(g, 4, 4, 1 / 255, 0.0)
    assert np.allclose(t[0, 0], t[0, 1]) and np.allclose(t[0, 0], t[0, 2])
    assert abs(t[0, 0, 0, 0] - 100 / 255) < 0.01


def test_letterbox_vs_golden():
    g = golden("letterbox_1280x720")
    img = ys.synth_image(0, 1280, 720)
    t, m = ys.letterbox(img, 640, 640, 1 / 255, 114 / 255)
    for k in ("pad_x", "pad_y", "scaled_w", "scaled_h"):
        assert m[k] == g["meta"][k]
    idx = np.asarray(g["samples"]["index"])
    np.testing.assert_allclose(t.reshape(-1)[idx], g["samples"]["value"], atol=1e-6)


# ------------------------------------------------------- decode / NMS

def test_decode_zeros_is_empty():
    assert postprocess.decode_yolo(np.zeros((1, 84, 8400), np.float32)) == []
    assert decode_ref.decode(np.zeros((1, 84, 8400), np.float32).tolist()) == []


def test_decode_matches_restatement():
    rng = np.random.default_rng(5)
    out = np.zeros((1, 84, 500), np.float32)
    out[0, :2] = rng.uniform(0, 640, (2, 500))
    out[0, 2:4] = rng.uniform(5, 80, (2, 500))
    out[0, 4:] = rng.uniform(0, 0.3, (80, 500))
    out[0, 4 + 7, :40] = 0.9  # duplicated classes -> suppression
    meta = {"ratio": 0.5, "pad_x": 0, "pad_y": 140, "orig_w": 1280, "orig_h": 720}
    a = postprocess.decode_yolo(out, meta, with_anchor=True)
    b = decode_ref.decode(out.tolist(), meta)
    assert len(a) > 5 and a == b


# ------------------------------------------------------- compiled reference

needs_ref = pytest.mark.skipif(not ref_lib.available(), reason="oracle/_ref not built (make -C oracle)")


@needs_ref
@pytest.mark.parametrize("cin,cout,k,s,hw", [(64, 64, 3, 1, 40), (32, 48, 3, 2, 33), (128, 64, 1, 1, 24),
                                             (16, 16, 3, 1, 20), (3, 16, 3, 2, 32), (600, 40, 3, 1, 6)])
def test_oracle_vs_compiled_reference_conv(tmp_path, cin, cout, k, s, hw):
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=cin + hw)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    r = ref_lib.RefSession(path).run(x)[0]
    o = graph_ref.run_graph(model, [x])[0]
    np.testing.assert_allclose(o, r, atol=2e-5, rtol=2e-5)


@needs_ref
@pytest.mark.parametrize("cin,cout,k,s,hw,groups", [(64, 64, 3, 1, 20, 64), (96, 96, 3, 2, 21, 96),
                                                    (64, 64, 3, 1, 20, 4), (32, 32, 3, 1, 20, 16),
                                                    (32, 64, 3, 1, 12, 32), (48, 96, 5, 2, 17, 8)])
def test_oracle_vs_compiled_reference_grouped_conv(tmp_path, cin, cout, k, s, hw, groups):
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=cin + hw, groups=groups)
    path = str(tmp_path / "g.engine")
    ys.save(model, path)
    r = ref_lib.RefSession(path).run(x)[0]
    o = graph_ref.run_graph(model, [x])[0]
    np.testing.assert_allclose(o, r, atol=2e-5, rtol=2e-5)


@needs_ref
def test_oracle_vs_compiled_reference_scdown(tmp_path):
    model, x = ys.build_scdown(64, 128, 40, n=2)
    path = str(tmp_path / "s.engine")
    ys.save(model, path)
    r = ref_lib.RefSession(path).run(x)[0]
    o = graph_ref.run_graph(model, [x])[0]
    np.testing.assert_allclose(o, r, atol=2e-5, rtol=2e-5)


@needs_ref
def test_oracle_vs_compiled_reference_yolov8n_small(tmp_path):
    model = ys.build_yolov8("n", seed=3, imgsz=160)
    path = str(tmp_path / "y.engine")
    ys.save(model, path)
    x, _ = ys.yolo_inputs(2, imgsz=160)
    r = ref_lib.RefSession(path).run(x[1:2])[0]
    o = graph_ref.run_graph(model, [x[1:2]])[0]
    np.testing.assert_allclose(o, r, **TOL)


@needs_ref
@pytest.mark.parametrize("w,h,ch", [(1280, 720, 3), (1024, 768, 3), (800, 800, 3), (37, 91, 3), (3, 2, 3),
                                    (1, 1, 3), (333, 200, 1), (64, 97, 4)])
def test_oracle_vs_compiled_reference_letterbox(w, h, ch):
    """The letterbox restatement and the product's pdefa_preprocess_letterbox
    equal the reference's preprocess_letterbox_direct bit for bit (its GCC
    build fuses the bilinear blend into FMAs; both follow that rounding)."""
    from pdefa_amd import pdefa
    img = ys.synth_image(w + h, w, h)
    img = img[:, :, 0] if ch == 1 else (np.dstack([img, img[:, :, :1]]) if ch == 4 else img)
    a, ma = ys.letterbox(img, 640, 640, 1 / 255, 114 / 255)
    b, mb = ref_lib.letterbox(img, 640, 640, 1 / 255, 114 / 255)
    t, mc = pdefa.preprocess_letterbox(pdefa.Image.from_array(img), 640, 640, 1 / 255, 114 / 255)
    for k in ("pad_x", "pad_y", "scaled_w", "scaled_h"):
        assert ma[k] == mb[k] == getattr(mc, k)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(t.to_numpy(), b)


@needs_ref
def test_compiled_reference_matmul():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((70, 130), dtype=np.float32)
    b = rng.standard_normal((130, 45), dtype=np.float32)
    np.testing.assert_allclose(ref_lib.matmul(a, b), a.astype(np.float64) @ b, atol=1e-4, rtol=1e-4)


def test_flip_takes_the_other_side_of_each_jump():
    """run_graph(flip=...) puts every compat-SiLU element within flip_tol of a
    jump on the other branch; with a tolerance covering every input all of a
    Winograd-path layer's elements switch branch."""
    model, x = ys.build_single_conv(32, 8, 3, 1, 6, seed=2)
    pre_model, _ = ys.build_single_conv(32, 8, 3, 1, 6, seed=2, silu=False)
    pre = graph_ref.run_graph(pre_model, [x])[0]
    straight = graph_ref.silu_winograd_compat(pre)
    lo, hi, unstable = graph_ref.silu_winograd_compat_branches(pre, tol=0.6)
    assert unstable.all()
    want = np.where(straight == lo, hi, lo)
    got = graph_ref.run_graph(model, [x], flip=lambda name: True, flip_tol=0.6)[0]
    np.testing.assert_array_equal(got, want)
    # each branch is the form with n one apart: they differ, by ~2% of |x| at the jump
    assert not np.array_equal(lo, hi)
    # no flip predicate: the straight compat form
    np.testing.assert_array_equal(graph_ref.run_graph(model, [x])[0], straight)


# ------------------------------------------------ decode / NMS known answers

from tests import decode_kats  # noqa: E402


def _decode_kat(fn, name):
    boxes, nc, kw, want = decode_kats.CASES[name]
    h = decode_kats.head(boxes, nc)
    kw = dict(kw)
    meta = kw.pop("meta", None)
    return fn(h, meta, **kw), want


@pytest.mark.parametrize("name", sorted(decode_kats.CASES))
def test_decode_restatement_known_answers(name):
    got, want = _decode_kat(lambda h, meta, **kw: decode_ref.decode(h.tolist(), meta, **kw), name)
    assert got == want


@pytest.mark.parametrize("name", sorted(decode_kats.CASES))
def test_decode_yolo_known_answers(name):
    got, want = _decode_kat(lambda h, meta, **kw: postprocess.decode_yolo(h[None], meta, with_anchor=True, **kw),
                            name)
    assert got == want


def test_decode_known_answers_catch_rule_changes(monkeypatch):
    """Each rule the known answers pin, changed in a copy of the restatement,
    makes at least one of them fail: '<' for '<=' at the IoU threshold, '<='
    for '<' at conf_thres, '>=' for '>' in the class scan, clamps dropped,
    sorting by anchor instead of by class order."""
    import inspect
    src = inspect.getsource(decode_ref)
    mutants = {
        "iou <= thr": ("if v <= iou_thres]", "if v < iou_thres]"),
        "conf <": ("if best_s < conf_thres:", "if best_s <= conf_thres:"),
        "strict >": ("if s > best_s:", "if s >= best_s:"),
        "clamp": ("x1 = 0.0 if x1 < 0 else (ow if x1 > ow else x1)", "pass"),
        "class order": ("keep.sort(key=lambda i: boxes[i][4], reverse=True)",
                        "keep.sort(key=lambda i: (-boxes[i][4], boxes[i][6]))"),
        "max_det": ("keep = keep[:max_det]", "keep = keep[:max_det + 1]"),
        "iou guard": ("- inter + 1e-9)", "- inter + 1e-3)"),
    }
    for what, (a, b) in mutants.items():
        assert a in src, what
        ns = {}
        exec(compile(src.replace(a, b), "decode_mutant", "exec"), ns)
        failed = []
        for name in decode_kats.CASES:
            got, want = _decode_kat(lambda h, meta, **kw: ns["decode"](h.tolist(), meta, **kw), name)
            if got != want:
                failed.append(name)
        assert failed, f"no known answer catches the change '{what}'"


# ---------------------------- fused single-consumer activations, by path

ACT_CONV_CASES = [
    # cin, cout, k, stride, hw: the reference's direct kernel (Cin <= 16),
    # its Winograd kernel (3x3 s1, 16 < Cin <= 512), its GEMM (1x1, 3x3 s2,
    # Cin > 512) and a direct-kernel 5x5
    (3, 16, 3, 1, 20), (12, 20, 5, 1, 11), (32, 24, 3, 1, 18), (576, 40, 3, 1, 8), (64, 48, 3, 2, 17),
    (24, 32, 1, 1, 13),
]


def _pole_safe_close(o, r, pre, act, path):
    """|o - r| <= 2e-5 (1 + |r|), except where the reference's direct-kernel
    sigmoid 1 / (1 + v) is near its pole (|1 + v| < 0.1), where fp32 is
    ill-conditioned (relative error amplified by |v / (1 + v)|): there the
    relative bound is 1e-3."""
    err = np.abs(o.astype(np.float64) - r.astype(np.float64))
    ok = err <= 2e-5 * (1 + np.abs(r))
    if act == "Sigmoid" and path == "direct":
        near = np.abs(1.0 + pre) < 0.1
        ok |= near & (err <= 1e-3 * np.abs(r))
    assert ok.all(), f"{int((~ok).sum())} elements differ, max {err.max():.3e}"


@needs_ref
@pytest.mark.parametrize("act", ["Relu", "LeakyRelu", "Sigmoid", "Tanh"])
@pytest.mark.parametrize("cin,cout,k,s,hw", ACT_CONV_CASES)
def test_oracle_fused_activation_vs_compiled_reference(tmp_path, act, cin, cout, k, s, hw):
    """Conv -> ReLU / LeakyReLU(0.1) / Sigmoid / Tanh, fused by the reference
    session (session_fusion.inc:85-107) and evaluated by the kernel its
    dispatcher picks.  On the Winograd and direct kernels a fused Tanh is
    tanh-form GELU and on the direct kernel a fused Sigmoid is 1 / (1 + v):
    the plain functions differ from the reference there (checked), the
    oracle's per-path functions do not."""
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=5, act=act, centered=True)
    path = str(tmp_path / "a.engine")
    ys.save(model, path)
    r = ref_lib.RefSession(path).run(x)[0]
    o = graph_ref.run_graph(model, [x])[0]
    pre_model, _ = ys.build_single_conv(cin, cout, k, s, hw, seed=5, silu=False, centered=True)
    pre = graph_ref.run_graph(pre_model, [x])[0].astype(np.float64)
    kpath = graph_ref.reference_conv_path(cin, k, k, (s, s), (k // 2, k // 2), (1, 1), 1)
    _pole_safe_close(o, r, pre, act, kpath)
    code = {"Relu": 1, "LeakyRelu": 2, "Sigmoid": 3, "Tanh": 4}[act]
    plain = graph_ref.activation(pre, code, 0.1)
    quirk = (act == "Tanh" and kpath in ("direct", "winograd")) or (act == "Sigmoid" and kpath == "direct")
    assert quirk == (not np.allclose(plain, r, atol=1e-3, rtol=1e-3)), (act, kpath)


def test_reference_conv_path_rule():
    p = graph_ref.reference_conv_path
    assert p(3, 3, 3, (2, 2), (1, 1), (1, 1), 1) == "direct"
    assert p(16, 3, 3, (1, 1), (1, 1), (1, 1), 1) == "direct"
    assert p(16, 1, 1, (1, 1), (0, 0), (1, 1), 1) == "other"     # plain 1x1
    assert p(16, 1, 1, (2, 2), (0, 0), (1, 1), 1) == "direct"    # strided 1x1
    assert p(16, 9, 9, (1, 1), (4, 4), (1, 1), 1) == "other"     # kernel > 7
    assert p(17, 3, 3, (1, 1), (1, 1), (1, 1), 1) == "winograd"
    assert p(512, 3, 3, (1, 1), (1, 1), (1, 1), 1) == "winograd"
    assert p(513, 3, 3, (1, 1), (1, 1), (1, 1), 1) == "other"
    assert p(64, 3, 3, (2, 2), (1, 1), (1, 1), 1) == "other"
    assert p(64, 3, 3, (1, 1), (1, 1), (2, 2), 1) == "other"
    assert p(64, 3, 3, (1, 1), (1, 1), (1, 1), 4) == "other"
    assert p(8, 3, 3, (1, 1), (1, 1), (1, 1), 8) == "other"      # depthwise


# --------------------------------------- TopK / GatherElements (YOLOv10 heads)

@needs_ref
@pytest.mark.parametrize("anchors,nc,k,k_dtype", [(8400, 80, 300, np.int64), (2100, 20, 100, np.float32),
                                                  (1000, 5, 0, np.int64), (700, 6, 5000, np.int64)])
def test_oracle_topk_head_vs_compiled_reference(tmp_path, anchors, nc, k, k_dtype):
    """The YOLOv10-style selection (Transpose, Slice, TopK, GatherElements,
    Concat) on a tie-free head: oracle = reference on every output element,
    k from an int64 or float constant (k <= 0 or > the axis length: all of
    it), the indices output typed I32 by the reference."""
    model, x = ys.build_topk_head(anchors, nc, k, k_dtype=k_dtype)
    path = str(tmp_path / "h.engine")
    ys.save(model, path)
    r = ref_lib.RefSession(path)
    ro = r.run(x)
    assert r.output_dtypes() == [12, 6]
    oo = graph_ref.run_graph(model, [x])
    kk = k if 0 < k <= anchors else anchors
    assert ro[0].shape == (1, kk, 8) and ro[1].shape == (1, kk, nc)
    for a, b in zip(ro, oo):
        np.testing.assert_array_equal(a, b)


@needs_ref
@pytest.mark.parametrize("shape,axis,k", [((5, 1000), 1, 7), ((1000, 3), 0, 10), ((2, 3, 50), -1, 50),
                                          ((4096,), 0, 1), ((3, 700, 2), 1, 699)])
def test_oracle_topk_gather_vs_compiled_reference(tmp_path, shape, axis, k):
    """TopK values and indices, and GatherElements with a constant int64
    index tensor holding negative and out-of-range entries (the reference
    wraps negatives once and reads element 0 for the rest)."""
    ax = axis % len(shape)
    rng = np.random.default_rng(len(shape) * 100 + k)
    gi = rng.integers(-shape[ax] - 3, shape[ax] + 3, size=shape).astype(np.int64)
    model, x = ys.build_topk_gather(shape, axis, k, gather_idx=gi)
    path = str(tmp_path / "t.engine")
    ys.save(model, path)
    ro = ref_lib.RefSession(path).run(x)
    oo = graph_ref.run_graph(model, [x])
    for a, b in zip(ro, oo):
        np.testing.assert_array_equal(a, b)
    # the gather rule by hand on one row
    flat_idx = np.moveaxis(gi, ax, 0).reshape(shape[ax], -1)[:, 0]
    want = np.moveaxis(x, ax, 0).reshape(shape[ax], -1)[:, 0]
    fixed = [v + shape[ax] if v < 0 else v for v in flat_idx]
    fixed = [v if 0 <= v < shape[ax] else 0 for v in fixed]
    np.testing.assert_array_equal(np.moveaxis(oo[2], ax, 0).reshape(shape[ax], -1)[:, 0], want[fixed])


def tied_rows(shape, seed=5):
    """Rows of few distinct values (ties everywhere), +0.0 and -0.0 among them."""
    rng = np.random.default_rng(seed)
    vals = np.array([0.5, -0.25, 0.0, -0.0, 1.0, 0.5], np.float32)
    return vals[rng.integers(0, len(vals), size=shape)]


@needs_ref
@pytest.mark.parametrize("shape,axis,k", [((4, 60), 1, 20), ((50, 3), 0, 49)])
def test_oracle_topk_ties_vs_compiled_reference(tmp_path, shape, axis, k):
    """With tied values (and +0.0 beside -0.0) the reference's
    std::partial_sort leaves the order inside a group of equal values
    open: its values equal the oracle's exactly, and each of its indices
    points at a value equal to the oracle's at that position (the indices
    may differ only inside groups of equal values)."""
    model, _ = ys.build_topk_gather(shape, axis, k)
    x = tied_rows(shape)
    path = str(tmp_path / "t.engine")
    ys.save(model, path)
    rv, ri = ref_lib.RefSession(path).run(x)[:2]
    ov, oi = graph_ref.run_graph(model, [x])[:2]
    np.testing.assert_array_equal(rv, ov)
    xa = np.moveaxis(x, axis, -1)
    take = lambda idx: np.take_along_axis(xa, np.moveaxis(idx, axis, -1).astype(np.int64), axis=-1)
    np.testing.assert_array_equal(take(ri), np.moveaxis(ov, axis, -1))
    np.testing.assert_array_equal(take(oi), np.moveaxis(ov, axis, -1))
    # the oracle's rule: ties by ascending index, +0.0 and -0.0 equal
    row = xa.reshape(-1, xa.shape[-1])[0]
    want = sorted(range(len(row)), key=lambda i: (-float(row[i]), i))[:k]
    assert np.moveaxis(oi, axis, -1).reshape(-1, k)[0].astype(np.int64).tolist() == want


def test_engine_format_keeps_int64_constants(tmp_path):
    from pdefa_amd import engine_format as ef
    model, _ = ys.build_topk_head(300, 4, 10)
    path = str(tmp_path / "h.engine")
    ys.save(model, path)
    back = ef.read_engine(path)
    k = back.weights[back.weight_names.index("/head/k")]
    assert k.dtype == np.int64 and k.tolist() == [10]
