"""The reference-compatible Python API (pdefa_amd.pdefa), tested the way the
reference tests its package (pdefa/tests/test_smoke.py, test_tensor*.py,
test_ops*.py, test_errors*.py, test_image.py, test_preprocess.py,
test_postprocess.py, test_engine.py, test_session.py, test_batch.py).

Differences, all from what this build ships:
- images are binary PPM (the reference tests read a 50x50 JPEG and PNG; the
  image loader here decodes PPM/PGM only) -- same 50x50 solid-colour content;
- tiny.engine (not shipped with the reference either) is replaced by
  yolo_synth.build_tiny: same [1,3,64,64] -> [1,4] shapes;
- anything that runs a model or a matmul needs the GPU and is marked `gpu`.
"""
import re

import os

import numpy as np
import pytest

from pdefa_amd import pdefa, yolo_synth as ys


def write_ppm(path, w=50, h=50, rgb=(200, 120, 40)):
    px = np.empty((h, w, 3), np.uint8)
    px[:] = rgb
    with open(path, "wb") as f:
        f.write(f"P6\n{w} {h}\n255\n".encode() + px.tobytes())
    return str(path)


@pytest.fixture
def cat_ppm(tmp_path):
    return write_ppm(tmp_path / "cat.ppm")


@pytest.fixture
def tiny_engine(tmp_path):
    path = str(tmp_path / "tiny.engine")
    ys.save(ys.build_tiny(), path)
    return path


# ---------------------------------------------------------------- smoke

def test_version_format():
    v = pdefa.version()
    assert re.fullmatch(r"\d+\.\d+\.\d+(?:[.\-][A-Za-z0-9]+)?", v), v


def test_imports():
    for name in ("Context", "Model", "Session", "Tensor", "Image", "load_image", "decode_yolo",
                 "prepare_for_engine", "prepare_for_model", "preprocess_letterbox", "ops_add", "ops_matmul",
                 "randn", "zeros", "ones", "BatchInference", "Box", "PreprocessMeta"):
        assert hasattr(pdefa, name), name
    for name in pdefa.__all__:
        assert hasattr(pdefa, name), name


def test_simd_and_brand():
    assert pdefa.simd_level() in ("AVX2", "AVX-512", "SSE", "SCALAR")
    assert len(pdefa.cpu_brand()) > 0
    assert pdefa.__license__ == "AGPL-3.0-or-later"


# ---------------------------------------------------------------- tensors

def test_zeros_shape():
    t = pdefa.zeros(3, 4)
    assert t.shape == (3, 4) and t.numel == 12 and t.ndim == 2
    t3 = pdefa.zeros(2, 3, 4)
    assert t3.shape == (2, 3, 4) and t3.numel == 24 and t3.ndim == 3


def test_ones_and_list_roundtrips():
    assert pdefa.ones(2, 3).tolist() == [[1.0] * 3] * 2
    src = [[1.0, 2.0], [3.0, 4.0]]
    assert pdefa.from_list(src).tolist() == src
    src3 = [[[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]]]
    t = pdefa.from_list(src3)
    assert t.shape == (2, 2, 2) and t.tolist() == src3


def test_from_list_deep_copy():
    src = [[1.0, 2.0]]
    t = pdefa.from_list(src)
    src[0][0] = 999.0
    assert t.tolist() == [[1.0, 2.0]]


def test_operators():
    one = pdefa.ones(2, 2)
    assert (one + one).tolist() == [[2.0, 2.0]] * 2
    assert (one - one).tolist() == [[0.0, 0.0]] * 2
    assert (one * 3.0).tolist() == [[3.0, 3.0]] * 2
    assert (one / 4.0).tolist() == [[0.25, 0.25]] * 2
    assert (-one).tolist() == [[-1.0, -1.0]] * 2


def test_fill_and_copy_from_list():
    t = pdefa.zeros(2, 2)
    t.fill(0.5)
    assert t.tolist() == [[0.5, 0.5]] * 2
    t = pdefa.zeros(2, 3)
    t.copy_from_list([[1, 2, 3], [4, 5, 6]])
    assert t.tolist() == [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]


def test_randn_deterministic():
    assert pdefa.randn(3, 3, seed=42).tolist() == pdefa.randn(3, 3, seed=42).tolist()
    assert pdefa.randn(3, 3, seed=1).tolist() != pdefa.randn(3, 3, seed=2).tolist()
    assert pdefa.randn(2, 3, 4, seed=42).shape == (2, 3, 4)
    u = np.array(pdefa.rand(1000, seed=5).tolist())
    assert u.min() >= 0.0 and u.max() < 1.0


def test_to_numpy():
    t = pdefa.from_list([[1.0, 2.0], [3.0, 4.0]])
    assert np.array_equal(t.to_numpy(), np.array([[1, 2], [3, 4]], np.float32))


# ---------------------------------------------------------------- ops (host helpers)

def test_unary_inplace():
    t = pdefa.from_list([[-1.0, 0.0, 2.0]])
    pdefa.ops_relu(t)
    assert t.tolist() == [[0.0, 0.0, 2.0]]
    t = pdefa.from_list([[0.0]])
    assert abs(pdefa.ops_sigmoid(t).tolist()[0][0] - 0.5) < 1e-6
    assert abs(pdefa.ops_tanh(pdefa.from_list([[0.0]])).tolist()[0][0]) < 1e-6
    assert abs(pdefa.ops_gelu(pdefa.from_list([[1.0]])).tolist()[0][0] - 0.8413) < 1e-3
    assert abs(pdefa.ops_gelu(pdefa.from_list([[0.0]])).tolist()[0][0]) < 1e-6
    assert abs(pdefa.ops_silu(pdefa.from_list([[1.0]])).tolist()[0][0] - 0.7311) < 1e-3
    assert abs(pdefa.ops_silu(pdefa.from_list([[0.0]])).tolist()[0][0]) < 1e-6
    assert pdefa.ops_clip(pdefa.from_list([[-5.0, 0.0, 5.0]]), -1.0, 1.0).tolist() == [[-1.0, 0.0, 1.0]]


def test_softmax():
    t = pdefa.ops_softmax(pdefa.from_list([[1.0, 2.0, 3.0]]), axis=-1)
    assert abs(sum(t.tolist()[0]) - 1.0) < 1e-5
    t = pdefa.ops_softmax(pdefa.from_list([[1.0, 1.0], [1.0, 1.0]]), axis=0).tolist()
    assert abs(t[0][0] + t[1][0] - 1.0) < 1e-5 and abs(t[0][1] + t[1][1] - 1.0) < 1e-5
    t = pdefa.ops_softmax(pdefa.from_list([[2.0], [1.0]]), axis=0).tolist()
    assert t[0][0] > t[1][0]


def test_reductions():
    t = pdefa.from_list([[1.0, 2.0], [3.0, 4.0]])
    assert pdefa.ops_reduce_sum(t, axis=0).tolist() == [4.0, 6.0]
    assert pdefa.ops_reduce_sum(t, axis=1, keepdims=True).shape == (2, 1)
    assert pdefa.ops_reduce_mean(t, axis=0).tolist() == [2.0, 3.0]
    assert pdefa.ops_reduce_mean(pdefa.from_list([[1.0, 3.0], [2.0, 4.0]]), axis=1).tolist() == [2.0, 3.0]
    m = pdefa.from_list([[1.0, 5.0, 2.0], [3.0, 4.0, 6.0]])
    assert pdefa.ops_reduce_max(m, axis=1).tolist() == [5.0, 6.0]
    assert pdefa.ops_reduce_max(pdefa.from_list([[1.0, 5.0], [3.0, 4.0]]), axis=0).tolist() == [3.0, 5.0]
    assert pdefa.ops_argmax(pdefa.from_list([[1.0, 5.0, 2.0]]), axis=1).tolist() == [1]


def test_shape_ops():
    a = pdefa.from_list([[1.0, 2.0], [3.0, 4.0]])
    assert pdefa.ops_add(a, pdefa.from_list([[10.0, 20.0]])).tolist() == [[11.0, 22.0], [13.0, 24.0]]
    assert pdefa.ops_mul(a, 2.0).tolist() == [[2.0, 4.0], [6.0, 8.0]]
    assert pdefa.ops_reshape(pdefa.from_list([[1.0, 2.0, 3.0, 4.0]]), [2, 2]).shape == (2, 2)
    assert pdefa.ops_transpose(a, [1, 0]).tolist() == [[1.0, 3.0], [2.0, 4.0]]
    r1, r2 = pdefa.from_list([[1.0, 2.0]]), pdefa.from_list([[3.0, 4.0]])
    assert pdefa.ops_concat([r1, r2], axis=0).tolist() == [[1.0, 2.0], [3.0, 4.0]]
    assert pdefa.ops_stack([r1, r2], axis=0).shape == (2, 1, 2)
    g = pdefa.ops_gather(pdefa.from_list([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]), pdefa.from_list([2, 0]), axis=0)
    assert g.tolist() == [[5.0, 6.0], [1.0, 2.0]]


# ---------------------------------------------------------------- errors

def test_error_paths(tmp_path):
    ctx = pdefa.Context()
    with pytest.raises(pdefa.PdefaError):
        pdefa.Model(ctx, str(tmp_path / "nonexistent_model_xyz.engine"))
    with pytest.raises(pdefa.PdefaError):
        _ = pdefa.zeros(2, 3) @ pdefa.zeros(4, 5)
    with pytest.raises(pdefa.PdefaError):
        _ = pdefa.zeros(2, 3, 4) @ pdefa.zeros(4, 5)
    with pytest.raises(pdefa.PdefaError):
        pdefa.load_image(str(tmp_path / "does_not_exist.jpg"))
    with pytest.raises(pdefa.PdefaError):
        pdefa.ops_softmax(pdefa.from_list([[1.0, 2.0]]), axis=99)
    with pytest.raises(pdefa.PdefaError):
        pdefa.ops_reshape(pdefa.from_list([[1.0, 2.0, 3.0]]), [2, 2])
    with pytest.raises(pdefa.PdefaError):
        pdefa.ops_reduce_sum(pdefa.from_list([[1.0, 2.0]]), axis=99)
    with pytest.raises(pdefa.PdefaError):
        pdefa.zeros(2, 2).copy_from_list([[1.0, 2.0, 3.0]])
    for n in (0, -1):
        with pytest.raises(pdefa.PdefaError):
            pdefa.Context().set_num_threads(n)
    bad = tmp_path / "bad.engine"
    bad.write_bytes(b"XXXX" + b"\0" * 64)
    with pytest.raises(pdefa.PdefaError):
        pdefa.Model(ctx, str(bad))


def test_context_threads():
    ctx = pdefa.Context()
    ctx.set_num_threads(4)
    assert ctx.get_num_threads() == 4
    ctx.set_num_threads(8)
    assert ctx.get_num_threads() == 8


# ---------------------------------------------------------------- image / preprocess / postprocess

def test_image(cat_ppm):
    img = pdefa.load_image(cat_ppm)
    assert (img.width, img.height, img.channels) == (50, 50, 3)
    assert img.format in (0, 1, 2)
    assert len(img.tobytes()) == img.width * img.height * img.channels
    arr = img.tolist()
    assert len(arr) == 50 and len(arr[0]) == 50 and arr[0][0] == [200, 120, 40]
    assert img.numpy().shape == (50, 50, 3)


def test_letterbox(cat_ppm):
    img = pdefa.load_image(cat_ppm)
    t, meta = pdefa.preprocess_letterbox(img, 640, 640)
    assert t.shape == (1, 3, 640, 640)
    assert (meta.orig_w, meta.orig_h) == (img.width, img.height)
    assert meta.ratio > 0.0 and meta.pad_x >= 0 and meta.pad_y >= 0
    t, _ = pdefa.preprocess_letterbox(img, 64, 64, scale=1.0 / 255.0)
    a = t.to_numpy()
    assert a.min() >= 0.0 and a.max() <= 1.0 + 1e-6
    t, m = pdefa.prepare_for_engine(cat_ppm, 640, 640)
    assert t.shape == (1, 3, 640, 640) and m.orig_w > 0 and m.orig_h > 0
    assert pdefa.load_image_as_tensor(cat_ppm, 64, 32).shape == (1, 3, 32, 64)


def test_map_back(cat_ppm):
    img = pdefa.load_image(cat_ppm)
    _, meta = pdefa.preprocess_letterbox(img, 640, 640)
    b = pdefa.map_box_to_original(pdefa.Box(meta.pad_x, meta.pad_y, meta.pad_x + 100, meta.pad_y + 100), meta)
    assert 0 <= b.x1 < img.width and 0 <= b.y1 < img.height and b.x2 > b.x1 and b.y2 > b.y1
    x, y = pdefa.map_point_to_original(320.0, 320.0, meta)
    assert 0 <= x <= img.width and 0 <= y <= img.height


def test_decode_yolo_empty_and_shapes(cat_ppm):
    _, meta = pdefa.preprocess_letterbox(pdefa.load_image(cat_ppm), 640, 640)
    assert pdefa.decode_yolo(pdefa.zeros(1, 84, 8400), meta, conf_thres=0.9) == []
    with pytest.raises(pdefa.PdefaError):
        pdefa.decode_yolo([[1.0, 2.0], [3.0, 4.0]])


def test_decode_yolo_matches_reference_loop():
    """Vectorised decode against the reference's literal loop (restated in
    the oracle) on a head with overlapping boxes and a tie."""
    from oracle import decode_ref
    rng = np.random.default_rng(0)
    A = 300
    head = np.zeros((84, A), np.float32)
    head[0] = rng.uniform(100, 540, A)
    head[1] = rng.uniform(100, 540, A)
    head[2:4] = rng.uniform(20, 120, (2, A))
    head[4:] = rng.uniform(0, 0.3, (80, A)) ** 2 * 10
    head[4 + 7, 5] = head[4 + 7, 6] = 0.99
    meta = pdefa.PreprocessMeta(640, 640, 1280, 720, 0, 140, 640, 360, 0.5)
    got = pdefa.decode_yolo(head[None], meta)
    want = decode_ref.decode(head.tolist(), vars(meta))
    assert len(got) > 5
    assert [(d["cls"], d["conf"]) for d in got] == [(d["cls"], d["conf"]) for d in want]
    for a, b in zip(got, want):
        for k in ("x1", "y1", "x2", "y2"):
            assert a[k] == pytest.approx(b[k], abs=1e-9)


# ---------------------------------------------------------------- model info (no GPU needed)

def test_model_info(tiny_engine):
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, tiny_engine)
    i, o = model.input_info(0), model.output_info(0)
    assert i.shape == (1, 3, 64, 64) and isinstance(i.name, str)
    assert o.shape == (1, 4) and isinstance(o.name, str)
    assert isinstance(model.name, str)
    em = pdefa.load(tiny_engine)
    assert hasattr(em, "set_num_threads") and hasattr(em, "session")
    em.set_num_threads(2)
    assert em.ctx.get_num_threads() == 2


# ---------------------------------------------------------------- on the GPU

@pytest.mark.gpu
def test_matmul_identity():
    a = pdefa.from_list([[1.0, 2.0], [3.0, 4.0]])
    i = pdefa.from_list([[1.0, 0.0], [0.0, 1.0]])
    assert (a @ i).tolist() == [[1.0, 2.0], [3.0, 4.0]]


@pytest.mark.gpu
def test_session_runs(tiny_engine):
    from oracle import graph_ref
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, tiny_engine)
    s = pdefa.Session(ctx, model)
    s.set_input(0, pdefa.zeros(1, 3, 64, 64))
    s.run()
    out_zero = s.output(0).tolist()
    assert s.output(0).shape == (1, 4)
    s.set_input(0, pdefa.ones(1, 3, 64, 64))
    s.run()
    out1 = s.output(0).tolist()
    s.run()
    assert s.output(0).tolist() == out1
    assert out_zero != out1
    for _ in range(3):
        s.run()
    st = s.stats()
    assert st["runs"] >= 5 and st["last_run_ms"] > 0
    want = graph_ref.run_graph(ys.build_tiny(), [np.ones((1, 3, 64, 64), np.float32)])[0]
    assert np.allclose(np.array(out1), want, atol=1e-3, rtol=1e-3)


@pytest.mark.gpu
def test_large_tensors_reused_blocks():
    """Tensors of 256 KiB and up created through the C ABI live in page-locked
    memory from a pool of freed blocks: contents survive creation and reuse
    of a freed block of the same or a larger size, and a freed block handed
    to a smaller tensor keeps that tensor's own size."""
    from pdefa_amd import native
    L = native.lib()
    rng = np.random.default_rng(5)
    for shape in [(1, 3, 200, 200), (1, 3, 200, 200), (1, 3, 180, 200), (2, 3, 200, 200), (1, 3, 200, 200)]:
        a = rng.standard_normal(shape).astype(np.float32)
        h = native.tensor_from_numpy(a)
        keep = native.tensor_from_numpy(a[:, :1].copy())  # a small tensor alive across the loop
        try:
            assert np.array_equal(native.tensor_to_numpy(h), a)
            assert np.array_equal(native.tensor_to_numpy(keep), a[:, :1])
        finally:
            L.engine_tensor_destroy(h)
            L.engine_tensor_destroy(keep)


@pytest.mark.gpu
def test_batch_inference(tmp_path):
    """BatchInference (one batched GPU program per chunk) against single runs."""
    path = str(tmp_path / "y.engine")
    ys.save(ys.build_yolov8("n", seed=0, imgsz=160), path)
    paths = [write_ppm(tmp_path / f"im{i}.ppm", 60 + 10 * i, 50, (30 * i, 100, 200 - 20 * i)) for i in range(3)]
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, path)
    with pdefa.BatchInference(ctx, model, batch_size=2, num_threads=2) as batch:
        results = batch.run(paths, 160, 160)
    assert len(results) == 3
    s = pdefa.Session(ctx, model)
    for (out, meta), p in zip(results, paths):
        assert out.shape == (1, 84, 525)
        t, m = pdefa.prepare_for_engine(p, 160, 160)
        assert m == meta
        s.set_input(0, t)
        s.run()
        assert np.allclose(out.to_numpy(), s.output(0).to_numpy(), atol=1e-4, rtol=1e-4)


# ---------------------------------------------------------------- on-device letterbox (extension)

def _synthetic_images():
    rng = np.random.default_rng(21)
    return [rng.integers(0, 256, (720, 1280, 3), dtype=np.uint8),
            rng.integers(0, 256, (768, 1024, 3), dtype=np.uint8),
            rng.integers(0, 256, (800, 800), dtype=np.uint8),         # gray
            rng.integers(0, 256, (517, 333, 4), dtype=np.uint8),      # RGBA
            rng.integers(0, 256, (1, 1, 3), dtype=np.uint8),          # 1x1
            rng.integers(0, 256, (3, 2, 3), dtype=np.uint8)]


def test_image_from_array_roundtrip():
    a = np.arange(2 * 3 * 4, dtype=np.uint8).reshape(2, 3, 4)
    im = pdefa.Image.from_array(a)
    assert (im.width, im.height, im.channels) == (3, 2, 4)
    assert im.tobytes() == a.tobytes()
    g = pdefa.Image.from_array(np.full((5, 7), 9, np.uint8))
    assert (g.width, g.height, g.channels) == (7, 5, 1)
    with pytest.raises(pdefa.PdefaError):
        pdefa.Image.from_array(np.zeros((4, 4, 2), np.uint8))
    with pytest.raises(pdefa.PdefaError):
        pdefa.Image.from_array(np.zeros((0, 4, 3), np.uint8))


def test_from_array_letterbox_matches_numpy_restatement():
    """Host letterbox of an in-memory image = the numpy restatement (which
    follows imageloader/src/preprocess.cpp:15-144), bit for bit: both
    evaluate the blend in the FMA form the reference's compiled code uses."""
    img = _synthetic_images()[0]
    t, meta = pdefa.preprocess_letterbox(pdefa.Image.from_array(img), 640, 640, 1 / 255, 114 / 255)
    want, wmeta = ys.letterbox(img, 640, 640, 1 / 255, 114 / 255)
    assert (meta.pad_x, meta.pad_y, meta.scaled_w, meta.scaled_h) == (wmeta["pad_x"], wmeta["pad_y"],
                                                                       wmeta["scaled_w"], wmeta["scaled_h"])
    np.testing.assert_array_equal(t.to_numpy(), want)


def _identity_engine(tmp_path):
    """Input -> Mul by 1 -> output: the letterboxed tensor itself, exactly (the
    letterbox extrapolates past the last source pixel when it upscales, so
    values can be negative)."""
    b = ys.GraphBuilder()
    one = b.const("/id/one", np.ones(1, np.float32))
    y = b.node("Mul", "/id/Mul", [-1, one])
    path = str(tmp_path / "identity.engine")
    ys.save(b.model([1, 3, 640, 640], [1, 3, 640, 640], [y]), path)
    return path


@pytest.mark.gpu
@pytest.mark.parametrize("tw,th", [(640, 640), (320, 256)])
def test_device_letterbox_bit_exact(tmp_path, tw, th):
    """set_images (letterbox on the GPU from 8-bit pixels) equals the host
    pdefa_preprocess_letterbox bit for bit, metas included, over RGB, gray,
    RGBA, 1x1 and 3x2 images in one batch."""
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, _identity_engine(tmp_path))
    imgs = [pdefa.Image.from_array(a) for a in _synthetic_images()]
    host = [pdefa.preprocess_letterbox(im, tw, th, 1 / 255, 114 / 255) for im in imgs]
    s = pdefa.Session(ctx, model)
    metas = s.set_images(0, imgs, tw, th, 1 / 255, 114 / 255)
    s.run()
    got = s.output(0).to_numpy()
    assert got.shape == (len(imgs), 3, th, tw)
    for i, (t, m) in enumerate(host):
        assert metas[i] == m
        np.testing.assert_array_equal(got[i:i + 1], t.to_numpy())
    # set_input replaces the device letterbox input
    s.set_input(0, host[0][0])
    s.run()
    np.testing.assert_array_equal(s.output(0).to_numpy(), host[0][0].to_numpy())


@pytest.mark.gpu
def test_device_letterbox_matches_reference_fixture(tmp_path):
    """The device letterbox of the synthetic 1280x720 image (seed 0) hashes
    to the reference's pdefa_preprocess_letterbox output recorded in
    tests/golden/letterbox_1280x720.json (imageloader/src/preprocess.cpp:15-144),
    and its meta equals the recorded one."""
    import hashlib
    import json
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "letterbox_1280x720.json")) as f:
        g = json.load(f)
    raw = ys.synth_image(0, 1280, 720)
    assert hashlib.sha256(raw.tobytes()).hexdigest() == g["image_sha256"]
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, _identity_engine(tmp_path))
    s = pdefa.Session(ctx, model)
    metas = s.set_images(0, [pdefa.Image.from_array(raw)], 640, 640, 1 / 255, 114 / 255)
    s.run()
    got = np.ascontiguousarray(s.output(0).to_numpy(), np.float32)
    assert hashlib.sha256(got.tobytes()).hexdigest() == g["output_sha256"]
    for k in ("pad_x", "pad_y", "scaled_w", "scaled_h"):
        assert getattr(metas[0], k) == g["meta"][k]
    assert metas[0].ratio == np.float32(g["meta"]["ratio"])


@pytest.mark.gpu
def test_batch_inference_device_preprocess(tmp_path):
    """BatchInference with the letterbox on the GPU gives the host path's
    outputs and metas exactly."""
    path = str(tmp_path / "y.engine")
    ys.save(ys.build_yolov8("n", seed=0, imgsz=160), path)
    paths = [write_ppm(tmp_path / f"im{i}.ppm", 60 + 10 * i, 50, (30 * i, 100, 200 - 20 * i)) for i in range(3)]
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, path)
    with pdefa.BatchInference(ctx, model, batch_size=2, num_threads=2) as batch:
        host = batch.run(paths, 160, 160)
    with pdefa.BatchInference(ctx, model, batch_size=2, num_threads=2, device_preprocess=True) as batch:
        dev = batch.run(paths, 160, 160)
    for (a, ma), (b, mb) in zip(host, dev):
        assert ma == mb
        np.testing.assert_array_equal(a.to_numpy(), b.to_numpy())
