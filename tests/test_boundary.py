"""The drop-in C ABI on the host: exports, handle/error behaviour and the
host-side helpers, mirroring the reference's own Python tests
(pdefa/tests/test_smoke.py, test_tensor*.py, test_ops*.py, test_errors*.py).
No GPU is touched here."""
import ctypes as C
import re
import subprocess

import numpy as np
import pytest

from pdefa_amd import engine_format as ef
from pdefa_amd import native, yolo_synth as ys

# The 77 names of pdefa/pdefa.def:3-96.
PDEFA_DEF = """
pdefa_version pdefa_last_error pdefa_image_load pdefa_image_free pdefa_image_width pdefa_image_height
pdefa_image_channels pdefa_image_format pdefa_image_pixels pdefa_preprocess_letterbox pdefa_prepare_for_engine
pdefa_load_image_as_tensor pdefa_map_box_to_original pdefa_map_point_to_original engine_version engine_last_error
engine_status_string engine_dtype_size engine_simd_level engine_cpu_brand engine_context_create
engine_context_destroy engine_context_set_num_threads engine_context_get_num_threads
engine_context_num_physical_cores engine_context_has_avx2 engine_context_has_avx512 engine_tensor_create
engine_tensor_create_from_data engine_tensor_data engine_tensor_shape engine_tensor_copy_from engine_tensor_copy_to
engine_tensor_numel engine_tensor_dtype engine_tensor_rank engine_tensor_destroy engine_model_load
engine_model_input_count engine_model_output_count engine_model_name engine_model_destroy engine_session_create
engine_session_set_input engine_session_run engine_session_get_output engine_session_destroy engine_run_simple
engine_model_input_info engine_model_output_info engine_session_get_stats engine_session_set_profile_callback
engine_session_clear_profile_callback engine_session_debug_intermediate engine_ops_matmul engine_ops_relu
engine_ops_silu engine_ops_add engine_ops_sub engine_ops_mul engine_ops_div engine_ops_sigmoid engine_ops_tanh
engine_ops_gelu engine_ops_clip engine_ops_softmax engine_ops_reduce_max engine_ops_reduce_sum
engine_ops_reduce_mean engine_ops_argmax engine_ops_gather engine_ops_reshape engine_ops_transpose
engine_ops_concat engine_ops_stack engine_random_randn engine_random_rand
""".split()

EXTENSIONS = ["pdefa_amd_session_replay", "pdefa_amd_session_step_times", "pdefa_amd_session_step_repeat",
              "pdefa_amd_session_plan", "pdefa_amd_session_set_images", "pdefa_amd_image_from_pixels",
              "pdefa_amd_session_decode",
              "pdefa_amd_plan_model", "pdefa_amd_device_name", "pdefa_amd_tune_stats", "pdefa_amd_pack_cache_stats",
              "pdefa_amd_ops_matmul_noalloc", "pdefa_amd_session_read_conv_input"]


def test_def_list_complete():
    assert len(PDEFA_DEF) == 77 and len(set(PDEFA_DEF)) == 77


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", native.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = set(PDEFA_DEF + EXTENSIONS) - exported
    assert not missing, missing
    # nothing else leaks: every exported function is declared in include/*.h
    assert exported == set(PDEFA_DEF + EXTENSIONS), sorted(exported - set(PDEFA_DEF + EXTENSIONS))


def test_headers_declare_every_symbol():
    import glob
    import os
    text = "".join(open(p).read() for p in glob.glob(os.path.join(native.HERE, "..", "include", "*.h")))
    for name in PDEFA_DEF + EXTENSIONS:
        assert re.search(r"\b" + name + r"\s*\(", text), name


def L():
    return native.lib()


def test_meta():
    lib = L()
    assert re.fullmatch(r"\d+\.\d+\.\d+", lib.engine_version().decode())
    assert lib.engine_simd_level().decode() in ("AVX2", "AVX-512", "scalar")
    assert len(lib.engine_cpu_brand().decode()) > 0
    lib.engine_status_string.restype = C.c_char_p
    assert lib.engine_status_string(7) == b"invalid argument"
    lib.engine_dtype_size.restype = C.c_size_t
    assert [lib.engine_dtype_size(d) for d in range(8)] == [4, 2, 2, 1, 1, 4, 8, 1]


def test_context_threads():
    lib = L()
    ctx = C.c_void_p()
    assert lib.engine_context_create(C.byref(ctx)) == 0
    assert lib.engine_context_get_num_threads(ctx) >= 1
    assert lib.engine_context_set_num_threads(ctx, 3) == 0
    assert lib.engine_context_get_num_threads(ctx) == 3
    assert lib.engine_context_set_num_threads(ctx, 0) == 7
    assert lib.engine_context_set_num_threads(ctx, -1) == 7
    lib.engine_context_destroy(ctx)
    assert lib.engine_context_create(None) == 1


def test_tensor_roundtrip_and_errors():
    lib = L()
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    h = native.tensor_from_numpy(a)
    np.testing.assert_array_equal(native.tensor_to_numpy(h), a)
    lib.engine_tensor_numel.restype = C.c_int64
    lib.engine_tensor_numel.argtypes = [C.c_void_p]
    assert lib.engine_tensor_numel(h) == 12
    lib.engine_tensor_copy_from.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    too_big = np.zeros(13, np.float32)
    assert lib.engine_tensor_copy_from(h, too_big.ctypes.data, too_big.nbytes) == 7
    lib.engine_tensor_destroy(h)
    # data larger than the shape -> INVALID_ARG (engine_api.cpp:482-486)
    shape = (C.c_int64 * 1)(2)
    out = C.c_void_p()
    data = np.zeros(3, np.float32)
    assert lib.engine_tensor_create_from_data(C.byref(out), shape, 1, 0, data.ctypes.data, data.nbytes) == 7
    assert lib.engine_tensor_create_from_data(None, shape, 1, 0, data.ctypes.data, data.nbytes) == 1
    # a stale handle is rejected, not dereferenced
    assert lib.engine_tensor_shape(C.c_void_p(0), None, None) == 2


def _binary(fn, a, b):
    out = C.c_void_p()
    getattr(L(), fn).argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]
    rc = getattr(L(), fn)(native.tensor_from_numpy(a), native.tensor_from_numpy(b), C.byref(out))
    return rc, (native.tensor_to_numpy(out) if rc == 0 else None)


def test_host_binary_ops_broadcast():
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.array([10, 20, 30], np.float32)
    for fn, ref in (("engine_ops_add", a + b), ("engine_ops_sub", a - b), ("engine_ops_mul", a * b),
                    ("engine_ops_div", a / b)):
        rc, got = _binary(fn, a, b)
        assert rc == 0
        np.testing.assert_allclose(got, ref, rtol=1e-6)
    rc, _ = _binary("engine_ops_add", a, np.zeros((4,), np.float32))
    assert rc == 6  # INVALID_SHAPE


def _unary(fn, a):
    h = native.tensor_from_numpy(a)
    getattr(L(), fn).argtypes = [C.c_void_p]
    assert getattr(L(), fn)(h) == 0
    return native.tensor_to_numpy(h)


def test_host_unary_kats():
    assert abs(_unary("engine_ops_silu", np.array([[1.0]], np.float32))[0, 0] - 0.7311) < 1e-3
    assert abs(_unary("engine_ops_gelu", np.array([[1.0]], np.float32))[0, 0] - 0.8413) < 1e-3
    assert _unary("engine_ops_sigmoid", np.array([[0.0]], np.float32))[0, 0] == 0.5
    assert _unary("engine_ops_relu", np.array([[-2.0, 3.0]], np.float32)).tolist() == [[0.0, 3.0]]
    s = _unary_axis("engine_ops_softmax", np.ones((2, 2), np.float32), 0)
    np.testing.assert_allclose(s.sum(0), [1.0, 1.0], rtol=1e-6)


def _unary_axis(fn, a, axis):
    h = native.tensor_from_numpy(a)
    getattr(L(), fn).argtypes = [C.c_void_p, C.c_int32]
    rc = getattr(L(), fn)(h, axis)
    return native.tensor_to_numpy(h) if rc == 0 else rc


def test_softmax_bad_axis():
    assert _unary_axis("engine_ops_softmax", np.ones((2, 2), np.float32), 99) == 7


def test_reduce_argmax_gather():
    lib = L()
    a = np.array([[1.0, 5.0, 2.0], [3.0, 4.0, 6.0]], np.float32)
    for fn, ref in (("engine_ops_reduce_max", a.max(1)), ("engine_ops_reduce_sum", a.sum(1)),
                    ("engine_ops_reduce_mean", a.mean(1))):
        getattr(lib, fn).argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_void_p)]
        out = C.c_void_p()
        assert getattr(lib, fn)(native.tensor_from_numpy(a), 1, 0, C.byref(out)) == 0
        np.testing.assert_allclose(native.tensor_to_numpy(out), ref, rtol=1e-6)
    lib.engine_ops_argmax.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_void_p)]
    out = C.c_void_p()
    assert lib.engine_ops_argmax(native.tensor_from_numpy(a), 1, 0, C.byref(out)) == 0
    assert native.tensor_to_numpy(out).tolist() == [1, 2]
    lib.engine_ops_gather.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.POINTER(C.c_void_p)]
    idx = native.tensor_from_numpy(np.array([2, 0], np.float32))
    out = C.c_void_p()
    src = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], np.float32)
    assert lib.engine_ops_gather(native.tensor_from_numpy(src), idx, 0, C.byref(out)) == 0
    assert native.tensor_to_numpy(out).tolist() == [[5.0, 6.0], [1.0, 2.0]]


def test_shape_ops():
    lib = L()
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    lib.engine_ops_transpose.argtypes = [C.c_void_p, C.POINTER(C.c_int32), C.c_int32, C.POINTER(C.c_void_p)]
    out = C.c_void_p()
    perm = (C.c_int32 * 3)(2, 0, 1)
    assert lib.engine_ops_transpose(native.tensor_from_numpy(a), perm, 3, C.byref(out)) == 0
    np.testing.assert_array_equal(native.tensor_to_numpy(out), a.transpose(2, 0, 1))
    lib.engine_ops_reshape.argtypes = [C.c_void_p, C.POINTER(C.c_int64), C.c_int32, C.POINTER(C.c_void_p)]
    shp = (C.c_int64 * 2)(-1, 6)
    assert lib.engine_ops_reshape(native.tensor_from_numpy(a), shp, 2, C.byref(out)) == 0
    assert native.tensor_to_numpy(out).shape == (4, 6)
    shp = (C.c_int64 * 2)(5, 5)
    assert lib.engine_ops_reshape(native.tensor_from_numpy(a), shp, 2, C.byref(out)) == 6
    hs = (C.c_void_p * 2)(native.tensor_from_numpy(a), native.tensor_from_numpy(a + 1))
    lib.engine_ops_concat.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_void_p)]
    assert lib.engine_ops_concat(hs, 2, 1, C.byref(out)) == 0
    np.testing.assert_array_equal(native.tensor_to_numpy(out), np.concatenate([a, a + 1], 1))
    lib.engine_ops_stack.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_void_p)]
    assert lib.engine_ops_stack(hs, 2, 1, C.byref(out)) == 0
    np.testing.assert_array_equal(native.tensor_to_numpy(out), np.stack([a, a + 1], 1))


def test_random_determinism():
    lib = L()
    lib.engine_random_randn.argtypes = [C.POINTER(C.c_int64), C.c_int32, C.c_uint64, C.POINTER(C.c_void_p)]
    lib.engine_random_rand.argtypes = [C.POINTER(C.c_int64), C.c_int32, C.c_uint64, C.POINTER(C.c_void_p)]
    shp = (C.c_int64 * 2)(3, 5)
    vals = []
    for seed in (7, 7, 8):
        out = C.c_void_p()
        assert lib.engine_random_randn(shp, 2, seed, C.byref(out)) == 0
        vals.append(native.tensor_to_numpy(out))
    np.testing.assert_array_equal(vals[0], vals[1])
    assert not np.array_equal(vals[0], vals[2])
    out = C.c_void_p()
    assert lib.engine_random_rand(shp, 2, 1, C.byref(out)) == 0
    u = native.tensor_to_numpy(out)
    assert u.min() >= 0.0 and u.max() < 1.0


def test_model_load_errors(tmp_path):
    lib = L()
    ctx = C.c_void_p()
    lib.engine_context_create(C.byref(ctx))
    m = C.c_void_p()
    assert lib.engine_model_load(ctx, str(tmp_path / "missing.engine").encode(), C.byref(m)) == 5
    assert b"failed to load" in lib.pdefa_last_error()
    bad = tmp_path / "bad.engine"
    bad.write_bytes(b"NOPE" + bytes(100))
    assert lib.engine_model_load(ctx, str(bad).encode(), C.byref(m)) == 5
    assert lib.engine_model_load(ctx, None, C.byref(m)) == 1
    lib.engine_context_destroy(ctx)


def test_model_info_v2_and_v1_defaults(tmp_path):
    lib = L()
    model, _ = ys.build_single_conv(8, 16, 3, 1, 12)
    for version in (2, 1):
        model.version = version
        path = str(tmp_path / f"m{version}.engine")
        ef.write_engine(path, model)
        ctx = C.c_void_p()
        lib.engine_context_create(C.byref(ctx))
        m = C.c_void_p()
        assert lib.engine_model_load(ctx, path.encode(), C.byref(m)) == 0
        name = C.c_char_p()
        shape = (C.c_int64 * 8)()
        nd = C.c_int32()
        dt = C.c_int()
        lib.engine_model_input_info.argtypes = [C.c_void_p, C.c_int32, C.POINTER(C.c_char_p),
                                                C.POINTER(C.c_int64), C.POINTER(C.c_int32), C.POINTER(C.c_int)]
        assert lib.engine_model_input_info(m, 0, C.byref(name), shape, C.byref(nd), C.byref(dt)) == 0
        got = [shape[i] for i in range(nd.value)]
        if version == 2:
            assert (name.value, got) == (b"images", [1, 8, 12, 12])
        else:
            assert (name.value, got) == (b"input_0", [1, 3, 640, 640])
        assert lib.engine_model_input_info(m, 5, None, None, None, None) == 7
        lib.engine_model_destroy(m)
        lib.engine_context_destroy(ctx)


def test_engine_file_roundtrip_and_reference_parse(tmp_path):
    model = ys.build_yolov8("n", seed=0, imgsz=160)
    path = str(tmp_path / "y.engine")
    ef.write_engine(path, model)
    back = ef.read_engine(path)
    assert len(back.nodes) == len(model.nodes) and len(back.weights) == len(model.weights)
    for a, b in zip(model.weights, back.weights):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(model.nodes, back.nodes):
        assert (a.op, a.name, a.inputs, a.outputs) == (b.op, b.name, b.inputs, b.outputs)
        for k, v in a.params.items():
            assert b.params[k] == pytest.approx(v)
    from oracle import ref_lib
    if ref_lib.available():
        r = ref_lib.RefSession(path)  # the reference loader parses the same bytes
        r.close()


@pytest.mark.parametrize("a_shape,b_shape,out_shape", [
    ((4, 5), (6, 3), (4, 3)),          # inner dimensions differ
    ((4, 5), (5, 3), (4, 4)),          # out has the wrong shape
    ((4, 5), (5, 3), (12,)),           # out is 1-D
    ((2, 4, 5), (2, 6, 3), (2, 4, 3)),  # batched, inner dimensions differ
    ((2, 4, 5), (5, 3), (4, 3)),       # batched, out too small for the batch
])
def test_matmul_shape_mismatch_is_a_silent_no_op(a_shape, b_shape, out_shape):
    """engine_ops_matmul with mismatched shapes returns ENGINE_OK and leaves
    `out` untouched (PDEFA1.0/src/ops/matmul.cpp:59-66,113-126); the checks
    come before any device work, so this runs without a GPU."""
    rng = np.random.default_rng(1)
    a = rng.standard_normal(a_shape).astype(np.float32)
    b = rng.standard_normal(b_shape).astype(np.float32)
    sentinel = np.full(out_shape, -7.25, np.float32)
    got = native.matmul_into(a, b, sentinel)
    np.testing.assert_array_equal(got, sentinel)
