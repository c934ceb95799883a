"""The reference's Python API over the MI355X build's C ABI.

Same names, argument meaning and error behaviour as the reference package
(pdefa/python/src/pdefa/__init__.py:41-138, _bindings.py, batch.py), so code
written against `import pdefa` runs with `from pdefa_amd import pdefa`:

    ctx = pdefa.Context()
    model = pdefa.Model(ctx, "yolov8n.engine")
    session = pdefa.Session(ctx, model)
    tensor, meta = pdefa.prepare_for_engine("image.ppm", 640, 640)
    session.set_input(0, tensor)
    session.run()                         # one hipGraph launch on the GPU
    boxes = pdefa.decode_yolo(session.output(0), meta)

Every call goes through libpdefa_native.so; a non-OK status raises
PdefaError carrying pdefa_last_error() (_bindings.py:476-486).  Tensors are
host tensors owned by the library, as in the reference; session outputs are
borrowed views of the session's pinned output buffer, valid until the next
run.  Nothing here computes on the CPU in place of the library: a model run
needs the HIP device and fails with PdefaError without one.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

from . import native
from .postprocess import decode_yolo as _decode_heads

__version__ = "1.0.3"
__license__ = "AGPL-3.0-or-later"

_F32, _I8, _U8, _I32, _I64 = 0, 3, 4, 5, 6
_CTYPE = {_I32: C.c_int32, _I64: C.c_int64, _I8: C.c_int8, _U8: C.c_uint8}


class _PreConfig(C.Structure):
    # PdefaPreprocessConfig (pdefa_c_api.h:49-54)
    _fields_ = [("target_w", C.c_int32), ("target_h", C.c_int32), ("scale", C.c_float), ("pad_value", C.c_float)]


class _PreMeta(C.Structure):
    # PdefaPreprocessMeta (pdefa_c_api.h:56-62)
    _fields_ = [("target_w", C.c_int32), ("target_h", C.c_int32), ("orig_w", C.c_int32), ("orig_h", C.c_int32),
                ("pad_x", C.c_int32), ("pad_y", C.c_int32), ("scaled_w", C.c_int32), ("scaled_h", C.c_int32),
                ("ratio", C.c_float)]


class _SessionStats(C.Structure):
    # EngineSessionStats (engine_c_api.h:126-131)
    _fields_ = [("last_run_ms", C.c_double), ("runs", C.c_uint64)]


_lib_cache: Optional[C.CDLL] = None


def _lib() -> C.CDLL:
    """libpdefa_native.so with the signatures this module calls."""
    global _lib_cache
    if _lib_cache is not None:
        return _lib_cache
    L = native.lib()
    vp, i32, i64, f32, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_size_t
    pvp, st = C.POINTER(C.c_void_p), C.c_int
    sig = {
        "pdefa_version": (C.c_char_p, []),
        "pdefa_last_error": (C.c_char_p, []),
        "engine_simd_level": (C.c_char_p, []),
        "engine_cpu_brand": (C.c_char_p, []),
        "engine_context_create": (st, [pvp]),
        "engine_context_destroy": (None, [vp]),
        "engine_context_set_num_threads": (st, [vp, i32]),
        "engine_context_get_num_threads": (i32, [vp]),
        "engine_tensor_create": (st, [pvp, C.POINTER(i64), i32, C.c_int]),
        "engine_tensor_destroy": (None, [vp]),
        "engine_tensor_numel": (i64, [vp]),
        "engine_tensor_rank": (i32, [vp]),
        "engine_tensor_shape": (st, [vp, C.POINTER(i64), C.POINTER(i32)]),
        "engine_tensor_data": (st, [vp, pvp, C.POINTER(sz)]),
        "engine_tensor_dtype": (C.c_int, [vp]),
        "engine_tensor_copy_from": (st, [vp, vp, sz]),
        "engine_model_load": (st, [vp, C.c_char_p, pvp]),
        "engine_model_destroy": (None, [vp]),
        "engine_model_name": (st, [vp, C.POINTER(C.c_char_p)]),
        "engine_model_input_info": (st, [vp, i32, C.POINTER(C.c_char_p), C.POINTER(i64), C.POINTER(i32),
                                         C.POINTER(C.c_int)]),
        "engine_model_output_info": (st, [vp, i32, C.POINTER(C.c_char_p), C.POINTER(i64), C.POINTER(i32),
                                          C.POINTER(C.c_int)]),
        "engine_session_create": (st, [vp, vp, pvp]),
        "engine_session_destroy": (None, [vp]),
        "engine_session_set_input": (st, [vp, i32, vp]),
        "engine_session_run": (st, [vp]),
        "engine_session_get_output": (st, [vp, i32, pvp]),
        "engine_session_get_stats": (st, [vp, C.POINTER(_SessionStats)]),
        "engine_session_debug_intermediate": (st, [vp, i32, pvp]),
        "engine_ops_matmul": (st, [vp, vp, vp]),
        "engine_ops_relu": (st, [vp]),
        "engine_ops_silu": (st, [vp]),
        "engine_ops_sigmoid": (st, [vp]),
        "engine_ops_tanh": (st, [vp]),
        "engine_ops_gelu": (st, [vp]),
        "engine_ops_clip": (st, [vp, f32, f32]),
        "engine_ops_softmax": (st, [vp, i32]),
        "engine_ops_argmax": (st, [vp, i32, i32, pvp]),
        "engine_ops_gather": (st, [vp, vp, i32, pvp]),
        "engine_ops_reshape": (st, [vp, C.POINTER(i64), i32, pvp]),
        "engine_ops_transpose": (st, [vp, C.POINTER(i32), i32, pvp]),
        "engine_ops_concat": (st, [pvp, i32, i32, pvp]),
        "engine_ops_stack": (st, [pvp, i32, i32, pvp]),
        "engine_random_randn": (st, [C.POINTER(i64), i32, C.c_uint64, pvp]),
        "engine_random_rand": (st, [C.POINTER(i64), i32, C.c_uint64, pvp]),
        "pdefa_image_load": (vp, [C.c_char_p]),
        "pdefa_image_free": (None, [vp]),
        "pdefa_image_width": (i32, [vp]),
        "pdefa_image_height": (i32, [vp]),
        "pdefa_image_channels": (i32, [vp]),
        "pdefa_image_format": (i32, [vp]),
        "pdefa_image_pixels": (C.POINTER(C.c_uint8), [vp, C.POINTER(sz)]),
        "pdefa_preprocess_letterbox": (st, [vp, C.POINTER(_PreConfig), pvp, C.POINTER(_PreMeta)]),
        "pdefa_prepare_for_engine": (st, [C.c_char_p, i32, i32, f32, f32, pvp, C.POINTER(_PreMeta)]),
        "pdefa_load_image_as_tensor": (st, [C.c_char_p, i32, i32, pvp]),
        "pdefa_map_box_to_original": (st, [C.POINTER(f32), C.POINTER(_PreMeta), C.POINTER(f32)]),
        "pdefa_map_point_to_original": (st, [C.POINTER(f32), C.POINTER(f32), C.POINTER(_PreMeta)]),
        # extensions (include/pdefa_amd_ext.h)
        "pdefa_amd_image_from_pixels": (vp, [C.POINTER(C.c_uint8), i32, i32, i32]),
        "pdefa_amd_session_set_images": (st, [vp, i32, i32, pvp, C.POINTER(_PreConfig), C.POINTER(_PreMeta)]),
        "pdefa_amd_session_decode": (st, [vp, i32, C.POINTER(_PreMeta), i32, C.c_double, C.c_double, i32,
                                          C.POINTER(_Detection), C.POINTER(i32)]),
    }
    for name in ("add", "sub", "mul", "div"):
        sig[f"engine_ops_{name}"] = (st, [vp, vp, pvp])
    for name in ("max", "sum", "mean"):
        sig[f"engine_ops_reduce_{name}"] = (st, [vp, i32, i32, pvp])
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _lib_cache = L
    return L


class _Detection(C.Structure):
    # PdefaAmdDetection (include/pdefa_amd_ext.h)
    _fields_ = [("x1", C.c_double), ("y1", C.c_double), ("x2", C.c_double), ("y2", C.c_double),
                ("conf", C.c_double), ("cls", C.c_int32), ("anchor", C.c_int32)]


class PdefaError(RuntimeError):
    """Any failed call into the library (_bindings.py:476-486)."""


def _check(rc: int, where: str = "") -> None:
    if rc != 0:
        raw = _lib().pdefa_last_error()
        msg = raw.decode("utf-8", "replace") if raw else "unknown"
        raise PdefaError(f"{where}: {msg}" if where else msg)


def _i64s(vals) -> C.Array:
    vals = [int(v) for v in vals]
    return (C.c_int64 * max(1, len(vals)))(*vals)


def _shape_args(shape) -> tuple:
    if len(shape) == 1 and isinstance(shape[0], (list, tuple)):
        return tuple(shape[0])
    return tuple(shape)


# ---------------------------------------------------------------- meta

def version() -> str:
    return _lib().pdefa_version().decode()


def simd_level() -> str:
    return _lib().engine_simd_level().decode()


def cpu_brand() -> str:
    return _lib().engine_cpu_brand().decode()


@dataclass
class PreprocessMeta:
    target_w: int = 0
    target_h: int = 0
    orig_w: int = 0
    orig_h: int = 0
    pad_x: int = 0
    pad_y: int = 0
    scaled_w: int = 0
    scaled_h: int = 0
    ratio: float = 1.0

    @classmethod
    def from_c(cls, c: _PreMeta) -> "PreprocessMeta":
        return cls(*(getattr(c, f) for f, _ in _PreMeta._fields_[:8]), float(c.ratio))

    def to_c(self) -> _PreMeta:
        return _PreMeta(self.target_w, self.target_h, self.orig_w, self.orig_h, self.pad_x, self.pad_y,
                        self.scaled_w, self.scaled_h, self.ratio)


@dataclass
class Box:
    x1: float
    y1: float
    x2: float
    y2: float


@dataclass
class TensorInfo:
    name: str
    shape: tuple
    dtype: int


# ---------------------------------------------------------------- tensors

def _nest(flat: list, shape: Sequence[int]):
    if len(shape) == 0:
        return flat[0] if flat else None
    if len(shape) == 1:
        return list(flat)
    step = math.prod(shape[1:])
    if step == 0:
        return []
    return [_nest(flat[i * step:(i + 1) * step], shape[1:]) for i in range(shape[0])]


def _flatten(data) -> Tuple[list, list]:
    """Nested list -> (flat values, shape); the shape follows first elements."""
    if not isinstance(data, (list, tuple)):
        return [data], []
    shape, cur = [], data
    while isinstance(cur, (list, tuple)):
        shape.append(len(cur))
        if not cur:
            break
        cur = cur[0]
    flat: list = []

    def walk(x, depth):
        if depth == len(shape):
            flat.append(x)
        else:
            for v in x:
                walk(v, depth + 1)

    walk(data, 0)
    return flat, shape


class Tensor:
    """A library-owned host tensor (owns=False: a borrowed view, not freed)."""

    def __init__(self, handle, owns: bool = True):
        self._owns = owns
        self._handle = handle if isinstance(handle, C.c_void_p) else C.c_void_p(handle)

    def __del__(self):
        try:
            if self._owns and self._handle and self._handle.value:
                _lib().engine_tensor_destroy(self._handle)
        except Exception:
            pass

    @property
    def raw(self):
        return self._handle

    @property
    def numel(self) -> int:
        return int(_lib().engine_tensor_numel(self._handle))

    @property
    def ndim(self) -> int:
        return int(_lib().engine_tensor_rank(self._handle))

    @property
    def dtype(self) -> int:
        return int(_lib().engine_tensor_dtype(self._handle))

    @property
    def shape(self) -> tuple:
        n = self.ndim
        if n <= 0:
            return ()
        dims, got = (C.c_int64 * n)(), C.c_int32(0)
        _check(_lib().engine_tensor_shape(self._handle, dims, C.byref(got)), "tensor_shape")
        return tuple(int(dims[i]) for i in range(got.value))

    def _data(self) -> Tuple[int, int]:
        ptr, size = C.c_void_p(), C.c_size_t()
        _check(_lib().engine_tensor_data(self._handle, C.byref(ptr), C.byref(size)), "tensor_data")
        return ptr.value or 0, size.value

    def tolist(self):
        addr, nbytes = self._data()
        ct = _CTYPE.get(self.dtype, C.c_float)
        n = nbytes // C.sizeof(ct)
        flat = list((ct * n).from_address(addr)) if n else []
        return _nest(flat, self.shape)

    def to_numpy(self):
        import numpy as np
        addr, nbytes = self._data()
        np_dt = {_I32: np.int32, _I64: np.int64, _I8: np.int8, _U8: np.uint8}.get(self.dtype, np.float32)
        buf = (C.c_uint8 * nbytes).from_address(addr) if nbytes else b""
        return np.frombuffer(bytes(buf), dtype=np_dt).reshape(self.shape)

    numpy = to_numpy

    def _write(self, values: Sequence[float]) -> None:
        arr = (C.c_float * max(1, len(values)))(*values)
        _check(_lib().engine_tensor_copy_from(self._handle, arr, len(values) * 4), "tensor_copy_from")

    def fill(self, value: float) -> "Tensor":
        self._write([float(value)] * self.numel)
        return self

    def copy_from_list(self, data) -> "Tensor":
        flat, shape = _flatten(data)
        if tuple(shape) != self.shape:
            raise PdefaError(f"shape mismatch: {tuple(shape)} != {self.shape}")
        self._write([float(v) for v in flat])
        return self

    def __add__(self, other):
        return ops_add(self, other)

    def __sub__(self, other):
        return ops_sub(self, other)

    def __mul__(self, other):
        return ops_mul(self, other)

    def __truediv__(self, other):
        return ops_div(self, other)

    def __neg__(self):
        return ops_mul(self, -1.0)

    def __matmul__(self, other):
        if not isinstance(other, Tensor):
            raise TypeError("matmul requires Tensor")
        return ops_matmul(self, other)

    def __repr__(self):
        return f"<Tensor shape={self.shape} numel={self.numel}>"


def tensor_empty(shape, dtype: int = _F32) -> Tensor:
    h = C.c_void_p()
    _check(_lib().engine_tensor_create(C.byref(h), _i64s(shape), len(shape), int(dtype)), "tensor_create")
    return Tensor(h)


def _scalar(v: float) -> Tensor:
    t = tensor_empty([1])
    t._write([float(v)])
    return t


def empty(*shape) -> Tensor:
    return tensor_empty(list(_shape_args(shape)))


def zeros(*shape) -> Tensor:
    return empty(*shape).fill(0.0)


def ones(*shape) -> Tensor:
    return empty(*shape).fill(1.0)


def from_list(data) -> Tensor:
    flat, shape = _flatten(data)
    t = tensor_empty(shape)
    t._write([float(v) for v in flat])
    return t


def random_randn(shape, seed: int = 0) -> Tensor:
    h = C.c_void_p()
    _check(_lib().engine_random_randn(_i64s(shape), len(shape), int(seed), C.byref(h)), "random_randn")
    return Tensor(h)


def random_rand(shape, seed: int = 0) -> Tensor:
    h = C.c_void_p()
    _check(_lib().engine_random_rand(_i64s(shape), len(shape), int(seed), C.byref(h)), "random_rand")
    return Tensor(h)


def randn(*shape, seed: int = 0) -> Tensor:
    return random_randn(list(_shape_args(shape)), seed)


def rand(*shape, seed: int = 0) -> Tensor:
    return random_rand(list(_shape_args(shape)), seed)


# ---------------------------------------------------------------- ops

def _binary(a, b, name: str) -> Tensor:
    a = a if isinstance(a, Tensor) else _scalar(float(a))
    b = b if isinstance(b, Tensor) else _scalar(float(b))
    h = C.c_void_p()
    _check(getattr(_lib(), f"engine_ops_{name}")(a.raw, b.raw, C.byref(h)), f"ops_{name}")
    return Tensor(h)


def ops_add(a, b) -> Tensor:
    return _binary(a, b, "add")


def ops_sub(a, b) -> Tensor:
    return _binary(a, b, "sub")


def ops_mul(a, b) -> Tensor:
    return _binary(a, b, "mul")


def ops_div(a, b) -> Tensor:
    return _binary(a, b, "div")


def ops_matmul(a: Tensor, b: Tensor, out: Optional[Tensor] = None) -> Tensor:
    """C = A @ B for 2-D F32 tensors, computed on the GPU (MFMA SGEMM).  The
    C entry point ignores mismatched shapes (matmul.cpp:119-126), so they are
    rejected here, as the reference's wrapper does (_bindings.py:1005-1017)."""
    if out is None:
        sa, sb = a.shape, b.shape
        if len(sa) != 2 or len(sb) != 2:
            raise PdefaError("ops_matmul: 2D tensors required")
        if sa[1] != sb[0]:
            raise PdefaError(f"ops_matmul: inner dims mismatch {sa} @ {sb}")
        out = tensor_empty([sa[0], sb[1]])
    _check(_lib().engine_ops_matmul(a.raw, b.raw, out.raw), "ops_matmul")
    return out


def _inplace(name: str, t: Tensor, *args) -> Tensor:
    _check(getattr(_lib(), f"engine_ops_{name}")(t.raw, *args), f"ops_{name}")
    return t


def ops_relu(t: Tensor) -> Tensor:
    return _inplace("relu", t)


def ops_silu(t: Tensor) -> Tensor:
    return _inplace("silu", t)


def ops_sigmoid(t: Tensor) -> Tensor:
    return _inplace("sigmoid", t)


def ops_tanh(t: Tensor) -> Tensor:
    return _inplace("tanh", t)


def ops_gelu(t: Tensor) -> Tensor:
    return _inplace("gelu", t)


def ops_clip(t: Tensor, lo: float, hi: float) -> Tensor:
    return _inplace("clip", t, float(lo), float(hi))


def ops_softmax(t: Tensor, axis: int = -1) -> Tensor:
    return _inplace("softmax", t, int(axis))


def _reduce(name: str, a: Tensor, axis: int, keepdims: bool) -> Tensor:
    h = C.c_void_p()
    _check(getattr(_lib(), f"engine_ops_{name}")(a.raw, int(axis), int(bool(keepdims)), C.byref(h)), f"ops_{name}")
    return Tensor(h)


def ops_reduce_max(a: Tensor, axis: int = -1, keepdims: bool = False) -> Tensor:
    return _reduce("reduce_max", a, axis, keepdims)


def ops_reduce_sum(a: Tensor, axis: int = -1, keepdims: bool = False) -> Tensor:
    return _reduce("reduce_sum", a, axis, keepdims)


def ops_reduce_mean(a: Tensor, axis: int = -1, keepdims: bool = False) -> Tensor:
    return _reduce("reduce_mean", a, axis, keepdims)


def ops_argmax(a: Tensor, axis: int = -1, keepdims: bool = False) -> Tensor:
    return _reduce("argmax", a, axis, keepdims)


def ops_gather(a: Tensor, indices: Tensor, axis: int = 0) -> Tensor:
    h = C.c_void_p()
    _check(_lib().engine_ops_gather(a.raw, indices.raw, int(axis), C.byref(h)), "ops_gather")
    return Tensor(h)


def ops_reshape(a: Tensor, shape) -> Tensor:
    h = C.c_void_p()
    _check(_lib().engine_ops_reshape(a.raw, _i64s(shape), len(shape), C.byref(h)), "ops_reshape")
    return Tensor(h)


def ops_transpose(a: Tensor, perm) -> Tensor:
    arr = (C.c_int32 * max(1, len(perm)))(*[int(p) for p in perm])
    h = C.c_void_p()
    _check(_lib().engine_ops_transpose(a.raw, arr, len(perm), C.byref(h)), "ops_transpose")
    return Tensor(h)


def _tensor_list(name: str, inputs, axis: int) -> Tensor:
    arr = (C.c_void_p * max(1, len(inputs)))(*[t.raw.value for t in inputs])
    h = C.c_void_p()
    _check(getattr(_lib(), f"engine_ops_{name}")(arr, len(inputs), int(axis), C.byref(h)), f"ops_{name}")
    return Tensor(h)


def ops_concat(inputs, axis: int = 0) -> Tensor:
    return _tensor_list("concat", inputs, axis)


def ops_stack(inputs, axis: int = 0) -> Tensor:
    return _tensor_list("stack", inputs, axis)


# ---------------------------------------------------------------- images

class Image:
    """A decoded image owned by the library (HWC uint8)."""

    def __init__(self, handle):
        self._handle = handle if isinstance(handle, C.c_void_p) else C.c_void_p(handle)

    def __del__(self):
        try:
            if self._handle and self._handle.value:
                _lib().pdefa_image_free(self._handle)
        except Exception:
            pass

    @classmethod
    def from_array(cls, arr) -> "Image":
        """An image holding a copy of an HxW or HxWxC (C = 1, 3, 4) uint8 array
        (extension: the reference builds images only from files)."""
        import numpy as np
        a = np.ascontiguousarray(arr, dtype=np.uint8)
        if a.ndim == 2:
            a = a[:, :, None]
        if a.ndim != 3 or a.shape[2] not in (1, 3, 4) or a.shape[0] == 0 or a.shape[1] == 0:
            raise PdefaError(f"from_array: expected HxW or HxWxC (C = 1, 3, 4) uint8, got shape {a.shape}")
        h = _lib().pdefa_amd_image_from_pixels(a.ctypes.data_as(C.POINTER(C.c_uint8)), a.shape[1], a.shape[0],
                                               a.shape[2])
        if not h:
            raw = _lib().pdefa_last_error()
            raise PdefaError(f"from_array: {raw.decode('utf-8', 'replace') if raw else 'unknown'}")
        return cls(h)

    @property
    def width(self) -> int:
        return int(_lib().pdefa_image_width(self._handle))

    @property
    def height(self) -> int:
        return int(_lib().pdefa_image_height(self._handle))

    @property
    def channels(self) -> int:
        return int(_lib().pdefa_image_channels(self._handle))

    @property
    def format(self) -> int:
        return int(_lib().pdefa_image_format(self._handle))

    def tobytes(self) -> bytes:
        n = C.c_size_t(0)
        ptr = _lib().pdefa_image_pixels(self._handle, C.byref(n))
        return C.string_at(ptr, n.value) if ptr and n.value else b""

    pixels_bytes = tobytes

    def tolist(self):
        b = self.tobytes()
        if not b:
            return []
        W, Ch = self.width, self.channels
        return [[list(b[(y * W + x) * Ch:(y * W + x + 1) * Ch]) for x in range(W)] for y in range(self.height)]

    def numpy(self):
        import numpy as np
        b = self.tobytes()
        return np.frombuffer(b, dtype=np.uint8).reshape(self.height, self.width, self.channels) if b else None

    def __repr__(self):
        return f"<Image {self.width}x{self.height} ch={self.channels} fmt={self.format}>"


def load_image(path: str) -> Image:
    h = _lib().pdefa_image_load(path.encode("utf-8"))
    if not h:
        raw = _lib().pdefa_last_error()
        raise PdefaError(f"load_image({path}): {raw.decode('utf-8', 'replace') if raw else 'unknown'}")
    return Image(h)


def preprocess_letterbox(img: Image, target_w: int = 640, target_h: int = 640, scale: float = 1.0 / 255.0,
                         pad_value: float = 0.0) -> Tuple[Tensor, PreprocessMeta]:
    cfg = _PreConfig(target_w, target_h, scale, pad_value)
    h, meta = C.c_void_p(), _PreMeta()
    _check(_lib().pdefa_preprocess_letterbox(img._handle, C.byref(cfg), C.byref(h), C.byref(meta)),
           "preprocess_letterbox")
    return Tensor(h), PreprocessMeta.from_c(meta)


def prepare_for_engine(path: str, target_w: int = 640, target_h: int = 640, scale: float = 1.0 / 255.0,
                       pad_value: float = 0.0) -> Tuple[Tensor, PreprocessMeta]:
    h, meta = C.c_void_p(), _PreMeta()
    _check(_lib().pdefa_prepare_for_engine(path.encode("utf-8"), target_w, target_h, scale, pad_value, C.byref(h),
                                           C.byref(meta)), "prepare_for_engine")
    return Tensor(h), PreprocessMeta.from_c(meta)


def load_image_as_tensor(path: str, target_w: int = 640, target_h: int = 640) -> Tensor:
    h = C.c_void_p()
    _check(_lib().pdefa_load_image_as_tensor(path.encode("utf-8"), target_w, target_h, C.byref(h)),
           "load_image_as_tensor")
    return Tensor(h)


def map_box_to_original(box: Box, meta: PreprocessMeta) -> Box:
    src = (C.c_float * 4)(box.x1, box.y1, box.x2, box.y2)
    dst = (C.c_float * 4)()
    cm = meta.to_c()
    _check(_lib().pdefa_map_box_to_original(src, C.byref(cm), dst), "map_box_to_original")
    return Box(dst[0], dst[1], dst[2], dst[3])


def map_point_to_original(x: float, y: float, meta: PreprocessMeta) -> Tuple[float, float]:
    cx, cy, cm = C.c_float(x), C.c_float(y), meta.to_c()
    _check(_lib().pdefa_map_point_to_original(C.byref(cx), C.byref(cy), C.byref(cm)), "map_point_to_original")
    return float(cx.value), float(cy.value)


# ---------------------------------------------------------------- engine

class Context:
    """Host-side settings (thread count for the host helpers); the GPU is
    chosen by HIP's current device."""

    def __init__(self):
        self._handle = C.c_void_p()
        _check(_lib().engine_context_create(C.byref(self._handle)), "context_create")

    def __del__(self):
        try:
            if self._handle and self._handle.value:
                _lib().engine_context_destroy(self._handle)
        except Exception:
            pass

    @property
    def raw(self):
        return self._handle

    def set_num_threads(self, n: int) -> "Context":
        _check(_lib().engine_context_set_num_threads(self._handle, int(n)), "set_num_threads")
        return self

    def get_num_threads(self) -> int:
        return int(_lib().engine_context_get_num_threads(self._handle))


def _info(handle, idx: int, fn) -> TensorInfo:
    name, dims = C.c_char_p(), (C.c_int64 * 8)()
    nd, dt = C.c_int32(0), C.c_int(0)
    rc = fn(handle, int(idx), C.byref(name), dims, C.byref(nd), C.byref(dt))
    if rc != 0:
        raise PdefaError(f"model_info(idx={idx}): rc={rc}")
    return TensorInfo(name=name.value.decode() if name.value else f"tensor_{idx}",
                      shape=tuple(int(dims[i]) for i in range(nd.value)), dtype=int(dt.value))


class Model:
    """An .engine model; its weights are uploaded to HBM (and conv weights
    packed for the matrix cores) once, at load, when a GPU is present."""

    def __init__(self, ctx: Context, path: str):
        self._handle = C.c_void_p()
        _check(_lib().engine_model_load(ctx.raw, path.encode("utf-8"), C.byref(self._handle)), "model_load")

    def __del__(self):
        try:
            if self._handle and self._handle.value:
                _lib().engine_model_destroy(self._handle)
        except Exception:
            pass

    @property
    def raw(self):
        return self._handle

    @property
    def name(self) -> str:
        p = C.c_char_p()
        _check(_lib().engine_model_name(self._handle, C.byref(p)), "model_name")
        return p.value.decode() if p.value else ""

    def input_info(self, idx: int) -> TensorInfo:
        return _info(self._handle, idx, _lib().engine_model_input_info)

    def output_info(self, idx: int) -> TensorInfo:
        return _info(self._handle, idx, _lib().engine_model_output_info)


class Session:
    """One GPU program per input shape (HIP stream + HBM arena + hipGraph).
    Inputs are kept alive here because the library keeps their pointers."""

    def __init__(self, ctx: Context, model: Model):
        self._handle = C.c_void_p()
        _check(_lib().engine_session_create(ctx.raw, model.raw, C.byref(self._handle)), "session_create")
        self._model = model  # the session borrows the model
        self._input_refs = {}

    def __del__(self):
        try:
            if self._handle and self._handle.value:
                _lib().engine_session_destroy(self._handle)
        except Exception:
            pass

    @property
    def raw(self):
        return self._handle

    def set_input(self, index: int, tensor: Tensor) -> None:
        _check(_lib().engine_session_set_input(self._handle, int(index), tensor.raw), "session_set_input")
        self._input_refs[index] = tensor

    def set_images(self, index: int, images, target_w: int = 640, target_h: int = 640, scale: float = 1.0 / 255.0,
                   pad_value: float = 0.0) -> List[PreprocessMeta]:
        """Input `index` becomes the letterbox of `images` (a batch), computed
        on the GPU at the next run from their 8-bit pixels; same values as
        preprocess_letterbox on each image.  Returns the per-image metas
        (extension, include/pdefa_amd_ext.h)."""
        imgs = [im if isinstance(im, Image) else Image.from_array(im) for im in images]
        if not imgs:
            raise PdefaError("set_images: no images")
        arr = (C.c_void_p * len(imgs))(*[im._handle.value for im in imgs])
        cfg = _PreConfig(target_w, target_h, scale, pad_value)
        metas = (_PreMeta * len(imgs))()
        _check(_lib().pdefa_amd_session_set_images(self._handle, int(index), len(imgs),
                                                   C.cast(arr, C.POINTER(C.c_void_p)), C.byref(cfg), metas),
               "session_set_images")
        self._input_refs.pop(index, None)
        return [PreprocessMeta.from_c(m) for m in metas]

    def run(self) -> None:
        _check(_lib().engine_session_run(self._handle), "session_run")

    def output(self, index: int = 0) -> Tensor:
        h = C.c_void_p()
        _check(_lib().engine_session_get_output(self._handle, int(index), C.byref(h)), "session_get_output")
        return Tensor(h, owns=False)

    def stats(self) -> dict:
        s = _SessionStats()
        _check(_lib().engine_session_get_stats(self._handle, C.byref(s)), "session_get_stats")
        return {"last_run_ms": s.last_run_ms, "runs": int(s.runs)}

    def debug_intermediate(self, idx: int) -> Tensor:
        h = C.c_void_p()
        _check(_lib().engine_session_debug_intermediate(self._handle, int(idx), C.byref(h)), "debug_intermediate")
        return Tensor(h, owns=False)

    def decode(self, metas=None, conf_thres: float = 0.25, iou_thres: float = 0.45, max_det: int = 300,
               output_index: int = 0, with_anchor: bool = False) -> List[List[dict]]:
        """decode_yolo of every image of output `output_index` (the [N, 4 +
        classes, A] head of the last run), computed on the GPU: the same
        detections, order and values as decode_yolo on each image.  metas:
        None or one PreprocessMeta per image (extension, include/pdefa_amd_ext.h)."""
        n_img = int(self.output(output_index).shape[0])
        if metas is not None and len(metas) != n_img:
            raise PdefaError(f"decode: {len(metas)} metas for {n_img} images")
        cm = (_PreMeta * n_img)(*[m.to_c() for m in metas]) if metas is not None else None
        dets = (_Detection * max(1, n_img * max_det))()
        counts = (C.c_int32 * n_img)()
        _check(_lib().pdefa_amd_session_decode(self._handle, int(output_index), cm, n_img if cm is not None else 0,
                                               float(conf_thres), float(iou_thres), int(max_det), dets, counts),
               "session_decode")
        out = []
        for i in range(n_img):
            rows = []
            for j in range(counts[i]):
                d = dets[i * max_det + j]
                r = {"x1": d.x1, "y1": d.y1, "x2": d.x2, "y2": d.y2, "conf": d.conf, "cls": int(d.cls)}
                if with_anchor:
                    r["anchor"] = int(d.anchor)
                rows.append(r)
            out.append(rows)
        return out

    def run_and_decode(self, meta: Optional[PreprocessMeta] = None, conf_thres: float = 0.25,
                       iou_thres: float = 0.45) -> List[dict]:
        """run() then decode_yolo of image 0 of output 0; the decode runs on the
        GPU (Session.decode) with decode_yolo's results."""
        self.run()
        res = self.decode([meta] if meta is not None else None, conf_thres, iou_thres)
        if len(res) != 1:
            raise PdefaError(f"decode_yolo: unexpected output shape {tuple(self.output(0).shape)}")
        return res[0]


# ---------------------------------------------------------------- decode

def decode_yolo(output, meta: Optional[PreprocessMeta] = None, conf_thres: float = 0.25, iou_thres: float = 0.45,
                max_det: int = 300) -> List[dict]:
    """[{'x1','y1','x2','y2','conf','cls'}, ...] from a (1, 4+nc, A) or
    (4+nc, A) head given as a Tensor, nested list or array; leading
    singleton dims are unwrapped and fewer than 5 rows raise PdefaError
    (_bindings.py:1095-1175).  The anchor scan is vectorised; NMS is the
    reference's per-class greedy loop."""
    import numpy as np
    arr = output.to_numpy() if isinstance(output, Tensor) else np.asarray(output, dtype=np.float32)
    while arr.ndim > 2 and arr.shape[0] == 1 and arr.shape[1] > 4:
        arr = arr[0]
    if arr.ndim != 2 or arr.shape[0] < 5:
        raise PdefaError(f"decode_yolo: unexpected output shape {tuple(arr.shape)}")
    return _decode_heads(arr, meta, conf_thres, iou_thres, max_det)


def _model_input_shape(model: Model, idx: int = 0) -> tuple:
    return model.input_info(idx).shape


def prepare_for_model(model: Model, path: str, input_idx: int = 0, scale: float = 1.0 / 255.0,
                      pad_value: float = 0.0) -> Tuple[Tensor, PreprocessMeta]:
    """Letterbox to the model's input H, W (_bindings.py:1224-1242)."""
    shape = _model_input_shape(model, input_idx)
    if len(shape) != 4:
        raise PdefaError(f"prepare_for_model: expected a 4-D input, got {shape}")
    return prepare_for_engine(path, shape[3], shape[2], scale, pad_value)


class EngineModel:
    """load(path)(image) -> detections (_bindings.py:1250-1280)."""

    def __init__(self, ctx: Context, model: Model, session: Session):
        self.ctx, self.model, self.session = ctx, model, session

    def __call__(self, image_path: str, conf_thres: float = 0.25, iou_thres: float = 0.45) -> List[dict]:
        tensor, meta = prepare_for_model(self.model, image_path)
        self.session.set_input(0, tensor)
        self.session.run()
        return decode_yolo(self.session.output(0), meta, conf_thres, iou_thres)

    def set_num_threads(self, n: int) -> "EngineModel":
        self.ctx.set_num_threads(n)
        return self


def load(engine_path: str) -> EngineModel:
    ctx = Context()
    model = Model(ctx, engine_path)
    return EngineModel(ctx, model, Session(ctx, model))


from .batch import BatchInference  # noqa: E402  (needs the names above)

__all__ = [
    "__version__", "PdefaError", "PreprocessMeta", "Box", "Image", "Tensor", "TensorInfo", "Context", "Model",
    "Session", "version", "simd_level", "cpu_brand", "load_image", "preprocess_letterbox", "prepare_for_engine",
    "load_image_as_tensor", "map_box_to_original", "map_point_to_original", "decode_yolo", "prepare_for_model",
    "ops_matmul", "ops_relu", "ops_silu", "tensor_empty", "ops_add", "ops_sub", "ops_mul", "ops_div",
    "ops_sigmoid", "ops_tanh", "ops_gelu", "ops_clip", "ops_softmax", "ops_reduce_max", "ops_reduce_sum",
    "ops_reduce_mean", "ops_argmax", "ops_gather", "ops_reshape", "ops_transpose", "ops_concat", "ops_stack",
    "random_randn", "random_rand", "randn", "rand", "zeros", "ones", "empty", "from_list", "load", "EngineModel",
    "BatchInference",
]
