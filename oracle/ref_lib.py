"""ctypes access to oracle/_ref/libpdefa_ref.so — TEST INFRASTRUCTURE ONLY.

The library is the reference CPU engine compiled from its own sources by
oracle/Makefile plus oracle/ref_driver.cpp.  Only tests/, smoke() and bench.py's
cpu_baseline leg use it, as the checker / the timed CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import List, Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_ref", "libpdefa_ref.so")
_lib: Optional[C.CDLL] = None


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not available():
            raise FileNotFoundError(f"{LIB_PATH} not built (run make -C oracle)")
        L = C.CDLL(LIB_PATH)
        vp, i64p, f32p = C.c_void_p, C.POINTER(C.c_int64), C.POINTER(C.c_float)
        L.ref_model_load.restype = vp
        L.ref_model_load.argtypes = [C.c_char_p]
        L.ref_model_free.argtypes = [vp]
        L.ref_session_new.restype = vp
        L.ref_session_new.argtypes = [vp]
        L.ref_session_free.argtypes = [vp]
        L.ref_session_run.argtypes = [vp, f32p, i64p, C.c_int]
        L.ref_session_rerun.argtypes = [vp]
        L.ref_session_last_ms.restype = C.c_double
        L.ref_session_last_ms.argtypes = [vp]
        L.ref_output_count.argtypes = [vp]
        L.ref_output_shape.argtypes = [vp, C.c_int, i64p]
        L.ref_output_copy.argtypes = [vp, C.c_int, f32p, C.c_int64]
        L.ref_output_dtype.argtypes = [vp, C.c_int]
        L.ref_set_threads.argtypes = [C.c_int]
        L.ref_matmul.argtypes = [f32p, f32p, f32p, C.c_int64, C.c_int64, C.c_int64]
        L.ref_letterbox.argtypes = [C.POINTER(C.c_uint8), C.c_int, C.c_int, C.c_int, C.c_int,
                                    C.c_int, C.c_float, C.c_float, f32p,
                                    C.POINTER(C.c_int32), f32p]
        _lib = L
    return _lib


def _f32p(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def set_threads(n: int) -> None:
    lib().ref_set_threads(int(n))


class RefSession:
    """Reference Model + Session over one `.engine` file."""

    def __init__(self, path: str):
        L = lib()
        self.model = L.ref_model_load(path.encode())
        if not self.model:
            raise RuntimeError(f"reference failed to load {path}")
        self.sess = L.ref_session_new(self.model)

    def run(self, x: np.ndarray) -> List[np.ndarray]:
        L = lib()
        x = np.ascontiguousarray(x, np.float32)
        shape = (C.c_int64 * x.ndim)(*x.shape)
        rc = L.ref_session_run(self.sess, _f32p(x), shape, x.ndim)
        if rc != 0:
            raise RuntimeError(f"reference Session::run failed ({rc})")
        return self.outputs()

    def rerun(self) -> None:
        if lib().ref_session_rerun(self.sess) != 0:
            raise RuntimeError("reference Session::run failed")

    def last_ms(self) -> float:
        return lib().ref_session_last_ms(self.sess)

    def output_dtypes(self) -> List[int]:
        """The engine's DType code of each output (12 F32, 6 I32, 8 I64)."""
        L = lib()
        return [L.ref_output_dtype(self.sess, i) for i in range(L.ref_output_count(self.sess))]

    def outputs(self) -> List[np.ndarray]:
        """Every output as float32 values (integer outputs converted)."""
        L = lib()
        outs = []
        for i in range(L.ref_output_count(self.sess)):
            dims = (C.c_int64 * 8)()
            r = L.ref_output_shape(self.sess, i, dims)
            if r < 0:
                raise RuntimeError(f"reference output {i} missing")
            o = np.empty([dims[d] for d in range(r)], np.float32)
            L.ref_output_copy(self.sess, i, _f32p(o), o.size)
            outs.append(o)
        return outs

    def close(self):
        L = lib()
        if self.sess:
            L.ref_session_free(self.sess)
            self.sess = None
        if self.model:
            L.ref_model_free(self.model)
            self.model = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().ref_matmul(_f32p(a), _f32p(b), _f32p(c), m, k, n)
    return c


def letterbox(img: np.ndarray, tw: int, th: int, scale: float, pad: float):
    img = np.ascontiguousarray(img, np.uint8)
    h, w = img.shape[:2]
    ch = 1 if img.ndim == 2 else img.shape[2]
    out = np.empty((3, th, tw), np.float32)
    meta = (C.c_int32 * 6)()
    ratio = C.c_float()
    rc = lib().ref_letterbox(img.ctypes.data_as(C.POINTER(C.c_uint8)), w, h, ch, tw, th,
                             scale, pad, _f32p(out), meta, C.byref(ratio))
    if rc != 0:
        raise RuntimeError("reference letterbox failed")
    m = dict(target_w=meta[0], target_h=meta[1], pad_x=meta[2], pad_y=meta[3],
             scaled_w=meta[4], scaled_h=meta[5], ratio=ratio.value)
    return out[None], m
