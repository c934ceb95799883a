"""Loader for libpdefa_native.so and numpy helpers over its C ABI.

The library is built in-tree by pdefa_amd/build.py.  Everything here talks to
the C ABI only (no torch); loading fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import List, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libpdefa_native.so")

ENGINE_OK = 0
ENGINE_ERR_INVALID_ARG = 7
STATUS = {0: "OK", 1: "NULL_PTR", 2: "INVALID_HANDLE", 3: "OUT_OF_MEMORY", 4: "FILE_NOT_FOUND",
          5: "INVALID_FORMAT", 6: "INVALID_SHAPE", 7: "INVALID_ARG", 8: "RUNTIME", 9: "NOT_IMPL",
          99: "UNKNOWN"}
F32, I32, I64 = 0, 5, 6
_NP = {0: np.float32, 1: np.float16, 3: np.int8, 4: np.uint8, 5: np.int32, 6: np.int64, 7: np.bool_}

_lib: Optional[C.CDLL] = None


class NativeError(RuntimeError):
    def __init__(self, status: int, where: str, msg: str = ""):
        self.status = status
        super().__init__(f"{where}: {STATUS.get(status, status)}" + (f" ({msg})" if msg else ""))


def lib() -> C.CDLL:
    """The loaded native library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: run `python -m pdefa_amd.build`")
        L = C.CDLL(LIB_PATH)
        vp, i32, i64, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t
        pvp = C.POINTER(C.c_void_p)
        sig = {
            "engine_version": (C.c_char_p, []),
            "engine_last_error": (C.c_char_p, []),
            "pdefa_last_error": (C.c_char_p, []),
            "engine_simd_level": (C.c_char_p, []),
            "engine_cpu_brand": (C.c_char_p, []),
            "engine_context_create": (C.c_int, [pvp]),
            "engine_context_destroy": (None, [vp]),
            "engine_context_set_num_threads": (C.c_int, [vp, i32]),
            "engine_context_get_num_threads": (i32, [vp]),
            "engine_tensor_create": (C.c_int, [pvp, C.POINTER(i64), i32, C.c_int]),
            "engine_tensor_create_from_data": (C.c_int, [pvp, C.POINTER(i64), i32, C.c_int, vp, sz]),
            "engine_tensor_data": (C.c_int, [vp, pvp, C.POINTER(sz)]),
            "engine_tensor_shape": (C.c_int, [vp, C.POINTER(i64), C.POINTER(i32)]),
            "engine_tensor_dtype": (C.c_int, [vp]),
            "engine_tensor_destroy": (None, [vp]),
            "engine_model_load": (C.c_int, [vp, C.c_char_p, pvp]),
            "engine_model_destroy": (None, [vp]),
            "engine_session_create": (C.c_int, [vp, vp, pvp]),
            "engine_session_set_input": (C.c_int, [vp, i32, vp]),
            "engine_session_run": (C.c_int, [vp]),
            "engine_session_get_output": (C.c_int, [vp, i32, pvp]),
            "engine_session_destroy": (None, [vp]),
            "engine_ops_matmul": (C.c_int, [vp, vp, vp]),
            "pdefa_amd_session_replay": (C.c_int, [vp, i32, C.POINTER(C.c_double)]),
            "pdefa_amd_session_step_repeat": (C.c_int, [vp, i32, i32, C.POINTER(C.c_double)]),
            "pdefa_amd_session_plan": (C.c_int, [vp, C.c_char_p, sz, C.POINTER(sz)]),
            "pdefa_amd_session_step_times": (C.c_int, [vp, i32, C.POINTER(C.c_double), C.POINTER(i32),
                                                       C.POINTER(i64), i32, C.POINTER(i32)]),
            "pdefa_amd_plan_model": (C.c_int, [vp, C.POINTER(i64), i32, C.c_char_p, sz, C.POINTER(sz)]),
            "pdefa_amd_device_name": (C.c_char_p, []),
            "pdefa_amd_tune_stats": (C.c_int, [C.POINTER(i64), C.POINTER(i64)]),
            "pdefa_amd_pack_cache_stats": (C.c_int, [C.POINTER(i64), C.POINTER(i64)]),
            "pdefa_amd_ops_matmul_noalloc": (C.c_int, [vp, vp, vp]),
            "pdefa_amd_session_read_conv_input": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_float), sz,
                                                            C.POINTER(i64)]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int, where: str) -> None:
    if status != ENGINE_OK:
        msg = lib().pdefa_last_error()
        raise NativeError(status, where, msg.decode() if msg else "")


def tensor_from_numpy(a: np.ndarray) -> C.c_void_p:
    a = np.ascontiguousarray(a, dtype=np.float32)
    shape = (C.c_int64 * max(a.ndim, 1))(*a.shape)
    h = C.c_void_p()
    check(lib().engine_tensor_create_from_data(C.byref(h), shape, a.ndim, F32,
                                               a.ctypes.data_as(C.c_void_p), a.nbytes),
          "engine_tensor_create_from_data")
    return h


def tensor_to_numpy(h: C.c_void_p) -> np.ndarray:
    L = lib()
    dims = (C.c_int64 * 8)()
    nd = C.c_int32()
    check(L.engine_tensor_shape(h, dims, C.byref(nd)), "engine_tensor_shape")
    ptr = C.c_void_p()
    nbytes = C.c_size_t()
    check(L.engine_tensor_data(h, C.byref(ptr), C.byref(nbytes)), "engine_tensor_data")
    dt = _NP.get(L.engine_tensor_dtype(h), np.float32)
    shape = [dims[i] for i in range(nd.value)]
    n = int(np.prod(shape)) if shape else 1
    if n == 0 or not ptr.value:
        return np.zeros(shape, dt)
    buf = (C.c_char * nbytes.value).from_address(ptr.value)
    return np.frombuffer(buf, dtype=dt, count=n).reshape(shape).copy()


class Engine:
    """One context + model + session over the C ABI, numpy in and out."""

    def __init__(self, path: str):
        L = lib()
        self.ctx = C.c_void_p()
        check(L.engine_context_create(C.byref(self.ctx)), "engine_context_create")
        self.model = C.c_void_p()
        check(L.engine_model_load(self.ctx, path.encode(), C.byref(self.model)), "engine_model_load")
        self.sess = C.c_void_p()
        check(L.engine_session_create(self.ctx, self.model, C.byref(self.sess)), "engine_session_create")
        self._inputs: List[C.c_void_p] = []

    def run(self, *xs: np.ndarray) -> List[np.ndarray]:
        L = lib()
        for h in self._inputs:
            L.engine_tensor_destroy(h)
        self._inputs = [tensor_from_numpy(x) for x in xs]
        for i, h in enumerate(self._inputs):
            check(L.engine_session_set_input(self.sess, i, h), "engine_session_set_input")
        check(L.engine_session_run(self.sess), "engine_session_run")
        outs = []
        i = 0
        while True:
            h = C.c_void_p()
            if L.engine_session_get_output(self.sess, i, C.byref(h)) != ENGINE_OK:
                break
            outs.append(tensor_to_numpy(h))
            i += 1
        return outs

    def session_run_times(self, warmup: int, runs: int) -> List[float]:
        """Wall ms of each of `runs` engine_session_run calls on the inputs of
        the last run() (host input uploaded, program launched, output
        downloaded and synchronised), after one untimed call and `warmup`
        more -- the protocol of the reference's bench_models.py:226-241."""
        import time
        L = lib()
        check(L.engine_session_run(self.sess), "engine_session_run")
        for _ in range(warmup):
            check(L.engine_session_run(self.sess), "engine_session_run")
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            st = L.engine_session_run(self.sess)
            ts.append((time.perf_counter() - t0) * 1e3)
            check(st, "engine_session_run")
        return ts

    def conv_input(self, node: str, cap: int = 1 << 26) -> np.ndarray:
        """The [N, C, H, W] input of the conv step implementing `node` after
        the last run (the session must have been created with
        PDEFA_KEEP_TENSORS=1)."""
        buf = np.empty(cap, np.float32)
        dims = (C.c_int64 * 4)()
        check(lib().pdefa_amd_session_read_conv_input(self.sess, node.encode(),
                                                      buf.ctypes.data_as(C.POINTER(C.c_float)), cap, dims),
              "pdefa_amd_session_read_conv_input")
        shape = tuple(int(d) for d in dims)
        return buf[:int(np.prod(shape))].reshape(shape).copy()

    def replay(self, iters: int) -> float:
        ms = C.c_double()
        check(lib().pdefa_amd_session_replay(self.sess, iters, C.byref(ms)), "pdefa_amd_session_replay")
        return ms.value

    def step_times(self, iters: int):
        """(ms, kind, flops) arrays: per-step average device time over `iters`."""
        cap = 4096
        ms = (C.c_double * cap)()
        kind = (C.c_int32 * cap)()
        flops = (C.c_int64 * cap)()
        n = C.c_int32()
        check(lib().pdefa_amd_session_step_times(self.sess, iters, ms, kind, flops, cap, C.byref(n)),
              "pdefa_amd_session_step_times")
        k = min(n.value, cap)
        return (np.array(ms[:k]), np.array(kind[:k]), np.array(flops[:k], dtype=np.int64))

    def step_repeat(self, step: int, iters: int) -> float:
        """Average ms per launch of step `step` launched `iters` times back to back."""
        ms = C.c_double()
        check(lib().pdefa_amd_session_step_repeat(self.sess, int(step), int(iters), C.byref(ms)),
              "pdefa_amd_session_step_repeat")
        return ms.value

    def plan(self) -> str:
        buf = C.create_string_buffer(1 << 20)
        n = C.c_size_t()
        check(lib().pdefa_amd_session_plan(self.sess, buf, len(buf), C.byref(n)), "pdefa_amd_session_plan")
        return buf.value.decode()

    def close(self) -> None:
        L = lib()
        for h in self._inputs:
            L.engine_tensor_destroy(h)
        self._inputs = []
        if self.sess:
            L.engine_session_destroy(self.sess)
            self.sess = C.c_void_p()
        if self.model:
            L.engine_model_destroy(self.model)
            self.model = C.c_void_p()
        if self.ctx:
            L.engine_context_destroy(self.ctx)
            self.ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def tune_stats():
    """(measured, from_table): conv launch-shape choices of this process
    timed on the device, and read from the launch-shape table."""
    m, t = C.c_int64(), C.c_int64()
    check(lib().pdefa_amd_tune_stats(C.byref(m), C.byref(t)), "pdefa_amd_tune_stats")
    return m.value, t.value


def pack_cache_stats():
    """(read, written): pre-pack cache files this process read and wrote
    (PDEFA_PACK_CACHE=1)."""
    r, w = C.c_int64(), C.c_int64()
    check(lib().pdefa_amd_pack_cache_stats(C.byref(r), C.byref(w)), "pdefa_amd_pack_cache_stats")
    return r.value, w.value


def plan_text(path: str, shape: Sequence[int]) -> str:
    """Device program for `path` at input `shape`, planned on the host."""
    L = lib()
    ctx = C.c_void_p()
    check(L.engine_context_create(C.byref(ctx)), "engine_context_create")
    model = C.c_void_p()
    try:
        check(L.engine_model_load(ctx, path.encode(), C.byref(model)), "engine_model_load")
        dims = (C.c_int64 * len(shape))(*shape)
        buf = C.create_string_buffer(1 << 20)
        n = C.c_size_t()
        check(L.pdefa_amd_plan_model(model, dims, len(shape), buf, len(buf), C.byref(n)), "pdefa_amd_plan_model")
        return buf.value.decode()
    finally:
        if model:
            L.engine_model_destroy(model)
        L.engine_context_destroy(ctx)


def matmul_into(a: np.ndarray, b: np.ndarray, out: np.ndarray, noalloc: bool = False) -> np.ndarray:
    """engine_ops_matmul(a, b, out) (or, with noalloc, its variant
    pdefa_amd_ops_matmul_noalloc, which allocates no device memory) with
    `out` a pre-filled tensor of any shape; returns what the call left in it
    (the call returns ENGINE_OK also when it leaves `out` untouched for
    mismatched shapes, as the reference's ops::matmul does)."""
    L = lib()
    fn, name = ((L.pdefa_amd_ops_matmul_noalloc, "pdefa_amd_ops_matmul_noalloc") if noalloc
                else (L.engine_ops_matmul, "engine_ops_matmul"))
    ha, hb, hc = tensor_from_numpy(a), tensor_from_numpy(b), tensor_from_numpy(out)
    try:
        check(fn(ha, hb, hc), name)
        return tensor_to_numpy(hc)
    finally:
        for h in (ha, hb, hc):
            L.engine_tensor_destroy(h)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = a @ b through engine_ops_matmul (runs on the GPU)."""
    L = lib()
    ha, hb = tensor_from_numpy(a), tensor_from_numpy(b)
    shape = (C.c_int64 * 2)(a.shape[0], b.shape[1])
    hc = C.c_void_p()
    check(L.engine_tensor_create(C.byref(hc), shape, 2, F32), "engine_tensor_create")
    try:
        check(L.engine_ops_matmul(ha, hb, hc), "engine_ops_matmul")
        return tensor_to_numpy(hc)
    finally:
        for h in (ha, hb, hc):
            L.engine_tensor_destroy(h)
