"""Batch inference with the reference's interface (pdefa/python/src/pdefa/batch.py:13-69).

The reference keeps one CPU session per batch slot and runs them on a thread
pool.  Here host threads only decode and letterbox the images; each chunk of
`batch_size` images then runs as ONE batched GPU program ([B, 3, H, W] ->
[B, 84, A] in a single hipGraph launch) and the output is split into
per-image tensors of the reference's per-session shape (1, 84, A), each
owned by the caller.  With device_preprocess=True the host threads only
decode; the letterbox runs on the GPU from the 8-bit pixels (same values).
"""
from __future__ import annotations

import ctypes as C
from concurrent.futures import ThreadPoolExecutor
from typing import List, Optional, Tuple

from . import pdefa as _api


class BatchInference:
    def __init__(self, ctx: "_api.Context", model: "_api.Model", batch_size: int = 4, num_threads: int = 4,
                 device_preprocess: bool = False):
        if batch_size < 1 or num_threads < 1:
            raise _api.PdefaError("BatchInference: batch_size and num_threads must be >= 1")
        self.ctx = ctx
        self.model = model
        self.batch_size = int(batch_size)
        self.num_threads = int(num_threads)
        self.device_preprocess = bool(device_preprocess)
        self._session: Optional[_api.Session] = _api.Session(ctx, model)
        self._executor = ThreadPoolExecutor(max_workers=self.num_threads)

    def _split(self, out: "_api.Tensor", n: int) -> List["_api.Tensor"]:
        """Per-image owned copies of a borrowed [n, ...] output."""
        shape = out.shape
        addr, nbytes = out._data()
        per = nbytes // n
        one = [1] + list(shape[1:])
        parts = []
        for i in range(n):
            t = _api.tensor_empty(one, out.dtype)
            _api._check(_api._lib().engine_tensor_copy_from(t.raw, C.c_void_p(addr + i * per), per),
                        "batch_split")
            parts.append(t)
        return parts

    def run(self, image_paths: List[str], target_w: int = 640,
            target_h: int = 640) -> List[Tuple["_api.Tensor", "_api.PreprocessMeta"]]:
        if self._session is None:
            raise _api.PdefaError("BatchInference: closed")
        results: List[Tuple[_api.Tensor, _api.PreprocessMeta]] = []
        for start in range(0, len(image_paths), self.batch_size):
            chunk = image_paths[start:start + self.batch_size]
            if self.device_preprocess:
                # prepare_for_engine's letterbox parameters, on the device
                imgs = list(self._executor.map(_api.load_image, chunk))
                metas = self._session.set_images(0, imgs, target_w, target_h, 1.0 / 255.0, 0.0)
            else:
                prepped = list(self._executor.map(lambda p: _api.prepare_for_engine(p, target_w, target_h), chunk))
                batch = _api.ops_concat([t for t, _ in prepped], axis=0) if len(prepped) > 1 else prepped[0][0]
                self._session.set_input(0, batch)
                metas = [m for _, m in prepped]
            self._session.run()
            outs = self._split(self._session.output(0), len(chunk))
            results.extend(zip(outs, metas))
        return results

    def close(self) -> None:
        self._executor.shutdown(wait=True)
        self._session = None

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()
