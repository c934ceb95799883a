"""The compiled reference engine (oracle/_ref, test infrastructure) run in a
worker process for the GPU tests.

The reference's ThreadPool::parallel_for
(PDEFA1.0/src/runtime/thread_pool.cpp:148-181) keeps its completion mutex and
condition variable in the caller's stack frame, and the task that finishes
last takes that mutex after it has decremented the remaining count.  When
the caller sees the count at zero first (its wait checks the count before it
sleeps), it returns, and the worker then locks a mutex in a dead stack frame:
once that memory is reused the lock can block the worker forever, and every
later join of the pool with it (setting the thread count resets the pool and
joins its workers).  In the GPU test process such a worker would hang the
whole run.  Here the reference runs in a child process, started before the
tests touch the GPU, with its thread count set once, and each call has a time
limit: a call that does not return in time kills the child (SIGKILL, so no
pool teardown runs) and is made once more in a fresh child.
"""
from __future__ import annotations

import multiprocessing as mp
import os
from typing import List, Optional

import numpy as np

CALL_TIMEOUT_S = 45.0
THREADS = 16  # the GPU box's CPU share for one GPU

_proc = None
_conn = None


def _serve(conn, threads: int) -> None:
    from oracle import ref_lib

    ref_lib.set_threads(threads)
    while True:
        msg = conn.recv()
        if msg is None:
            return
        path, x, split = msg
        try:
            r = ref_lib.RefSession(path)
            try:
                outs = [r.run(x[i:i + 1]) for i in range(x.shape[0])] if split else [r.run(x)]
            finally:
                r.close()
            conn.send(("ok", outs))
        except Exception as e:  # reported to the caller, the worker keeps serving
            conn.send(("err", repr(e)))


def start() -> None:
    """Starts the worker if it is not running (idempotent)."""
    global _proc, _conn
    if _proc is not None and _proc.is_alive():
        return
    ctx = mp.get_context("spawn")
    parent, child = ctx.Pipe()
    _proc = ctx.Process(target=_serve, args=(child, min(THREADS, os.cpu_count() or 1)), daemon=True)
    _proc.start()
    child.close()
    _conn = parent


def stop() -> None:
    global _proc, _conn
    if _proc is not None:
        _proc.kill()
        _proc.join(5)
    _proc, _conn = None, None


def run(path: str, x: np.ndarray, split: bool = True) -> List[List[np.ndarray]]:
    """The reference engine's outputs for each image of x, run one image at a
    time (the reference has no batch path; BatchInference runs one session
    per image): a list over images of that run's output list.  split=False:
    one run on the whole of x (a one-element list)."""
    x = np.ascontiguousarray(x, np.float32)
    last: Optional[str] = None
    for _ in range(2):
        start()
        try:
            _conn.send((path, x, split))
            if _conn.poll(CALL_TIMEOUT_S):
                status, payload = _conn.recv()
                if status != "ok":
                    raise RuntimeError(f"reference engine failed on {path}: {payload}")
                return payload
            last = f"no result within {CALL_TIMEOUT_S:.0f} s"
        except (EOFError, OSError) as e:  # the worker died
            last = f"worker lost ({e!r})"
        stop()  # a stuck or lost reference call: a fresh worker runs it once more
    raise RuntimeError(f"reference engine on {path}: {last}, twice")
