"""Timed run of the compiled reference engine — TEST INFRASTRUCTURE ONLY.

bench.py's cpu_baseline leg starts this as a child process, so the reference
engine's worker threads live and end in their own process:

    python -m oracle.ref_bench MODEL.engine INPUT.npy THREADS [RUNS] [WARMUP]

The protocol of the reference's own benchmark (pdefa/benchmarks/
bench_models.py:61-62,226-241): one untimed Session::run, WARMUP (5) more,
then RUNS (30) timed with the host clock; prints one JSON line
{"ms": [...], "threads": n} (the caller takes the median as the reference
does, the upper one of an even count).
"""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

from oracle import ref_lib


def main() -> None:
    path, npy, threads = sys.argv[1], sys.argv[2], int(sys.argv[3])
    runs = int(sys.argv[4]) if len(sys.argv) > 4 else 30
    warmup = int(sys.argv[5]) if len(sys.argv) > 5 else 5
    x = np.load(npy)  # written by bench.py (no pickled objects)
    ref_lib.set_threads(threads)
    r = ref_lib.RefSession(path)
    r.run(x)
    for _ in range(warmup):
        r.rerun()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        r.rerun()
        times.append((time.perf_counter() - t0) * 1e3)
    r.close()
    sys.stdout.write(json.dumps({"ms": times, "threads": threads}) + "\n")
    sys.stdout.flush()
    # the timing is out; end without running library teardown
    os._exit(0)


if __name__ == "__main__":
    main()
