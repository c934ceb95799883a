"""Timed run of the compiled reference engine — TEST INFRASTRUCTURE ONLY.

bench.py's cpu_baseline leg starts this as a child process, so the reference
engine's worker threads live and end in their own process:

    python -m oracle.ref_bench MODEL.engine INPUT.npy BUDGET_S THREADS

Runs Session::run once, two warm-up reruns, then reruns for up to BUDGET_S
seconds (at most 30) and prints one JSON line {"ms": [...], "threads": n}.
"""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

from oracle import ref_lib


def main() -> None:
    path, npy, budget_s, threads = sys.argv[1], sys.argv[2], float(sys.argv[3]), int(sys.argv[4])
    x = np.load(npy)  # written by bench.py (no pickled objects)
    ref_lib.set_threads(threads)
    r = ref_lib.RefSession(path)
    r.run(x)
    for _ in range(2):
        r.rerun()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end and len(times) < 30:
        r.rerun()
        times.append(r.last_ms())
    r.close()
    sys.stdout.write(json.dumps({"ms": times, "threads": threads}) + "\n")
    sys.stdout.flush()
    # the timing is out; end without running library teardown
    os._exit(0)


if __name__ == "__main__":
    main()
