"""Benchmark: YOLOv8n 640x640 fp32 images/s on one MI355X (b1 and b8), plus
the conv roofline and the reference CPU engine timed on the host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one forward of the whole YOLOv8n device program over one batch of
synthetic letterboxed input already resident in HBM: the session's captured
hipGraph is replayed K times after W warm-up replays, timed with HIP events
on the session stream and with the host clock around a device synchronise on
both sides.  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from pdefa_amd import native, yolo_synth as ys  # noqa: E402

METRIC = "images/s YOLOv8n 640² b1/b8 on 1 GPU; conv fp32 TFLOP/s vs MFMA peak"
PUBLISHED_B1_IMAGES_PER_S = 1000.0 / 37.0  # reference README.md:629,635 (37 ms, Ryzen 5 7535HS)
MFMA_FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
# Algorithmic work of the roofline kernel: conv 3x3 s1 pad 1, 64 -> 64 channels
# on a 1x64x160x160 input: 2 * Cout * Cin * 9 * 160 * 160 flops per launch.
CONV_ROOF = dict(cin=64, cout=64, k=3, stride=1, hw=160)
CONV_ROOF_FLOPS = 2 * 64 * 64 * 9 * 160 * 160
KIND_CONV_MFMA, KIND_CONV_DIRECT = 0, 1
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "conv3x3s1_64x64_160_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_program(eng: native.Engine, x: np.ndarray, steps: int, warmup: int):
    """ms per forward: W warm-up replays, then K timed replays of the graph."""
    eng.run(x)  # uploads the input, plans, captures the graph
    if warmup > 0:
        eng.replay(warmup)
    lib = native.lib()
    t0 = time.perf_counter()
    dev_ms = eng.replay(steps)
    wall_ms = (time.perf_counter() - t0) * 1e3
    log(f"  {steps} steps: device {dev_ms:.3f} ms, host wall {wall_ms:.3f} ms")
    return max(dev_ms, 0.0) / steps, wall_ms / steps


def conv_stats(eng: native.Engine, iters: int):
    ms, kind, flops = eng.step_times(iters)
    conv = (kind == KIND_CONV_MFMA) | (kind == KIND_CONV_DIRECT)
    conv_ms = float(ms[conv].sum())
    conv_flops = int(flops[conv].sum())
    return dict(conv_ms=conv_ms, conv_flops=conv_flops, step_ms=float(ms.sum()),
                conv_tflops=(conv_flops / (conv_ms * 1e-3) / 1e12) if conv_ms > 0 else 0.0,
                n_steps=int(len(ms)), n_conv=int(conv.sum()))


def roofline(tmp: str, iters: int):
    """Average duration of the conv_mfma launch on the 3x3/s1 64->64 160x160 layer."""
    model, x = ys.build_single_conv(**CONV_ROOF, seed=7)
    path = os.path.join(tmp, "conv3x3.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        eng.run(x)
        ms, kind, flops = eng.step_times(iters)
    finally:
        eng.close()
    i = int(np.nonzero(kind == KIND_CONV_MFMA)[0][0])
    assert int(flops[i]) == CONV_ROOF_FLOPS
    achieved = CONV_ROOF_FLOPS / (ms[i] * 1e-3) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    return dict(bound="mfma", achieved=round(achieved, 3), peak=MFMA_FP32_PEAK_TFLOPS, unit="TFLOP/s",
                frac=round(achieved / MFMA_FP32_PEAK_TFLOPS, 4), traffic=traffic,
                kernel="conv_mfma_kernel", launch_us=round(float(ms[i]) * 1e3, 2),
                workload="conv3x3 s1 p1 64->64 1x64x160x160 +bias+SiLU")


def cpu_baseline(path: str, x: np.ndarray, budget_s: float = 12.0):
    """The reference CPU engine (oracle/_ref, built from the reference sources)
    on the same YOLOv8n b1 workload: median Session::run over a bounded sample."""
    from oracle import ref_lib  # checker / baseline only

    if not ref_lib.available():
        return None
    threads = max(1, min(16, os.cpu_count() or 1))
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
    med = statistics.median(times)
    return dict(value=round(1000.0 / med, 3), unit="images/s", cores=threads, kind="reference",
                sample=f"YOLOv8n b1 640x640, median of {len(times)} Session::run after 3 warm-ups "
                       f"({med:.1f} ms), {threads} threads")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the reference CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("RANK", "0")) != 0:
        return

    log(f"device: {native.lib().pdefa_amd_device_name().decode()}")
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "yolov8n.engine")
        ys.save(ys.build_yolov8("n", seed=0), path)
        res = {}
        for batch in (1, 8):
            x, _ = ys.yolo_inputs(batch)
            eng = native.Engine(path)
            try:
                log(f"yolov8n b{batch}:")
                ms, wall = time_program(eng, x, args.steps, args.warmup)
                cs = conv_stats(eng, 20)
            finally:
                eng.close()
            res[batch] = dict(ms=ms, wall=wall, ips=batch * 1000.0 / ms, **cs)
            log(f"  {res[batch]['ips']:.1f} images/s, {ms:.4f} ms/step; convs {cs['conv_ms']:.4f} ms "
                f"({cs['conv_tflops']:.2f} TFLOP/s over {cs['n_conv']} convs, {cs['n_steps']} steps)")
        roof = roofline(tmp, 50)
        log(f"roofline conv3x3: {roof['launch_us']} us/launch, {roof['achieved']} TFLOP/s ({roof['frac']:.1%})")
        cpu = None
        if not args.no_cpu:
            x1, _ = ys.yolo_inputs(1)
            cpu = cpu_baseline(path, x1)
            if cpu:
                log(f"cpu baseline: {cpu['value']} images/s ({cpu['sample']})")

    b1, b8 = res[1], res[8]
    line = {
        "metric": METRIC,
        "value": round(b1["ips"], 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(b1["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(b1["ips"] / PUBLISHED_B1_IMAGES_PER_S, 2),
        "dtype": "f32",
        "data": "synthetic: seeded random-init YOLOv8n weights (BN folded), 1280x720 U[0,255] images letterboxed to 640x640",
        "config": {"workload": "yolov8n_640_b1", "model": "YOLOv8n (depth 0.33, width 0.25, 80 classes)",
                   "global_batch": 1, "seq_len": None, "parallelism": "single GPU",
                   "input": "1x3x640x640 fp32", "output": "1x84x8400"},
        "b8": {"value": round(b8["ips"], 2), "unit": "images/s", "ms_per_step": round(b8["ms"], 5),
               "conv_tflops": round(b8["conv_tflops"], 3)},
        "conv_tflops_b1": round(b1["conv_tflops"], 3),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
