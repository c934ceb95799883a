"""Benchmark: YOLOv8n 640x640 fp32 images/s on one MI355X (b1 and b8), plus
the conv roofline and the reference CPU engine timed on the host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
    python bench.py --only roofline [--calib-copy]   # the roofline layer alone (profiling runs)
    python bench.py --ingest-pmc FETCH.csv WRITE.csv TILE  # HBM traffic of the roofline launch -> profiles/

A step is one forward of the whole YOLOv8n device program over one batch of
synthetic letterboxed input already resident in HBM: the session's captured
hipGraph is replayed K times after W warm-up replays, timed with HIP events
on the session stream and with the host clock around a device synchronise on
both sides.  Prints ONE JSON line.

Roofline: the 3x3 s1 p1 64->64 conv + bias + SiLU on a 1x64x160x160 input
(1.887 GFLOP per launch).  Its average launch duration comes from HIP events
around back-to-back launches of that step on the session stream; `traffic`
is read from the PMC summary that --ingest-pmc writes (FETCH_SIZE and
WRITE_SIZE per dispatch, scaled by the same counters on a 64 MiB copy).
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
import subprocess
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
CALIB_SHAPE = (1, 16, 1024, 1024)  # 64 MiB in, 64 MiB out: larger than all L2s together
CALIB_BYTES = 4 * 16 * 1024 * 1024


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_program(eng: native.Engine, x: np.ndarray, steps: int, warmup: int):
    """ms per forward: W warm-up replays, then K timed replays of the graph."""
    t0 = time.perf_counter()
    eng.run(x)  # uploads the input, plans (timing conv candidates), captures the graph
    first_ms = (time.perf_counter() - t0) * 1e3
    if warmup > 0:
        eng.replay(warmup)
    t0 = time.perf_counter()
    dev_ms = eng.replay(steps)
    wall_ms = (time.perf_counter() - t0) * 1e3
    log(f"  first run (plan + tune + capture) {first_ms:.1f} ms; {steps} steps: device {dev_ms:.3f} ms, "
        f"host wall {wall_ms:.3f} ms")
    return max(dev_ms, 0.0) / steps, wall_ms / steps, first_ms


def launch_count(plan: str) -> int:
    """Launches of a prepared program: one per plan step, except that
    consecutive steps of one conv group share a grouped launch."""
    n, prev = 0, None
    for line in plan.splitlines()[1:]:
        if line.startswith("arena"):
            break
        g = line.split(" group=")[1].split()[0] if " group=" in line else None
        if g is None or g != prev:
            n += 1
        prev = g
    return n


def conv_stats(eng: native.Engine, iters: int):
    ms, kind, flops = eng.step_times(iters)
    conv = (kind == KIND_CONV_MFMA) | (kind == KIND_CONV_DIRECT)
    conv_ms = float(ms[conv].sum())
    conv_flops = int(flops[conv].sum())
    return dict(conv_ms=conv_ms, conv_flops=conv_flops, step_ms=float(ms.sum()),
                conv_tflops=(conv_flops / (conv_ms * 1e-3) / 1e12) if conv_ms > 0 else 0.0,
                n_steps=int(len(ms)), n_conv=int(conv.sum()))


def roofline_engine(tmp: str):
    model, x = ys.build_single_conv(**CONV_ROOF, seed=7)
    path = os.path.join(tmp, "conv3x3.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    eng.run(x)
    lines = eng.plan().splitlines()[1:]
    idx = [i for i, l in enumerate(lines) if " conv_mfma" in l][0]
    return eng, idx, lines[idx]


def roofline(tmp: str, iters: int):
    """Average duration of the conv_mfma launch on the 3x3/s1 64->64 160x160 layer."""
    eng, idx, line = roofline_engine(tmp)
    try:
        ms = eng.step_repeat(idx, iters)
    finally:
        eng.close()
    achieved = CONV_ROOF_FLOPS / (ms * 1e-3) / 1e12
    shape = line.split("(")[1].split(")")[0]
    tile = shape.split(",")[0].split("=")[1]
    # HBM bytes per launch measured for this launch shape (the measured choice
    # between close shapes can differ from run to run)
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("tiles", {}).get(tile, {}).get("hbm_bytes_per_launch")
    wino = "tile=wino" in shape
    out = dict(bound="mfma", achieved=round(achieved, 3), peak=MFMA_FP32_PEAK_TFLOPS, unit="TFLOP/s",
               frac=round(achieved / MFMA_FP32_PEAK_TFLOPS, 4), traffic=traffic,
               kernel="conv_wino_kernel" if wino else "conv_mfma_kernel", launch_shape=shape,
               launch_us=round(ms * 1e3, 2),
               workload="conv3x3 s1 p1 64->64 1x64x160x160 +bias+SiLU, 1.887 GFLOP/launch (direct-conv count)")
    if wino:
        # Winograd F(2x2,3x3) runs 16 * Cin * Cout MACs per 2x2 output tile
        executed = 2 * 16 * 64 * 64 * 80 * 80
        out["algorithm"] = "winograd F(2x2,3x3): 0.839 GFLOP of MFMA work per launch"
        out["mfma_tflops_executed"] = round(executed / (ms * 1e-3) / 1e12, 3)
    return out


def calibration_copy(tmp: str, iters: int = 5):
    """A plain streaming pass of known size for the PMC byte counters: ReLU of a
    64 MiB tensor (64 MiB read, 64 MiB written per dispatch)."""
    b = ys.GraphBuilder()
    y = b.node("Relu", "/calib/Relu", [-1])
    model = b.model(list(CALIB_SHAPE), list(CALIB_SHAPE), [y])
    path = os.path.join(tmp, "calib.engine")
    ys.save(model, path)
    x = np.random.default_rng(0).random(CALIB_SHAPE, dtype=np.float32)
    eng = native.Engine(path)
    try:
        eng.run(x)
        ms = eng.step_repeat(0, iters)
    finally:
        eng.close()
    log(f"calibration copy: {CALIB_BYTES / 2**20:.0f} MiB in + out, {ms * 1e3:.1f} us/dispatch "
        f"({2 * CALIB_BYTES / (ms * 1e-3) / 1e9:.0f} GB/s)")


def ingest_pmc(fetch_csv: str, write_csv: str, tile: str):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the roofline conv launches
    (run with PDEFA_CONV_TILE=tile) and of the calibration copy -> the entry
    for `tile` in profiles/conv3x3s1_64x64_160_traffic.json."""
    def read(path, counter):
        convs, calib = {}, []
        with open(path) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name, val = row["Kernel_Name"], float(row["Counter_Value"])
                if "conv_mfma_kernel" in name or "conv_wino_kernel" in name:
                    convs.setdefault(name, []).append(val)
                elif "eltwise_kernel" in name and int(row.get("Grid_Size", 0)) >= CALIB_BYTES // 4:
                    calib.append(val)
        if not convs or not calib:
            raise SystemExit(f"{path}: no {counter} rows for the conv or the calibration copy")
        # the planned kernel runs 50+ times; the other conv kernels are the
        # candidates timed while planning
        name = max(convs, key=lambda n: len(convs[n]))
        conv = convs[name]
        return statistics.median(conv), statistics.median(calib), len(conv), len(calib), name
    fc, fk, nfc, nfk, kname = read(fetch_csv, "FETCH_SIZE")
    wc, wk, nwc, nwk, _ = read(write_csv, "WRITE_SIZE")
    f_scale = CALIB_BYTES / (fk * 1024.0)
    w_scale = CALIB_BYTES / (wk * 1024.0)
    read_b = fc * 1024.0 * f_scale
    write_b = wc * 1024.0 * w_scale
    algo = 4 * (64 * 160 * 160 * 2 + 64 * 64 * 9 + 64)  # input + output + weights + bias
    entry = dict(kernel=kname, fetch_kib_per_dispatch=fc, write_kib_per_dispatch=wc, conv_dispatches=[nfc, nwc],
                 calib_fetch_kib=fk, calib_write_kib=wk, calib_dispatches=[nfk, nwk],
                 calib_bytes_each_way=CALIB_BYTES, fetch_scale=round(f_scale, 4), write_scale=round(w_scale, 4),
                 hbm_read_bytes_per_launch=round(read_b), hbm_write_bytes_per_launch=round(write_b),
                 hbm_bytes_per_launch=round(read_b + write_b))
    out = {"layer": "conv 3x3 s1 p1 64->64, 1x64x160x160", "algorithmic_bytes_per_launch": algo, "tiles": {}}
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            old = json.load(f)
        out["tiles"] = old.get("tiles", {})
    out["tiles"][tile] = entry
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def pipeline(path: str, batch: int = 8, iters: int = 20):
    """8-bit images in host memory -> post-NMS detections in host memory, per
    batch of YOLOv8n: letterbox (on the GPU from the pixels), the program and
    decode + NMS (on the GPU), against the same session fed by the host
    letterbox with decode_yolo on the host."""
    from pdefa_amd import pdefa

    raws = [ys.synth_image(i, *ys.ASPECT_SIZES[i % len(ys.ASPECT_SIZES)]) for i in range(batch)]
    imgs = [pdefa.Image.from_array(a) for a in raws]
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, path)
    s = pdefa.Session(ctx, model)
    args = (640, 640, 1.0 / 255.0, 114.0 / 255.0)

    def device_pass():
        metas = s.set_images(0, imgs, *args)
        s.run()
        return s.decode(metas)

    def host_pass():
        pre = [pdefa.preprocess_letterbox(im, *args) for im in imgs]
        s.set_input(0, pdefa.ops_concat([t for t, _ in pre], axis=0))
        s.run()
        out = s.output(0).to_numpy()
        return [pdefa.decode_yolo(out[i:i + 1], pre[i][1]) for i in range(batch)]

    dev, host = device_pass(), host_pass()
    same = all([{k: v for k, v in d.items()} for d in a] == b for a, b in zip(dev, host))
    t0 = time.perf_counter()
    for _ in range(iters):
        device_pass()
    dev_ms = (time.perf_counter() - t0) * 1e3 / iters
    h_iters = max(1, iters // 4)
    t0 = time.perf_counter()
    for _ in range(h_iters):
        host_pass()
    host_ms = (time.perf_counter() - t0) * 1e3 / h_iters
    n_det = sum(len(d) for d in dev)
    return dict(workload=f"YOLOv8n b{batch}: {batch} synthetic 8-bit images (1280x720, 1024x768, 800x800) in host "
                         f"memory -> post-NMS detections ({n_det} boxes) in host memory",
                value=round(batch * 1000.0 / dev_ms, 2), unit="images/s", ms_per_batch=round(dev_ms, 3),
                host_pre_post=dict(value=round(batch * 1000.0 / host_ms, 2), ms_per_batch=round(host_ms, 3),
                                   note="host letterbox (C++), H2D of the float tensor, host decode_yolo"),
                same_detections=bool(same))


def cpu_baseline(path: str, x: np.ndarray, budget_s: float = 12.0):
    """The reference CPU engine (oracle/_ref, built from the reference sources)
    on the same YOLOv8n b1 workload: median Session::run over a bounded sample,
    timed in a child process (oracle/ref_bench.py) so that the reference's
    worker threads begin and end there."""
    from oracle import ref_lib  # checker / baseline only

    if not ref_lib.available():
        return None
    threads = max(1, min(16, os.cpu_count() or 1))
    npy = os.path.join(os.path.dirname(path), "cpu_baseline_input.npy")
    np.save(npy, x)
    try:
        r = subprocess.run([sys.executable, "-m", "oracle.ref_bench", path, npy, str(budget_s), str(threads)],
                           cwd=ROOT, capture_output=True, text=True, timeout=budget_s + 120)
    except subprocess.TimeoutExpired:
        log("cpu baseline: the reference run did not finish")
        return None
    if r.returncode != 0 or not r.stdout.strip():
        log(f"cpu baseline: the reference run failed ({r.returncode}): {r.stderr[-400:]}")
        return None
    times = json.loads(r.stdout.strip().splitlines()[-1])["ms"]
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
    ap.add_argument("--no-m16", action="store_true", help="skip the YOLOv8m batch-16 line")
    ap.add_argument("--no-pipeline", action="store_true", help="skip the pixels-to-detections pipeline line")
    ap.add_argument("--only", choices=["all", "roofline", "program"], default="all",
                    help="program: plan YOLOv8n at --batch, then only warm-up and timed graph replays "
                         "(a kernel trace's last steps x launches dispatches are the timed forwards)")
    ap.add_argument("--batch", type=int, default=1, help="with --only program: the batch size")
    ap.add_argument("--calib-copy", action="store_true", help="with --only roofline: also run the PMC calibration copy")
    ap.add_argument("--ingest-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "TILE"))
    args = ap.parse_args()
    if args.ingest_pmc:
        ingest_pmc(*args.ingest_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("RANK", "0")) != 0:
        return

    log(f"device: {native.lib().pdefa_amd_device_name().decode()}")
    if args.only == "program":
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "yolov8n.engine")
            ys.save(ys.build_yolov8("n", seed=0), path)
            x, _ = ys.yolo_inputs(args.batch)
            eng = native.Engine(path)
            try:
                log(f"yolov8n b{args.batch}:")
                ms, wall, first = time_program(eng, x, args.steps, args.warmup)
                launches = launch_count(eng.plan())
            finally:
                eng.close()
        print(json.dumps({"program": {"workload": f"yolov8n_640_b{args.batch}", "batch": args.batch,
                                      "launches": launches, "steps": args.steps, "warmup": args.warmup,
                                      "ms_per_step": round(ms, 5),
                                      "images_per_s": round(args.batch * 1000.0 / ms, 2)}}), flush=True)
        return
    if args.only == "roofline":
        with tempfile.TemporaryDirectory() as tmp:
            roof = roofline(tmp, 50)
            log(f"roofline conv3x3 [{roof['launch_shape']}]: {roof['launch_us']} us/launch, "
                f"{roof['achieved']} TFLOP/s ({roof['frac']:.1%})")
            if args.calib_copy:
                calibration_copy(tmp)
        print(json.dumps({"roofline": roof}), flush=True)
        return

    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "yolov8n.engine")
        ys.save(ys.build_yolov8("n", seed=0), path)
        res = {}
        for batch in (1, 8):
            x, _ = ys.yolo_inputs(batch)
            eng = native.Engine(path)
            try:
                log(f"yolov8n b{batch}:")
                ms, wall, first = time_program(eng, x, args.steps, args.warmup)
                cs = conv_stats(eng, 20)
            finally:
                eng.close()
            res[batch] = dict(ms=ms, wall=wall, first=first, ips=batch * 1000.0 / ms, **cs)
            log(f"  {res[batch]['ips']:.1f} images/s, {ms:.4f} ms/step; convs {cs['conv_ms']:.4f} ms "
                f"({cs['conv_tflops']:.2f} TFLOP/s over {cs['n_conv']} convs, {cs['n_steps']} steps)")
        m16 = None
        if not args.no_m16:
            mpath = os.path.join(tmp, "yolov8m.engine")
            ys.save(ys.build_yolov8("m", seed=1), mpath)
            x, _ = ys.yolo_inputs(16)
            eng = native.Engine(mpath)
            try:
                log("yolov8m b16:")
                ms, wall, first = time_program(eng, x, max(5, args.steps // 10), max(1, args.warmup // 10))
            finally:
                eng.close()
            m16 = dict(value=round(16000.0 / ms, 2), unit="images/s", ms_per_step=round(ms, 4),
                       first_run_ms=round(first, 1))
            log(f"  {m16['value']} images/s")
        roof = roofline(tmp, 50)
        log(f"roofline conv3x3 [{roof['launch_shape']}]: {roof['launch_us']} us/launch, "
            f"{roof['achieved']} TFLOP/s ({roof['frac']:.1%})")
        pipe = None
        if not args.no_pipeline:
            pipe = pipeline(path)
            log(f"pipeline b8 (pixels -> detections): {pipe['value']} images/s with letterbox + decode on the GPU, "
                f"{pipe['host_pre_post']['value']} images/s with them on the host; same detections: "
                f"{pipe['same_detections']}")
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
        "yolov8m_b16": m16,
        "conv_tflops_b1": round(b1["conv_tflops"], 3),
        "first_run_ms": {"b1": round(b1["first"], 1), "b8": round(b8["first"], 1)},
        "pipeline_b8": pipe,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
