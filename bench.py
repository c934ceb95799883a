"""Benchmark: YOLOv8n 640x640 fp32 images/s on one MI355X (b1 and b8), plus
the conv roofline and the reference CPU engine timed on the host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
    python bench.py --only roofline [--calib-copy]   # the roofline layer alone (profiling runs)
    python bench.py --only program --batch B [--calib-copy]  # one batch size's replays alone
    python bench.py --ingest-pmc FETCH.csv WRITE.csv TILE  # HBM traffic of the roofline launch -> profiles/
    python bench.py --ingest-counters NAME --trace T.csv --mfma M.csv [--fetch F.csv --write W.csv]

A step is one engine_session_run of YOLOv8n at batch 1 with the input in host
memory: one H2D copy of the letterboxed 1x3x640x640 input, the whole device
program, one D2H copy of the 1x84x8400 head and a synchronise -- the quantity
the reference's own benchmark times (session.run(), bench_models.py:226-241,
269-277).  W untimed runs, then K runs each timed with the host clock (the
call returns after its synchronise); `value` is images/s at the median run,
as the reference takes it.  Beside it, `replay` reports the captured
hipGraph replayed with the input already resident in HBM (K replays after W,
timed with HIP events on the session stream), and batch 8 both ways.
Prints ONE JSON line.

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
CALIB_SHAPE = (4096, 4096)  # 64 MiB in, 64 MiB out, contiguous: larger than all L2s together
CALIB_BYTES = 4 * 16 * 1024 * 1024
# the calibration dispatch: an elementwise kernel with at least one lane per
# 4 elements of the 64 MiB tensor (no other elementwise launch is as large)
CALIB_GRID = CALIB_BYTES // 16
CALIB_KEY = "calibration copy (eltwise, 64 MiB ReLU)"


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
    return len(plan_launches(plan))


def conv_stats(eng: native.Engine, iters: int):
    ms, kind, flops = eng.step_times(iters)
    conv = (kind == KIND_CONV_MFMA) | (kind == KIND_CONV_DIRECT)
    conv_ms = float(ms[conv].sum())
    conv_flops = int(flops[conv].sum())
    return dict(conv_ms=conv_ms, conv_flops=conv_flops, step_ms=float(ms.sum()),
                conv_tflops=(conv_flops / (conv_ms * 1e-3) / 1e12) if conv_ms > 0 else 0.0,
                n_steps=int(len(ms)), n_conv=int(conv.sum()))


def plan_launches(plan: str):
    """The plan's step lines grouped by launch (consecutive steps of one conv
    group share a grouped launch), in launch order."""
    out, prev = [], None
    for line in plan.splitlines()[1:]:
        if line.startswith("arena"):
            break
        g = line.split(" group=")[1].split()[0] if " group=" in line else None
        if g is None or g != prev:
            out.append([])
        out[-1].append(line)
        prev = g
    return out


def conv3x3_layers(eng: native.Engine, iters: int = 20):
    """Every launch of the forward whose convs are all 3x3, timed back to back
    on the session stream (step_repeat: the launch boundary included, like
    the roofline layer), in direct-conv flops (2*N*Ho*Wo*Cout*Cin*9) against
    the fp32 MFMA peak.  MFMA launches (Winograd and implicit GEMM) are
    summarised by stride; the direct-kernel stem (VALU) is listed apart."""
    _, kind, flops = eng.step_times(1)
    rows = []
    for i, lines in enumerate(plan_launches(eng.plan())):
        if not all(" k=3x3 " in l for l in lines):
            continue
        ms = eng.step_repeat(i, iters)
        fl = int(flops[i])
        tf = fl / (ms * 1e-3) / 1e12
        first = lines[0]
        rows.append(dict(launch=i, stride=int(first.split(" s=")[1].split("x")[0]),
                         kernel="direct" if int(kind[i]) == KIND_CONV_DIRECT else
                         ("wino" if "tile=wino" in first else "gemm"),
                         tile=first.split("tile=")[1].split(",")[0] if "tile=" in first else "direct",
                         convs=len(lines), names=[l.split("'")[1] for l in lines], us=round(ms * 1e3, 2),
                         gflop=round(fl / 1e9, 4), tflops=round(tf, 2),
                         frac=round(tf / MFMA_FP32_PEAK_TFLOPS, 4)))

    def agg(rs):
        if not rs:
            return None
        us = sum(r["us"] for r in rs)
        gf = sum(r["gflop"] for r in rs)
        tf = gf * 1e9 / (us * 1e-6) / 1e12
        return dict(launches=len(rs), us=round(us, 2), gflop=round(gf, 3), tflops=round(tf, 2),
                    frac=round(tf / MFMA_FP32_PEAK_TFLOPS, 4),
                    launches_at_50pct=int(sum(r["frac"] >= 0.5 for r in rs)),
                    min_frac=min(r["frac"] for r in rs), max_frac=max(r["frac"] for r in rs))

    mf = [r for r in rows if r["kernel"] != "direct"]
    summary = dict(mfma=agg(mf), s1=agg([r for r in mf if r["stride"] == 1]),
                   s2=agg([r for r in mf if r["stride"] == 2]),
                   direct=[{k: r[k] for k in ("names", "us", "tflops", "frac")} for r in rows
                           if r["kernel"] == "direct"])
    return summary, rows


def log_layers(rows):
    for r in rows:
        log(f"  3x3 s{r['stride']} {r['kernel']:6s} {r['tile']:10s} {r['us']:8.2f} us {r['gflop']:8.4f} GFLOP "
            f"{r['tflops']:7.2f} TFLOP/s {r['frac']:6.1%}  {' + '.join(r['names'])}")


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
        out["frac_executed"] = round(out["mfma_tflops_executed"] / MFMA_FP32_PEAK_TFLOPS, 4)
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
                elif "eltwise" in name and int(row.get("Grid_Size", 0)) >= CALIB_GRID:
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


def median_upper(ts):
    """The median as the reference's bench_models.py:236-238 takes it (the
    upper one of an even count)."""
    return sorted(ts)[len(ts) // 2]


def host_cores() -> int:
    """CPUs this process may run on, capped at 16 (a one-GPU box's share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(path: str, x: np.ndarray):
    """The reference CPU engine (oracle/_ref, built from the reference sources)
    on the same YOLOv8n b1 workload with the protocol of its own benchmark
    (bench_models.py:61-62,226-241: one untimed run, 5 warm-ups, median of 30
    Session::run), with all of this host's cores and with 12 threads (the
    reference README's setting); each count timed in a child process
    (oracle/ref_bench.py) so that the reference's worker threads begin and
    end there."""
    from oracle import ref_lib  # checker / baseline only

    if not ref_lib.available():
        return None
    npy = os.path.join(os.path.dirname(path), "cpu_baseline_input.npy")
    np.save(npy, x)
    res, aborts = {}, {}
    for threads in sorted({host_cores(), 12}, reverse=True):
        aborts[threads] = 0
        # A child that aborts is started once more: the reference's
        # ThreadPool::parallel_for keeps its completion mutex and condition
        # variable in the caller's frame (PDEFA1.0/src/runtime/thread_pool.cpp:
        # 154,170) and its last worker can lock them after the caller has
        # returned, which glibc reports as a failed pthread_mutex_lock
        # assertion (SIGABRT).  The child is a CPU-only process.
        for attempt in range(2):
            try:
                r = subprocess.run([sys.executable, "-m", "oracle.ref_bench", path, npy, str(threads), "30", "5"],
                                   cwd=ROOT, capture_output=True, text=True, timeout=180)
            except subprocess.TimeoutExpired:
                log(f"cpu baseline: the reference run with {threads} threads did not finish")
                break
            if r.returncode == 0 and r.stdout.strip():
                times = json.loads(r.stdout.strip().splitlines()[-1])["ms"]
                res[threads] = median_upper(times)
                log(f"cpu baseline: {threads} threads, median {res[threads]:.2f} ms over {len(times)} runs")
                break
            aborts[threads] += 1
            log(f"cpu baseline: the reference run with {threads} threads failed ({r.returncode}), "
                f"attempt {attempt + 1}: {r.stderr[-300:]}")
    if not res:
        return None
    cores = host_cores() if host_cores() in res else max(res)
    out = dict(value=round(1000.0 / res[cores], 3), unit="images/s", cores=cores, kind="reference",
               sample=f"YOLOv8n b1 640x640 (the bench's b1 input), the reference engine compiled from its sources: "
                      f"median of 30 Session::run after 1 + 5 warm-ups ({res[cores]:.2f} ms) with {cores} "
                      f"threads (all of this host's cores, at most 16)",
               threads={str(t): (dict(value=round(1000.0 / res[t], 3), median_ms=round(res[t], 3), aborts=aborts[t])
                                 if t in res else dict(value=None, aborts=aborts[t])) for t in aborts},
               aborts_note=("a child process that aborts (the reference's thread-pool race, "
                            "PDEFA1.0/src/runtime/thread_pool.cpp:154,170) is started once more; "
                            "aborts counts the failed children per thread count"))
    return out


def session_run_stats(eng: native.Engine, batch: int, warmup: int = 5, runs: int = 30):
    """images/s from the median wall time of engine_session_run with the
    input in host memory (one H2D copy of the input, the program, one D2H
    copy of the output, a synchronise), as the reference's benchmark times
    session.run() (bench_models.py:226-241,269-277)."""
    ts = eng.session_run_times(warmup, runs)
    med = median_upper(ts)
    return dict(images_per_s=round(batch * 1000.0 / med, 2), median_ms=round(med, 4), min_ms=round(min(ts), 4),
                p95_ms=round(sorted(ts)[int(0.95 * len(ts))], 4), runs=runs, warmup=warmup)


COUNTER_DIR = os.path.join(ROOT, "profiles")
BANDWIDTH_KERNELS = ("maxpool_chain_kernel", "maxpool_chain_vec_kernel", "detect_head_kernel", "detect_decode_kernel",
                     "eltwise_kernel", "eltwise_vec_kernel", "transpose_elt_kernel", "calibration copy",
                     "resize_nearest_kernel", "maxpool_kernel", "softmax_kernel", "letterbox_kernel")


def _kernel_key(name: str) -> str:
    """A kernel's template instance without its parameter list."""
    name = name.strip()
    if name.startswith("void "):
        name = name[5:]
    depth, out = 0, []
    for ch in name:
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out).replace("pdefa::k::", "")


def _read_rows(path):
    with open(path) as f:
        return list(csv.DictReader(f))


def ingest_counters(name: str, trace_csv: str, mfma_csv: str, fetch_csv: str = None, write_csv: str = None,
                    command: str = ""):
    """Per-kernel summary of one profiled workload -> profiles/counters_<name>.{json,md}.

    trace_csv: rocprofv3 --kernel-trace of the workload (durations);
    mfma_csv: rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_F32 of the same
    workload (MfmaUtil = MFMA-busy cycles over all SIMDs / (GPU-busy cycles x
    SIMDs); the MOPS counter x 512 = fp32 MFMA flops executed);
    fetch_csv / write_csv: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) runs
    with the 64 MiB calibration copy, which scales each counter to bytes."""
    calib_grid = CALIB_GRID
    dur, calls = {}, {}
    for r in _read_rows(trace_csv):
        k = _kernel_key(r["Kernel_Name"])
        grid = int(r.get("Grid_Size") or r.get("Grid_Size_X") or 0)
        if "eltwise" in k and grid >= calib_grid:
            k = CALIB_KEY
        dur.setdefault(k, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    def counter(path, cname):
        vals = {}
        for r in _read_rows(path):
            if r.get("Counter_Name") != cname:
                continue
            k = _kernel_key(r["Kernel_Name"])
            if "eltwise" in k and int(r.get("Grid_Size", 0) or 0) >= calib_grid:
                k = CALIB_KEY
            vals.setdefault(k, []).append(float(r["Counter_Value"]))
        return vals
    util = counter(mfma_csv, "MfmaUtil")
    mops = counter(mfma_csv, "SQ_INSTS_VALU_MFMA_MOPS_F32")
    fetch = counter(fetch_csv, "FETCH_SIZE") if fetch_csv else {}
    write = counter(write_csv, "WRITE_SIZE") if write_csv else {}
    calib = CALIB_KEY
    f_scale = w_scale = None
    if calib in fetch and calib in write:
        f_scale = CALIB_BYTES / (statistics.median(fetch[calib]) * 1024.0)
        w_scale = CALIB_BYTES / (statistics.median(write[calib]) * 1024.0)
    kernels = []
    for k, ds in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        e = dict(kernel=k, calls=len(ds), avg_us=round(statistics.mean(ds), 3), total_us=round(sum(ds), 2))
        if k in util:
            e["mfma_util_pct"] = round(statistics.mean(util[k]), 2)
        if k in mops and statistics.mean(mops[k]) > 0:
            fl = statistics.mean(mops[k]) * 512.0
            e["mfma_gflop_per_call"] = round(fl / 1e9, 5)
            e["mfma_tflops_executed"] = round(fl / (e["avg_us"] * 1e-6) / 1e12, 3)
            e["mfma_frac_of_peak"] = round(e["mfma_tflops_executed"] / MFMA_FP32_PEAK_TFLOPS, 4)
        if f_scale and k in fetch and k in write:
            b = statistics.mean(fetch[k]) * 1024.0 * f_scale + statistics.mean(write[k]) * 1024.0 * w_scale
            e["hbm_bytes_per_call"] = round(b)
            e["hbm_gbs"] = round(b / (e["avg_us"] * 1e-6) / 1e9, 1)
            e["hbm_frac_of_peak"] = round(e["hbm_gbs"] / HBM_PEAK_GBS, 4)
        kernels.append(e)
    # YOLO programs: one detect_head_kernel launch per forward, so its call
    # count is the number of forwards in the trace; kernels launched a whole
    # number of times per forward are the forward's (the weight packing and
    # the calibration copy run once per process)
    heads = [e["calls"] for e in kernels if e["kernel"].startswith("detect_head_kernel")]
    forwards = heads[0] if len(heads) == 1 else None
    if forwards:
        for e in kernels:
            if e["calls"] % forwards == 0:
                e["per_forward"] = e["calls"] // forwards
                e["us_per_forward"] = round(e["total_us"] / forwards, 2)
    fw = [e for e in kernels if "per_forward" in e]
    per_fw = dict(launches=sum(e["per_forward"] for e in fw),
                  kernel_us=round(sum(e["us_per_forward"] for e in fw), 2)) if forwards else None
    conv = [e for e in kernels if e["kernel"].startswith("conv_")]
    conv_us = sum(e["total_us"] for e in conv)
    conv_fl = sum(e.get("mfma_gflop_per_call", 0.0) * 1e9 * e["calls"] for e in conv)
    util_w = sum(e.get("mfma_util_pct", 0.0) * e["total_us"] for e in conv)
    out = dict(workload=name, command=command, calibration=dict(fetch_scale=f_scale, write_scale=w_scale),
               forwards=forwards, per_forward=per_fw,
               conv=dict(total_us=round(conv_us, 2),
                         mfma_tflops_executed=round(conv_fl / (conv_us * 1e-6) / 1e12, 3) if conv_us else None,
                         mfma_util_pct_time_weighted=round(util_w / conv_us, 2) if conv_us else None),
               kernels=kernels)
    os.makedirs(COUNTER_DIR, exist_ok=True)
    with open(os.path.join(COUNTER_DIR, f"counters_{name}.json"), "w") as f:
        json.dump(out, f, indent=1)
    lines = [f"# Counters: {name}", "", "Commands (GPU box, repo root, `export TMPDIR=/tmp`):", "",
             *[f"    {c}" for c in command.split(" ;; ") if c], "",
             "Per kernel template: calls, average duration (kernel trace), MfmaUtil (MFMA-busy cycles over all "
             "SIMDs / GPU-busy cycles x SIMDs), fp32 MFMA work executed (SQ_INSTS_VALU_MFMA_MOPS_F32 x 512) per "
             "call and its rate over the traced duration, HBM bytes per call (FETCH_SIZE + WRITE_SIZE scaled by "
             "the same counters on a 64 MiB copy) and their rate.", "",
             f"Conv kernels: {out['conv']['total_us']} us in total, "
             f"{out['conv']['mfma_tflops_executed']} TFLOP/s of MFMA work executed "
             f"({(out['conv']['mfma_tflops_executed'] or 0) / MFMA_FP32_PEAK_TFLOPS:.1%} of 157.3), "
             f"MfmaUtil {out['conv']['mfma_util_pct_time_weighted']}% (time-weighted)."
             + (f"  Calibration: FETCH_SIZE x {f_scale:.3f}, WRITE_SIZE x {w_scale:.3f}." if f_scale else ""),
             ""]
    if forwards:
        lines += [f"{forwards} forwards in the trace (detect_head_kernel calls): per forward "
                  f"{per_fw['launches']} launches, {per_fw['kernel_us']:.1f} us of kernel time (`/fwd` launches and "
                  f"`us/fwd` time per forward; the kernels without them run once per process).", ""]
    lines.append("```")
    for e in kernels:
        parts = [f"{e['kernel'][:64]:64s}", f"x{e['calls']:5d}", f"{e['avg_us']:9.2f} us"]
        if "per_forward" in e:
            parts.append(f"{e['per_forward']:3d}/fwd {e['us_per_forward']:8.2f} us/fwd")
        if "mfma_util_pct" in e:
            parts.append(f"MfmaUtil {e['mfma_util_pct']:6.2f}%")
        if "mfma_tflops_executed" in e:
            parts.append(f"MFMA {e['mfma_tflops_executed']:7.2f} TFLOP/s")
        if "hbm_gbs" in e:
            parts.append(f"HBM {e['hbm_bytes_per_call'] / 1e6:8.3f} MB {e['hbm_gbs']:7.1f} GB/s")
        lines.append("  ".join(parts))
    lines.append("```")
    with open(os.path.join(COUNTER_DIR, f"counters_{name}.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(out["conv"]))


def counters_summary():
    """The committed counter summaries (profiles/counters_*.json), condensed
    for the bench line."""
    out = {}
    for name in ("roofline", "yolov8n_b1", "yolov8n_b8"):
        path = os.path.join(COUNTER_DIR, f"counters_{name}.json")
        if not os.path.exists(path):
            continue
        with open(path) as f:
            c = json.load(f)
        e = dict(conv=c["conv"])
        bw = {k["kernel"]: dict(avg_us=k["avg_us"], hbm_gbs=k["hbm_gbs"], frac=k["hbm_frac_of_peak"])
              for k in c["kernels"] if "hbm_gbs" in k and any(b in k["kernel"] for b in BANDWIDTH_KERNELS)}
        if bw:
            e["bandwidth_kernels"] = bw
        out[name] = e
    return out or None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the reference CPU baseline")
    ap.add_argument("--no-m16", action="store_true", help="skip the YOLOv8m batch-16 line")
    ap.add_argument("--no-pipeline", action="store_true", help="skip the pixels-to-detections pipeline line")
    ap.add_argument("--only", choices=["all", "roofline", "program", "layers", "session_run"], default="all",
                    help="program: plan YOLOv8n at --batch, then only warm-up and timed graph replays "
                         "(a kernel trace's last steps x launches dispatches are the timed forwards); "
                         "layers: YOLOv8n's 3x3 conv launches at --batch, one by one; "
                         "session_run: engine_session_run of YOLOv8n at --batch alone")
    ap.add_argument("--batch", type=int, default=1, help="with --only program / layers / session_run: the batch size")
    ap.add_argument("--calib-copy", action="store_true",
                    help="with --only roofline / program: also run the PMC calibration copy")
    ap.add_argument("--ingest-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "TILE"))
    ap.add_argument("--ingest-counters", metavar="NAME",
                    help="write profiles/counters_NAME.{json,md} from --trace, --mfma [, --fetch, --write]")
    ap.add_argument("--trace")
    ap.add_argument("--mfma")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--command", default="")
    args = ap.parse_args()
    if args.ingest_pmc:
        ingest_pmc(*args.ingest_pmc)
        return
    if args.ingest_counters:
        ingest_counters(args.ingest_counters, args.trace, args.mfma, args.fetch, args.write, args.command)
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
            if args.calib_copy:
                calibration_copy(tmp)
        print(json.dumps({"program": {"workload": f"yolov8n_640_b{args.batch}", "batch": args.batch,
                                      "launches": launches, "steps": args.steps, "warmup": args.warmup,
                                      "ms_per_step": round(ms, 5),
                                      "images_per_s": round(args.batch * 1000.0 / ms, 2)}}), flush=True)
        return
    if args.only == "session_run":
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "yolov8n.engine")
            ys.save(ys.build_yolov8("n", seed=0), path)
            x, _ = ys.yolo_inputs(args.batch)
            eng = native.Engine(path)
            try:
                eng.run(x)
                sr = session_run_stats(eng, args.batch, warmup=args.warmup, runs=args.steps)
            finally:
                eng.close()
        log(f"yolov8n b{args.batch} engine_session_run: median {sr['median_ms']} ms, {sr['images_per_s']} images/s")
        print(json.dumps({"session_run": {f"b{args.batch}": sr}}), flush=True)
        return
    if args.only == "layers":
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "yolov8n.engine")
            ys.save(ys.build_yolov8("n", seed=0), path)
            x, _ = ys.yolo_inputs(args.batch)
            eng = native.Engine(path)
            try:
                eng.run(x)
                c3, rows = conv3x3_layers(eng)
            finally:
                eng.close()
        log(f"yolov8n b{args.batch} 3x3 launches:")
        log_layers(rows)
        print(json.dumps({"conv3x3_layers": {f"b{args.batch}": c3}}), flush=True)
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
                sr = session_run_stats(eng, batch, warmup=args.warmup, runs=args.steps)
                c3, c3_rows = conv3x3_layers(eng)
            finally:
                eng.close()
            log_layers(c3_rows)
            res[batch] = dict(ms=ms, wall=wall, first=first, ips=batch * 1000.0 / ms, session_run=sr, conv3x3=c3,
                              **cs)
            log(f"  {res[batch]['ips']:.1f} images/s replayed from HBM, {ms:.4f} ms/step; engine_session_run "
                f"(host input and output) median {sr['median_ms']:.4f} ms = {sr['images_per_s']} images/s; convs "
                f"{cs['conv_ms']:.4f} ms launch by launch ({cs['n_conv']} convs, {cs['n_steps']} launches)")
        m16 = None
        if not args.no_m16:
            mpath = os.path.join(tmp, "yolov8m.engine")
            ys.save(ys.build_yolov8("m", seed=1), mpath)
            x, _ = ys.yolo_inputs(16)
            eng = native.Engine(mpath)
            try:
                log("yolov8m b16:")
                ms, wall, first = time_program(eng, x, max(20, args.steps // 10), max(5, args.warmup // 4))
                sr = session_run_stats(eng, 16, warmup=5, runs=30)
            finally:
                eng.close()
            m16 = dict(value=round(16000.0 / ms, 2), unit="images/s", ms_per_step=round(ms, 4),
                       first_run_ms=round(first, 1), session_run=sr)
            log(f"  {m16['value']} images/s replayed; engine_session_run {sr['images_per_s']} images/s")
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
        "value": b1["session_run"]["images_per_s"],
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": b1["session_run"]["median_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(b1["session_run"]["images_per_s"] / PUBLISHED_B1_IMAGES_PER_S, 2),
        "vs_baseline_basis": ("engine_session_run b1 images/s / 27.0 (the reference's published 37 ms per "
                              "session.run() of YOLOv8n 640 b1, README.md:629,635, Ryzen 5 7535HS, 12 threads)"),
        "dtype": "f32",
        "data": "synthetic: seeded random-init YOLOv8n weights (BN folded), 1280x720 U[0,255] images letterboxed to 640x640",
        "config": {"workload": "yolov8n_640_b1", "model": "YOLOv8n (depth 0.33, width 0.25, 80 classes)",
                   "global_batch": 1, "seq_len": None, "parallelism": "single GPU",
                   "input": "1x3x640x640 fp32 in host memory (engine_session_set_input tensor)",
                   "output": "1x84x8400 fp32 in host memory (engine_session_get_output tensor)",
                   "step": "one engine_session_run: H2D of the input, the device program, D2H of the output, "
                           "synchronise; median of K after W"},
        "session_run": {
            "note": ("engine_session_run wall time with the input in host memory: H2D of the input, the program, "
                     "D2H of the output, a synchronise (the reference benchmark's session.run(), "
                     "bench_models.py:226-241,269-277), median of --steps after --warmup"),
            "b1": b1["session_run"], "b8": b8["session_run"]},
        "replay": {
            "note": ("the captured hipGraph replayed with the input already resident in HBM and the output left "
                     "there: --steps replays after --warmup, HIP events on the session stream"),
            "b1": {"value": round(b1["ips"], 2), "unit": "images/s", "ms_per_step": round(b1["ms"], 5)},
            "b8": {"value": round(b8["ips"], 2), "unit": "images/s", "ms_per_step": round(b8["ms"], 5)}},
        "yolov8m_b16": m16,
        "first_run_ms": {"b1": round(b1["first"], 1), "b8": round(b8["first"], 1)},
        "pipeline_b8": pipe,
        "roofline": roof,
        "conv3x3_layers": {
            "note": ("every 3x3 conv launch of the YOLOv8n forward timed back to back, direct-conv flops "
                     "(2*N*Ho*Wo*Cout*Cin*9) over the fp32 MFMA peak; Winograd and implicit-GEMM launches by stride, "
                     "the VALU stem apart"),
            "b1": b1["conv3x3"], "b8": b8["conv3x3"]},
        "counters": counters_summary(),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
