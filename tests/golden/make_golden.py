"""Writes tests/golden/*.json from the reference CPU engine.

The reference (oracle/_ref/libpdefa_ref.so, compiled from the reference's own
sources by oracle/Makefile) is run on the seeded workloads of this repository
and small fixtures are kept: input/model digests, strided output samples,
per-channel means and the post-NMS detection list.  The reference's own tests
hold no golden vectors for this path, so these are the pinned vectors.

    make -C oracle && python tests/golden/make_golden.py [fixture names]
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import decode_ref, ref_lib  # noqa: E402
from pdefa_amd import yolo_synth as ys  # noqa: E402

N_SAMPLES = 2000


def sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


def samples(a: np.ndarray, n: int = N_SAMPLES):
    flat = a.reshape(-1)
    idx = np.unique(np.linspace(0, flat.size - 1, n).astype(np.int64))
    return {"index": idx.tolist(), "value": [float(v) for v in flat[idx]]}


def channel_means(a: np.ndarray):
    return [float(v) for v in a.reshape(a.shape[0], a.shape[1], -1).astype(np.float64).mean(axis=(0, 2))]


def file_sha(path: str) -> str:
    with open(path, "rb") as f:
        return sha(f.read())


def conv_case(tmp, name, cin, cout, k, s, hw, groups=1):
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=7, groups=groups)
    path = os.path.join(tmp, name + ".engine")
    ys.save(model, path)
    out = ref_lib.RefSession(path).run(x)[0]
    return {"cin": cin, "cout": cout, "k": k, "stride": s, "hw": hw, "seed": 7, "groups": groups,
            "engine_sha256": file_sha(path), "input_sha256": sha(x.tobytes()),
            "shape": list(out.shape), "samples": samples(out), "channel_means": channel_means(out)}


def yolo_case(tmp, scale, seed, batch_index=0, imgsz=640):
    model = ys.build_yolov8(scale, seed=seed, imgsz=imgsz)
    path = os.path.join(tmp, f"yolov8{scale}.engine")
    ys.save(model, path)
    x, metas = ys.yolo_inputs(batch_index + 1, imgsz=imgsz)
    x = x[batch_index:batch_index + 1]
    out = ref_lib.RefSession(path).run(x)[0]
    # a conf_thres with no best-class score within 1e-2 of it, so that outputs
    # within the parity tolerance select the same candidates
    conf, gap = decode_ref.robust_conf(out)
    if conf is None:
        raise SystemExit(f"yolov8{scale} image {batch_index}: no conf_thres with a 1e-2 score gap")
    dets = decode_ref.decode(out.tolist(), metas[batch_index], conf)
    return {"scale": scale, "weight_seed": seed, "image_index": batch_index, "imgsz": imgsz,
            "engine_sha256": file_sha(path), "input_sha256": sha(x.tobytes()), "meta": metas[batch_index],
            "shape": list(out.shape), "samples": samples(out), "channel_means": channel_means(out),
            "conf_thres": conf, "iou_thres": 0.45, "min_score_gap_to_threshold": gap,
            "min_iou_gap_to_threshold": decode_ref.min_iou_gap(out.tolist(), metas[batch_index], conf),
            "detections": dets}


def sgemm_case():
    rng = np.random.default_rng(42)
    a = rng.standard_normal((512, 512), dtype=np.float32)
    b = rng.standard_normal((512, 512), dtype=np.float32)
    c = ref_lib.matmul(a, b)
    return {"seed": 42, "a_sha256": sha(a.tobytes()), "b_sha256": sha(b.tobytes()),
            "samples": samples(c), "row_sums": [float(v) for v in c.astype(np.float64).sum(1)]}


def letterbox_case():
    img = ys.synth_image(0, 1280, 720)
    lb, meta = ref_lib.letterbox(img, 640, 640, 1.0 / 255.0, 114.0 / 255.0)
    return {"image_sha256": sha(img.tobytes()), "meta": meta, "samples": samples(lb),
            "output_sha256": sha(lb.tobytes())}


CASES = {
    "conv3x3_s1_64_160": lambda t: conv_case(t, "c2a", 64, 64, 3, 1, 160),
    "conv3x3_s2_64_160": lambda t: conv_case(t, "c2b", 64, 64, 3, 2, 160),
    "conv1x1_128_64_160": lambda t: conv_case(t, "c2c", 128, 64, 1, 1, 160),
    # grouped convs: depthwise (the reference's depthwise kernel) and groups
    # of 16 and 2 channels (its grouped GEMM)
    "dwconv3x3_s1_64_80": lambda t: conv_case(t, "g1", 64, 64, 3, 1, 80, groups=64),
    "dwconv3x3_s2_96_41": lambda t: conv_case(t, "g2", 96, 96, 3, 2, 41, groups=96),
    "gconv3x3_g4_64_40": lambda t: conv_case(t, "g3", 64, 64, 3, 1, 40, groups=4),
    "gconv3x3_g16_32_40": lambda t: conv_case(t, "g4", 32, 32, 3, 1, 40, groups=16),
    "yolov8n_640_img0": lambda t: yolo_case(t, "n", 0, 0),
    "yolov8n_640_img1": lambda t: yolo_case(t, "n", 0, 1),
    "yolov8n_640_img2": lambda t: yolo_case(t, "n", 0, 2),
    "yolov8m_640_img0": lambda t: yolo_case(t, "m", 1, 0),
    "yolov8m_640_img1": lambda t: yolo_case(t, "m", 1, 1),
    "sgemm_512": lambda t: sgemm_case(),
    "letterbox_1280x720": lambda t: letterbox_case(),
}


def main(names):
    """Writes the named fixtures (all when none is named)."""
    if not ref_lib.available():
        sys.exit("build the reference oracle first: make -C oracle")
    ref_lib.set_threads(8)
    unknown = [n for n in names if n not in CASES]
    if unknown:
        sys.exit(f"unknown fixtures: {unknown}")
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for name in names or CASES:
            out[name] = CASES[name](tmp)
    for name, case in out.items():
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(case, f, separators=(",", ":"))
        print("wrote", name)


if __name__ == "__main__":
    main(sys.argv[1:])
