"""YOLO head decode + per-class greedy NMS on the host.

Restates the reference's decode_yolo / _iou / _nms
(pdefa/python/src/pdefa/_bindings.py:1095-1212) with numpy doing the anchor
scan: per anchor the first maximum class score wins, anchors scoring below
conf_thres are dropped, xywh becomes xyxy, boxes map back through the
letterbox (clamped to the original image), then per class the boxes are
visited by descending score (stable on ties) and a box survives when its IoU
(with a 1e-9 guard) with every kept box is <= iou_thres; survivors are sorted
by score (stable) and cut to max_det.  Arithmetic is float64 on the float32
scores/boxes, as the reference's Python floats are.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np


def _as_heads(output) -> np.ndarray:
    arr = np.asarray(output, dtype=np.float32)
    while arr.ndim > 2 and arr.shape[0] == 1:
        arr = arr[0]
    if arr.ndim != 2 or arr.shape[0] < 5:
        raise ValueError(f"decode_yolo: unexpected output shape {arr.shape}")
    return arr


def candidates(output, conf_thres: float = 0.25):
    """Anchor indices passing the confidence filter, with score and class."""
    arr = _as_heads(output)
    cls = arr[4:]
    best_c = np.argmax(cls, axis=0)  # first maximum wins, as the reference's strict '>' scan
    best_s = cls[best_c, np.arange(cls.shape[1])].astype(np.float64)
    keep = np.nonzero(~(best_s < conf_thres))[0]
    return keep, best_s[keep], best_c[keep], arr


def _iou(a, b) -> float:
    x1 = a[0] if a[0] > b[0] else b[0]
    y1 = a[1] if a[1] > b[1] else b[1]
    x2 = a[2] if a[2] < b[2] else b[2]
    y2 = a[3] if a[3] < b[3] else b[3]
    w = x2 - x1
    h = y2 - y1
    if w <= 0 or h <= 0:
        return 0.0
    inter = w * h
    area_a = (a[2] - a[0]) * (a[3] - a[1])
    area_b = (b[2] - b[0]) * (b[3] - b[1])
    return inter / (area_a + area_b - inter + 1e-9)


def nms(boxes: List[tuple], iou_thres: float) -> List[int]:
    by_class: Dict[int, List[int]] = {}
    for i, b in enumerate(boxes):
        by_class.setdefault(b[5], []).append(i)
    keep_all: List[int] = []
    for _, idxs in by_class.items():
        idxs.sort(key=lambda i: boxes[i][4], reverse=True)
        while idxs:
            cur = idxs.pop(0)
            keep_all.append(cur)
            if not idxs:
                break
            cb = boxes[cur]
            idxs = [j for j in idxs if _iou(cb, boxes[j]) <= iou_thres]
    keep_all.sort(key=lambda i: boxes[i][4], reverse=True)
    return keep_all


def decode_yolo(output, meta=None, conf_thres: float = 0.25, iou_thres: float = 0.45,
                max_det: int = 300, with_anchor: bool = False) -> List[dict]:
    """[{'x1','y1','x2','y2','conf','cls'}, ...] for a [1, 4+nc, A] head.

    `meta` is anything with ratio/pad_x/pad_y/orig_w/orig_h attributes or keys.
    with_anchor=True adds the anchor index of each detection (for parity checks)."""
    idx, score, cls, arr = candidates(output, conf_thres)
    if idx.size == 0:
        return []
    cx = arr[0, idx].astype(np.float64)
    cy = arr[1, idx].astype(np.float64)
    w = arr[2, idx].astype(np.float64)
    h = arr[3, idx].astype(np.float64)
    x1, y1, x2, y2 = cx - w * 0.5, cy - h * 0.5, cx + w * 0.5, cy + h * 0.5
    if meta is not None:
        g = (lambda k: meta[k]) if isinstance(meta, dict) else (lambda k: getattr(meta, k))
        scale = 1.0 / g("ratio")
        px, py, ow, oh = g("pad_x"), g("pad_y"), g("orig_w"), g("orig_h")
        x1 = np.clip((x1 - px) * scale, 0.0, ow)
        y1 = np.clip((y1 - py) * scale, 0.0, oh)
        x2 = np.clip((x2 - px) * scale, 0.0, ow)
        y2 = np.clip((y2 - py) * scale, 0.0, oh)
    boxes = [(float(x1[i]), float(y1[i]), float(x2[i]), float(y2[i]), float(score[i]), int(cls[i]))
             for i in range(idx.size)]
    keep = nms(boxes, iou_thres)[:max_det]
    out = []
    for i in keep:
        d = {"x1": boxes[i][0], "y1": boxes[i][1], "x2": boxes[i][2], "y2": boxes[i][3],
             "conf": boxes[i][4], "cls": boxes[i][5]}
        if with_anchor:
            d["anchor"] = int(idx[i])
        out.append(d)
    return out
