"""Pure-Python restatement of the reference's YOLO decode + NMS — TEST
INFRASTRUCTURE ONLY (the checker for pdefa_amd.postprocess).

Follows pdefa/python/src/pdefa/_bindings.py:1095-1212 line by line on nested
lists of Python floats: strict '>' class scan (first maximum wins),
`best_s < conf_thres` rejection, xywh -> xyxy, letterbox mapping with clamps,
per-class greedy NMS (stable descending sort, IoU with a 1e-9 guard, keep when
IoU <= thr), global stable sort by score, max_det cut.  Each detection also
carries the anchor index it came from.
"""
from collections import defaultdict


def decode(arr, meta=None, conf_thres=0.25, iou_thres=0.45, max_det=300, iou_log=None):
    """Detections of one [4 + classes, A] head (nested lists, batch dims of 1
    unwrapped), as the reference's decode_yolo returns them plus the anchor.
    iou_log: optional list that receives every IoU the NMS compares with
    iou_thres (for robustness margins of test fixtures)."""
    while isinstance(arr, list) and len(arr) == 1 and isinstance(arr[0], list) and len(arr[0]) > 4:
        arr = arr[0]
    n_classes = len(arr) - 4
    boxes = []
    for i in range(len(arr[0])):
        best_c, best_s = 0, arr[4][i]
        for c in range(1, n_classes):
            s = arr[4 + c][i]
            if s > best_s:
                best_s, best_c = s, c
        if best_s < conf_thres:
            continue
        cx, cy, w, h = arr[0][i], arr[1][i], arr[2][i], arr[3][i]
        boxes.append((cx - w * 0.5, cy - h * 0.5, cx + w * 0.5, cy + h * 0.5, best_s, best_c, i))
    if not boxes:
        return []
    if meta is not None:
        scale = 1.0 / meta["ratio"]
        px, py, ow, oh = meta["pad_x"], meta["pad_y"], meta["orig_w"], meta["orig_h"]
        moved = []
        for b in boxes:
            x1 = (b[0] - px) * scale
            y1 = (b[1] - py) * scale
            x2 = (b[2] - px) * scale
            y2 = (b[3] - py) * scale
            x1 = 0.0 if x1 < 0 else (ow if x1 > ow else x1)
            y1 = 0.0 if y1 < 0 else (oh if y1 > oh else y1)
            x2 = 0.0 if x2 < 0 else (ow if x2 > ow else x2)
            y2 = 0.0 if y2 < 0 else (oh if y2 > oh else y2)
            moved.append((x1, y1, x2, y2, b[4], b[5], b[6]))
        boxes = moved

    def iou(a, b):
        x1 = a[0] if a[0] > b[0] else b[0]
        y1 = a[1] if a[1] > b[1] else b[1]
        x2 = a[2] if a[2] < b[2] else b[2]
        y2 = a[3] if a[3] < b[3] else b[3]
        w, h = x2 - x1, y2 - y1
        if w <= 0 or h <= 0:
            return 0.0
        inter = w * h
        return inter / ((a[2] - a[0]) * (a[3] - a[1]) + (b[2] - b[0]) * (b[3] - b[1]) - inter + 1e-9)

    by_class = defaultdict(list)
    for i, b in enumerate(boxes):
        by_class[b[5]].append(i)
    keep = []
    for _, idxs in by_class.items():
        idxs.sort(key=lambda i: boxes[i][4], reverse=True)
        while idxs:
            cur = idxs.pop(0)
            keep.append(cur)
            if not idxs:
                break
            ious = [iou(boxes[cur], boxes[j]) for j in idxs]
            if iou_log is not None:
                iou_log.extend(ious)
            idxs = [j for j, v in zip(idxs, ious) if v <= iou_thres]
    keep.sort(key=lambda i: boxes[i][4], reverse=True)
    keep = keep[:max_det]
    return [{"x1": boxes[i][0], "y1": boxes[i][1], "x2": boxes[i][2], "y2": boxes[i][3],
             "conf": boxes[i][4], "cls": boxes[i][5], "anchor": boxes[i][6]} for i in keep]


def robust_conf(arr, start=0.25, min_gap=1e-2, min_candidates=5, step=0.0025, stop=0.9):
    """The smallest conf_thres >= start on a `step` grid such that no anchor's
    best class score lies within min_gap of it and at least min_candidates
    anchors score above it (a threshold at which outputs within the parity
    tolerance select the same candidates), with that gap; (None, None) when
    there is none.  arr: [4 + classes, A] (numpy or nested lists)."""
    import numpy as np
    a = np.asarray(arr, np.float64)
    while a.ndim > 2:
        a = a[0]
    best = np.sort(a[4:].max(axis=0))
    for i in range(int(round((stop - start) / step)) + 1):
        t = round(start + i * step, 6)
        gap = float(np.abs(best - t).min())
        if gap >= min_gap and int((best > t).sum()) >= min_candidates:
            return t, gap
    return None, None


def min_iou_gap(arr, meta=None, conf_thres=0.25, iou_thres=0.45):
    """The smallest |IoU - iou_thres| over the comparisons the NMS makes
    (inf when it makes none)."""
    log = []
    decode(arr, meta, conf_thres, iou_thres, max_det=1 << 30, iou_log=log)
    return min((abs(v - iou_thres) for v in log), default=float("inf"))
