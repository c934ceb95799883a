"""Hand-worked known answers for YOLO decode + per-class NMS.

Each case is a small head (rows cx, cy, w, h, then one score row per class,
one column per anchor), the decode arguments, and the detection list worked
out by hand from the reference's rules (pdefa/python/src/pdefa/_bindings.py:
1095-1212):

- the best class of an anchor is the first maximum (strict '>' scan, 1123-1128);
- an anchor is dropped when its best score is < conf_thres (1129), so a
  score equal to the threshold is kept;
- xywh -> xyxy (1132-1135), then the letterbox mapping (x - pad) / ratio,
  clamped to [0, orig] (1141-1156);
- per class, boxes in descending score order (stable) and a box survives
  while IoU = inter / (area_a + area_b - inter + 1e-9) <= iou_thres with the
  kept box (1175-1212); touching boxes have IoU 0;
- survivors of all classes, visited class by class in order of each class's
  first anchor, sorted by score (stable), cut to max_det (1160-1163, 1211).

Coordinates are chosen so that every value is exact in float32 and float64
(the IoU cases use areas of 2^29 and 2^30, where the 1e-9 guard vanishes in
rounding, so the IoU is exactly 0.5 or 0.5 + 2^-15).
"""
from __future__ import annotations

import numpy as np


def head(boxes, nc):
    """boxes: [(cx, cy, w, h, {cls: score, ...}), ...] -> float32 [4 + nc, A]."""
    h = np.zeros((4 + nc, len(boxes)), np.float32)
    for a, (cx, cy, w, hh, scores) in enumerate(boxes):
        h[0, a], h[1, a], h[2, a], h[3, a] = cx, cy, w, hh
        for c, s in scores.items():
            h[4 + c, a] = s
    return h


def det(x1, y1, x2, y2, conf, cls, anchor):
    return {"x1": float(x1), "y1": float(y1), "x2": float(x2), "y2": float(y2), "conf": float(np.float32(conf)),
            "cls": cls, "anchor": anchor}


# name -> (boxes, nc, kwargs for decode, expected detections)
CASES = {
    # IoU exactly at the threshold is kept, just above it is suppressed.
    # a = [0,0,32768,32768] (area 2^30); b = [0,0,32768,16384] inside a,
    # IoU = 2^29 / 2^30 = 0.5; c = [0,0,32768,16385], IoU = 0.5 + 2^-15.
    "iou_at_threshold": (
        [(16384, 16384, 32768, 32768, {1: 0.9}),
         (16384, 8192, 32768, 16384, {1: 0.8}),
         (16384, 8192.5, 32768, 16385, {1: 0.7})],
        3, dict(conf_thres=0.25, iou_thres=0.5, max_det=300),
        [det(0, 0, 32768, 32768, 0.9, 1, 0), det(0, 0, 32768, 16384, 0.8, 1, 1)]),
    # b survives a, and is then the kept box against which nothing remains;
    # with the threshold lowered below 0.5 it is suppressed too
    "iou_below_threshold_suppresses": (
        [(16384, 16384, 32768, 32768, {1: 0.9}),
         (16384, 8192, 32768, 16384, {1: 0.8})],
        3, dict(conf_thres=0.25, iou_thres=0.4999, max_det=300),
        [det(0, 0, 32768, 32768, 0.9, 1, 0)]),
    # equal scores in two classes: the class whose first anchor comes first
    # (class 5 at anchor 0) leads, although its tied box is at anchor 2
    "tie_across_classes": (
        [(10, 10, 10, 10, {5: 0.9}),
         (100, 100, 10, 10, {2: 0.625}),
         (200, 200, 10, 10, {5: 0.625})],
        8, dict(conf_thres=0.25, iou_thres=0.45, max_det=300),
        [det(5, 5, 15, 15, 0.9, 5, 0), det(195, 195, 205, 205, 0.625, 5, 2),
         det(95, 95, 105, 105, 0.625, 2, 1)]),
    # a best score equal to conf_thres is kept; one just below it is dropped
    "score_at_threshold": (
        [(50, 50, 20, 20, {0: 0.25}),
         (150, 150, 20, 20, {0: np.nextafter(np.float32(0.25), np.float32(0))})],
        2, dict(conf_thres=0.25, iou_thres=0.45, max_det=300),
        [det(40, 40, 60, 60, 0.25, 0, 0)]),
    # two classes tied within one anchor: the first (lower) class wins
    "tie_within_anchor": (
        [(50, 50, 20, 20, {3: 0.75, 7: 0.75})],
        9, dict(conf_thres=0.25, iou_thres=0.45, max_det=300),
        [det(40, 40, 60, 60, 0.75, 3, 0)]),
    # letterbox mapping (ratio 0.5, pad_y 140, 1280x720 source) with clamps:
    # [-10,130,30,170] -> [-20,-20,60,60] -> [0,0,60,60];
    # [610,500,650,540] -> [1220,720,1300,800] -> [1220,720,1280,720]
    "letterbox_clamp": (
        [(10, 150, 40, 40, {4: 0.5}),
         (630, 520, 40, 40, {4: 0.75})],
        6, dict(conf_thres=0.25, iou_thres=0.45, max_det=300,
                meta={"ratio": 0.5, "pad_x": 0, "pad_y": 140, "orig_w": 1280, "orig_h": 720}),
        [det(1220, 720, 1280, 720, 0.75, 4, 1), det(0, 0, 60, 60, 0.5, 4, 0)]),
    # max_det keeps the best ones after the global sort
    "max_det_cut": (
        [(20 + 40 * i, 20, 10, 10, {i % 2: s}) for i, s in enumerate([0.5, 0.875, 0.625, 0.75, 0.9375])],
        2, dict(conf_thres=0.25, iou_thres=0.45, max_det=3),
        [det(175, 15, 185, 25, 0.9375, 0, 4), det(55, 15, 65, 25, 0.875, 1, 1),
         det(135, 15, 145, 25, 0.75, 1, 3)]),
    # boxes sharing an edge have IoU 0 and both survive even at iou_thres 0
    "touching_boxes": (
        [(5, 5, 10, 10, {0: 0.5}),
         (15, 5, 10, 10, {0: 0.75})],
        1, dict(conf_thres=0.25, iou_thres=0.0, max_det=300),
        [det(10, 0, 20, 10, 0.75, 0, 1), det(0, 0, 10, 10, 0.5, 0, 0)]),
    # the 1e-9 guard on tiny boxes: two identical boxes of side 2^-13
    # (area 2^-26 ~ 1.49e-8) have IoU 2^-26 / (2^-26 + 1e-9) ~ 0.937 > 0.5
    "guard_on_tiny_boxes": (
        [(2.0 ** -14, 2.0 ** -14, 2.0 ** -13, 2.0 ** -13, {0: 0.75}),
         (2.0 ** -14, 2.0 ** -14, 2.0 ** -13, 2.0 ** -13, {0: 0.5})],
        1, dict(conf_thres=0.25, iou_thres=0.5, max_det=300),
        [det(0, 0, 2.0 ** -13, 2.0 ** -13, 0.75, 0, 0)]),
    # a suppressed box does not suppress others: b overlaps a (IoU 1/3 > 0.3,
    # suppressed), c overlaps b but only touches a, so c stays
    "suppressed_box_does_not_suppress": (
        [(10, 10, 20, 20, {0: 0.9}),
         (20, 10, 20, 20, {0: 0.8}),
         (30, 10, 20, 20, {0: 0.7})],
        1, dict(conf_thres=0.25, iou_thres=0.3, max_det=300),
        [det(0, 0, 20, 20, 0.9, 0, 0), det(20, 0, 40, 20, 0.7, 0, 2)]),
}
