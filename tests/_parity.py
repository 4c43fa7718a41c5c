"""Whole-network parity helpers shared by the GPU model tests (no torch).

Bars: raw head within max-rel 1e-3 (relative to max(1, |ref|), as the
reference's Near), detection index sets after NMS equal except where scores
tie within 1e-5, matched boxes IoU >= 0.999.
"""
import numpy as np

import oracle
from simdyolo_amd.detector import DetectorOptions, decode_detections


def max_rel(got, exp):
    return float((np.abs(got.astype(np.float64) - exp) / np.maximum(1.0, np.abs(exp))).max())


def _iou(a, b):
    w = max(0.0, min(a.x + a.width, b.x + b.width) - max(a.x, b.x))
    h = max(0.0, min(a.y + a.height, b.y + b.height) - max(a.y, b.y))
    i = w * h
    return i / max(1e-30, a.width * a.height + b.width * b.height - i)


def check_detections(head_gpu, head_ref, conf=0.25, size=640):
    o = DetectorOptions(confidence=conf, width=size, height=size)
    got = decode_detections(head_gpu, o)
    exp = oracle.nms_decode(head_ref, layout=0, confidence=conf,
                            transform=oracle.Letterbox(size, size, size, size, 1.0, 1.0, 0, 0))
    ga = {d.anchor: d for d in got}
    ea = {d.anchor: d for d in exp}
    # Anchors present on one side only must be explained by a near-tie
    # (threshold or suppression decided by scores within 1e-5).
    for a in set(ga) ^ set(ea):
        d = ga.get(a) or ea.get(a)
        near_threshold = abs(d.confidence - conf) <= 1e-4
        tied = any(abs(d.confidence - o2.confidence) <= 1e-5 for o2 in (got + exp) if o2.anchor != a)
        assert near_threshold or tied, f"anchor {a} conf {d.confidence} only on one side"
    for a in set(ga) & set(ea):
        assert ga[a].class_id == ea[a].class_id
        assert _iou(ga[a], ea[a]) >= 0.999
    return len(got), len(exp)


def adaptive_threshold(head, candidates=500):
    """A confidence threshold that admits about `candidates` anchors.  With
    random-init weights and the -4.6 class bias every score sits near
    sigmoid(-4.6) = 0.01, so the 0.25 default keeps no detection and index
    parity would be vacuous; this threshold makes NMS decide real cases."""
    best = head[4:].max(0)
    return float(np.sort(best)[-candidates])
