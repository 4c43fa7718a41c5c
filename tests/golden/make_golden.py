"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture pins one seeded network (synthetic random-init weights and
uniform u8 images, simdyolo_amd.synth) at 640x640, batch 1: the head tensor's
shape, sums, per-channel sums, 512 sampled values, and the NMS detection
lists at the default 0.25 threshold and at a threshold that admits about 500
candidates.  The oracle is deterministic (each output element is one serial
double-precision sum), so the fixtures pin it against drift and give the GPU
tests a committed target.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from simdyolo_amd import synth  # noqa: E402

CASES = {
    "yolov8n_640_b1": ("yolov8", "n"),
    "yolo11n_640_b1": ("yolo11", "n"),
}
SIZE = 640
N_SAMPLES = 512


def forward(arch, scale, params, x):
    if arch == "yolo11":
        d, w, mc = synth.SCALES_11[scale]
        return oracle.yolo11_forward(params, x, depth=d, width=w, max_channels=mc)
    d, w, mc = synth.SCALES[scale]
    return oracle.yolov8_forward(params, x, depth=d, width=w, max_channels=mc)


def detections(head, conf):
    lb = oracle.Letterbox(SIZE, SIZE, SIZE, SIZE, 1.0, 1.0, 0, 0)
    return [[d.anchor, d.class_id, float(d.confidence), float(d.x), float(d.y), float(d.width), float(d.height)]
            for d in oracle.nms_decode(head, layout=0, confidence=conf, transform=lb)]


def adaptive_threshold(head, candidates=500):
    return float(np.sort(head[4:].max(0))[-candidates])


def make(name, arch, scale):
    cfg = synth.config(scale, arch=arch)
    params = synth.params(cfg)
    x = synth.images(1, SIZE, SIZE)
    head = forward(arch, scale, params, x)
    flat = head.reshape(-1)
    rng = np.random.Generator(np.random.PCG64(7))
    idx = np.sort(rng.choice(flat.size, N_SAMPLES, replace=False))
    thr = adaptive_threshold(head[0])
    return {
        "network": f"{arch}{scale}", "size": SIZE, "batch": 1,
        "weights_seed": synth.SEED, "image_seed": synth.SEED + 1,
        "shape": list(head.shape),
        "sum": float(head.astype(np.float64).sum()),
        "abs_sum": float(np.abs(head.astype(np.float64)).sum()),
        "channel_sums": head[0].astype(np.float64).sum(1).tolist(),
        "sample_index": idx.tolist(),
        "sample_value": flat[idx].astype(float).tolist(),
        "detections_default": detections(head[0], 0.25),
        "adaptive_threshold": thr,
        "detections_adaptive": detections(head[0], thr),
    }


def main():
    for name, (arch, scale) in CASES.items():
        data = make(name, arch, scale)
        path = os.path.join(HERE, f"{name}.json")
        with open(path, "w") as f:
            json.dump(data, f, indent=0)
        print(f"{path}: {len(data['detections_adaptive'])} detections at {data['adaptive_threshold']:.6f}")


if __name__ == "__main__":
    main()
