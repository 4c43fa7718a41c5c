"""Seeded synthetic model parameters and images for the YOLOv8 and YOLO11 families.

The reference loads trained .pt/.onnx weights; none can be fetched here, so
every benchmark and test uses random-init weights of the real architecture,
generated from a seed by this scheme:

* conv weights: Kaiming-normal, std = sqrt(2 / fan_in);
* BatchNorm: gamma ~ U[0.5, 1.5], beta ~ N(0, 0.1), running mean 0, var 1
  (eps 1e-3, ultralytics' default), folded at load as the reference does;
* Detect's final Conv2d biases: box 1.0 (ultralytics' init), class -4.6;
  other biases (Segment's mask-coefficient Conv2d, Proto's ConvTranspose2d)
  N(0, 0.1);
* images: uint8 pixels uniform in [0, 255], divided by 255 (the letterbox is
  the identity at the network size), NCHW.

Parameters are laid out in the canonical state_dict order reported by the
library (sy_model_layout).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N

SEED = 20261013  # the reference's validation RNG seed (tools/validate-reference.py:39)

# (depth, width, max_channels) per scale: ultralytics yolov8.yaml / yolo11.yaml.
SCALES = {
    "n": (0.33, 0.25, 1024),
    "s": (0.33, 0.50, 1024),
    "m": (0.67, 0.75, 768),
    "l": (1.00, 1.00, 512),
    "x": (1.00, 1.25, 512),
}
SCALES_11 = {
    "n": (0.50, 0.25, 1024),
    "s": (0.50, 0.50, 1024),
    "m": (0.50, 1.00, 512),
    "l": (1.00, 1.00, 512),
    "x": (1.00, 1.50, 512),
}
ARCHS = {"yolov8": N.ARCH_YOLOV8, "yolo11": N.ARCH_YOLO11, "yolo26": N.ARCH_YOLO26}


def config(scale: str = "n", nc: int = 80, reg_max: int | None = None, bn_eps: float = 1e-3,
           arch: str = "yolov8", nm: int = 0, npr: int = 256) -> N.ModelConfig:
    """nm > 0 selects the Segment head (nm mask coefficients, npr Proto channels).
    YOLO26 shares YOLO11's scales and defaults to its single-bin head (reg_max 1)."""
    depth, width, max_ch = (SCALES if arch == "yolov8" else SCALES_11)[scale]
    if reg_max is None:
        reg_max = 1 if arch == "yolo26" else 16
    return N.ModelConfig(ARCHS[arch], depth, width, max_ch, nc, reg_max, bn_eps, nm, npr)


def layout(cfg: N.ModelConfig) -> np.ndarray:
    lib = N.lib()
    count = ctypes.c_int()
    N.check(lib.sy_model_layout(ctypes.byref(cfg), None, 0, ctypes.byref(count)))
    buf = (ctypes.c_int32 * (6 * count.value))()
    N.check(lib.sy_model_layout(ctypes.byref(cfg), buf, count.value, ctypes.byref(count)))
    return np.frombuffer(buf, dtype=np.int32).reshape(count.value, 6).copy()


def params_for_layout(entries: np.ndarray, seed: int = SEED, box_bias: float = 1.0,
                      cls_bias: float = -4.6) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    chunks = []
    for kind, d0, d1, d2, d3, fan_in in entries:
        n = int(d0) * int(d1) * int(d2) * int(d3)
        if kind == 0:  # SY_P_CONV_WEIGHT
            v = rng.standard_normal(n) * np.sqrt(2.0 / fan_in)
        elif kind == 1:  # gamma
            v = rng.uniform(0.5, 1.5, n)
        elif kind == 2:  # beta
            v = rng.standard_normal(n) * 0.1
        elif kind == 3:  # running mean
            v = np.zeros(n)
        elif kind == 4:  # running var
            v = np.ones(n)
        elif kind == 5:
            v = np.full(n, box_bias)
        elif kind == 6:
            v = np.full(n, cls_bias)
        elif kind == 7:  # other biases (mask-coefficient Conv2d, Proto's ConvTranspose2d)
            v = rng.standard_normal(n) * 0.1
        else:
            raise ValueError(f"unknown parameter kind {kind}")
        chunks.append(v.astype(np.float32))
    return np.concatenate(chunks)


def params(cfg: N.ModelConfig, seed: int = SEED) -> np.ndarray:
    return params_for_layout(layout(cfg), seed)


def image_u8(batch: int, h: int, w: int, seed: int = SEED + 1) -> np.ndarray:
    """uint8 pixels, [batch, 3, h, w]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, 256, size=(batch, 3, h, w), dtype=np.uint8)


def images(batch: int, h: int, w: int, seed: int = SEED + 1) -> np.ndarray:
    """Network input: u8 / 255 as float32 NCHW."""
    return image_u8(batch, h, w, seed).astype(np.float32) / np.float32(255.0)


def activations(shape, seed: int) -> np.ndarray:
    """N(0, 1) activations for per-layer tests."""
    return np.random.Generator(np.random.PCG64(seed)).standard_normal(shape).astype(np.float32)


def kaiming(shape, seed: int) -> np.ndarray:
    fan_in = int(np.prod(shape[1:]))
    return (np.random.Generator(np.random.PCG64(seed)).standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(
        np.float32)
