"""YoloDetector / DetectorOptions over the HIP backend, shaped like the
reference's public API (src/SimdYolo/YoloDetector.cs:73-126 options,
:211-241 construction, :262-265 PredictRaw, :327-378 Predict).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native as N
from .device import HipContext


@dataclass
class DetectorOptions:
    device: int = 0
    width: int = 640
    height: int = 640
    confidence: float = 0.25
    iou_threshold: float = 0.45
    max_detections: int = 300
    max_candidates: int = 30000
    class_agnostic_nms: bool = False
    class_count: int = 0
    output_layout: int = N.LAYOUT_NHWC  # 0 = auto (OutputLayout.Auto)


@dataclass
class Detection:
    class_id: int
    confidence: float
    x: float
    y: float
    width: float
    height: float
    anchor: int


class YoloDetector:
    """A YOLOv8 / YOLO11 detector whose forward runs on MI355X."""

    def __init__(self, cfg: N.ModelConfig, params: np.ndarray, options: DetectorOptions | None = None,
                 ctx: HipContext | None = None):
        self.options = options or DetectorOptions()
        self.cfg = cfg
        self._own_ctx = ctx is None
        self.ctx = ctx or HipContext(self.options.device)
        lib = N.lib()
        p = np.ascontiguousarray(params, dtype=np.float32)
        h = ctypes.c_void_p()
        N.check(lib.sy_model_create(self.ctx.handle, ctypes.byref(cfg), N.fptr(p), p.size, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            N.lib().sy_model_destroy(self.handle)
            self.handle = None
        if self._own_ctx and self.ctx:
            self.ctx.close()
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def output_shape(self, batch: int, h: int, w: int):
        ch, an = ctypes.c_int(), ctypes.c_int()
        N.check(N.lib().sy_model_output_shape(self.handle, batch, h, w, ctypes.byref(ch), ctypes.byref(an)))
        return batch, ch.value, an.value

    def predict_raw(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 4 or x.shape[1] != 3:
            raise ValueError("PT YOLO expects NCHW RGB input")
        b, _, h, w = x.shape
        out = np.empty(self.output_shape(b, h, w), np.float32)
        N.check(N.lib().sy_model_predict_raw(self.handle, N.fptr(x), b, h, w, N.fptr(out)))
        return out

    def predict_seg(self, x: np.ndarray):
        """Segment model: (head [B, nc+4+nm, anchors], or for end-to-end models
        the selected rows [B, k, 6+nm]; protos [B, nm, H/4, W/4])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 4 or x.shape[1] != 3:
            raise ValueError("PT YOLO expects NCHW RGB input")
        b, _, h, w = x.shape
        out = np.empty(self.output_shape(b, h, w), np.float32)
        nm = self.cfg.nm
        protos = np.empty((b, nm, h // 4, w // 4), np.float32)
        N.check(N.lib().sy_model_predict_seg(self.handle, N.fptr(x), b, h, w, N.fptr(out), N.fptr(protos)))
        return out, protos

    def proto_buffer(self, batch: int, h: int, w: int):
        """Device address and shape (nm, H/4, W/4) of the planned Proto output."""
        p, c, ph, pw = ctypes.c_void_p(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        N.check(N.lib().sy_model_proto(self.handle, batch, h, w, ctypes.byref(p), ctypes.byref(c), ctypes.byref(ph),
                                       ctypes.byref(pw)))
        return p.value, (c.value, ph.value, pw.value)

    def head_buffer(self, batch: int, h: int, w: int):
        """Device address and (channels, anchors) of the joined, decoded head
        (for end-to-end models the head before the top-k selection)."""
        p, c, a = ctypes.c_void_p(), ctypes.c_int(), ctypes.c_int()
        N.check(N.lib().sy_model_head(self.handle, batch, h, w, ctypes.byref(p), ctypes.byref(c), ctypes.byref(a)))
        return p.value, (c.value, a.value)

    def set_graph(self, enabled: bool):
        N.check(N.lib().sy_model_set_graph(self.handle, int(enabled)))

    def set_branch_level(self, level: int):
        """-1: the captured forward's branch level is chosen by timing; 0..2 forces it."""
        N.check(N.lib().sy_model_set_branch_level(self.handle, level))

    def branch_level(self, batch: int, h: int, w: int) -> int:
        lv = ctypes.c_int()
        N.check(N.lib().sy_model_branch_level(self.handle, batch, h, w, ctypes.byref(lv)))
        return lv.value

    def buffers(self, batch: int, h: int, w: int):
        inp, out = ctypes.c_void_p(), ctypes.c_void_p()
        N.check(N.lib().sy_model_buffers(self.handle, batch, h, w, ctypes.byref(inp), ctypes.byref(out)))
        return inp.value, out.value

    def run(self, batch: int, h: int, w: int):
        N.check(N.lib().sy_model_run(self.handle, batch, h, w))

    def memory(self):
        wb, ab = ctypes.c_size_t(), ctypes.c_size_t()
        N.check(N.lib().sy_model_memory(self.handle, ctypes.byref(wb), ctypes.byref(ab)))
        return wb.value, ab.value

    def plan_memory(self, batch: int, h: int, w: int):
        """(arena bytes shared by liveness, unshared bytes, scratch bytes) of one input shape."""
        a, u, sc = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        N.check(N.lib().sy_model_plan_memory(self.handle, batch, h, w, ctypes.byref(a), ctypes.byref(u),
                                             ctypes.byref(sc)))
        return a.value, u.value, sc.value

    def predict(self, pixels: np.ndarray, width: int, height: int, bgr: bool = False):
        """pixels: HxWx3 uint8 (RGB unless bgr).  Letterbox -> forward -> NMS."""
        o = self.options
        inp = np.empty((1, 3, o.height, o.width), np.float32)
        t = N.LetterboxT()
        px = np.ascontiguousarray(pixels, dtype=np.uint8)
        N.check(N.lib().sy_letterbox_rgb(px.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), width, height, o.width,
                                         o.height, int(bgr), 0, N.fptr(inp), ctypes.byref(t)))
        head = self.predict_raw(inp)[0]
        return decode_detections(head, o, t)


def decode_detections(head: np.ndarray, o: DetectorOptions, t: N.LetterboxT | None = None):
    """DetectionDecoder.DecodeIndexed on one image's [dim1, dim2] head."""
    head = np.ascontiguousarray(head, dtype=np.float32)
    d1, d2 = head.shape
    if t is None:
        t = N.LetterboxT(o.width, o.height, o.width, o.height, 1.0, 1.0, 0, 0)
    opts = N.DecodeOptions(o.confidence, o.iou_threshold, o.max_detections, o.max_candidates, o.class_count,
                           int(o.class_agnostic_nms), o.output_layout)
    cap = o.max_detections
    out = (N.DetectionT * cap)()
    count = ctypes.c_int()
    N.check(N.lib().sy_decode_detections(N.fptr(head), d1, d2, ctypes.byref(opts), ctypes.byref(t), out, cap,
                                         ctypes.byref(count)))
    return [Detection(d.class_id, d.confidence, d.x, d.y, d.width, d.height, d.anchor)
            for d in out[:count.value]]
