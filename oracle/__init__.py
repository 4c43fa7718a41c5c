"""ctypes front end of the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
as the checker, and by bench.py's ``cpu_baseline`` leg.  The shipped package
(``simdyolo_amd``) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)


def build() -> None:
    """Compile oracle.c and cpu_fast.c with the committed Makefile (always
    recompiled: this is also the does-it-build check)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


class Letterbox(ctypes.Structure):
    _fields_ = [("source_width", ctypes.c_int), ("source_height", ctypes.c_int),
                ("target_width", ctypes.c_int), ("target_height", ctypes.c_int),
                ("scale_x", ctypes.c_float), ("scale_y", ctypes.c_float),
                ("pad_x", ctypes.c_int), ("pad_y", ctypes.c_int)]


class Detection(ctypes.Structure):
    _fields_ = [("class_id", ctypes.c_int), ("confidence", ctypes.c_float),
                ("x", ctypes.c_float), ("y", ctypes.c_float),
                ("width", ctypes.c_float), ("height", ctypes.c_float),
                ("anchor", ctypes.c_int)]


class YoloCfg(ctypes.Structure):
    _fields_ = [("depth", ctypes.c_float), ("width", ctypes.c_float),
                ("max_channels", ctypes.c_int), ("nc", ctypes.c_int),
                ("reg_max", ctypes.c_int), ("bn_eps", ctypes.c_float),
                ("nm", ctypes.c_int), ("npr", ctypes.c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def fold_bn(w, conv_bias, gamma, beta, mean, var, eps):
    w = _f32(w)
    oc = w.shape[0]
    per = w.size // oc
    wo = np.empty_like(w)
    bo = np.empty(oc, np.float32)
    cb = _f32(conv_bias) if conv_bias is not None else None
    g, b, m, v = (_f32(t) for t in (gamma, beta, mean, var))
    lib().or_fold_bn(_p(w), oc, per, _p(cb) if cb is not None else None, _p(g), _p(b), _p(m), _p(v),
                     ctypes.c_float(eps), _p(wo), _p(bo))
    return wo, bo


def conv2d(x, w, bias=None, stride=(1, 1), pads=(0, 0, 0, 0), dilation=(1, 1), groups=1, silu=False):
    """NCHW conv; pads are (top, left, bottom, right) like the reference."""
    x, w = _f32(x), _f32(w)
    n, c, h, wd = x.shape
    oc, _, kh, kw = w.shape
    b = _f32(bias) if bias is not None else None
    oh, ow = ctypes.c_int(), ctypes.c_int()
    args = (n, c, h, wd, _p(w), _p(b) if b is not None else None, oc, kh, kw, stride[0], stride[1],
            pads[0], pads[1], pads[2], pads[3], dilation[0], dilation[1], groups, int(silu))
    rc = lib().or_conv2d(_p(x), *args, None, ctypes.byref(oh), ctypes.byref(ow))
    if rc:
        raise ValueError("invalid convolution")
    y = np.empty((n, oc, oh.value, ow.value), np.float32)
    lib().or_conv2d(_p(x), *args, _p(y), None, None)
    return y


def maxpool(x, kernel, stride, pads, ceil_mode=False):
    x = _f32(x)
    n, c, h, w = x.shape
    oh, ow = ctypes.c_int(), ctypes.c_int()
    args = (n, c, h, w, kernel[0], kernel[1], stride[0], stride[1], pads[0], pads[1], pads[2], pads[3],
            int(ceil_mode))
    if lib().or_maxpool(_p(x), *args, None, ctypes.byref(oh), ctypes.byref(ow)):
        raise ValueError("invalid pooling")
    y = np.empty((n, c, oh.value, ow.value), np.float32)
    lib().or_maxpool(_p(x), *args, _p(y), None, None)
    return y


def resize_nearest(x, oh, ow):
    x = _f32(x)
    n, c, h, w = x.shape
    y = np.empty((n, c, oh, ow), np.float32)
    lib().or_resize_nearest(_p(x), n, c, h, w, oh, ow, _p(y))
    return y


def detect_decode(levels, bins, xyxy=False):
    """levels: list of (boxes[B,4*bins,h,w], scores[B,nc,h,w], stride)."""
    batch, nc = levels[0][1].shape[:2]
    total = sum(b.shape[2] * b.shape[3] for b, _, _ in levels)
    out = np.empty((batch, nc + 4, total), np.float32)
    start = 0
    for boxes, scores, stride in levels:
        boxes, scores = _f32(boxes), _f32(scores)
        h, w = boxes.shape[2:]
        lib().or_detect_decode(_p(boxes), _p(scores), batch, nc, h, w, bins, ctypes.c_float(stride),
                               int(xyxy), _p(out), total, start)
        start += h * w
    return out


def e2e_select(x, maximum, classes, onnx=False):
    x = _f32(x)
    batch, channels, anchors = x.shape
    k = min(maximum, anchors)
    out = np.empty((batch, k, 6 + channels - classes - 4), np.float32)
    fn = lib().or_e2e_select_onnx if onnx else lib().or_e2e_select_pt
    if fn(_p(x), batch, channels, anchors, classes, maximum, _p(out)):
        raise ValueError("invalid top-k arguments")
    return out


def nms_decode(head, layout=0, class_count=0, confidence=0.25, iou=0.45, max_detections=300,
               max_candidates=30000, agnostic=False, transform=None):
    """head: [d1, d2] of a single image (batch dimension removed)."""
    head = _f32(head)
    d1, d2 = head.shape
    if transform is None:
        transform = Letterbox(d2 if layout != 1 else 640, 640, 640, 640, 1.0, 1.0, 0, 0)
    out = (Detection * max(1, max_detections))()
    count = ctypes.c_int()
    rc = lib().or_nms_decode(_p(head), d1, d2, layout, class_count, ctypes.c_float(confidence),
                             ctypes.c_float(iou), max_detections, max_candidates, int(agnostic),
                             ctypes.byref(transform), out, ctypes.byref(count))
    if rc:
        raise ValueError(f"nms decode failed ({rc})")
    return [out[i] for i in range(count.value)]


def mask_decode(proto, coeffs, box, transform):
    """proto [nm, mh, mw]; box (x, y, w, h) in source pixels.
    Returns (probabilities [height, width], (left, top, width, height))."""
    proto, coeffs = _f32(proto), _f32(coeffs)
    nm, mh, mw = proto.shape
    det = Detection(0, 1.0, *[float(v) for v in box], 0)
    info = (ctypes.c_int * 4)()
    lib().or_mask_decode(_p(proto), nm, mh, mw, _p(coeffs), ctypes.byref(det), ctypes.byref(transform), None, info)
    out = np.empty((max(info[3], 0), max(info[2], 0)), np.float32)
    if lib().or_mask_decode(_p(proto), nm, mh, mw, _p(coeffs), ctypes.byref(det), ctypes.byref(transform), _p(out),
                            info):
        raise ValueError("invalid mask box")
    return out, tuple(info)


def letterbox(pixels: np.ndarray, width, height, tw, th, bgr=False, row_stride=0):
    pixels = np.ascontiguousarray(pixels, dtype=np.uint8)
    out = np.empty((1, 3, th, tw), np.float32)
    t = Letterbox()
    rc = lib().or_letterbox(pixels.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), width, height, tw, th,
                            int(bgr), row_stride, _p(out), ctypes.byref(t))
    if rc:
        raise ValueError("invalid letterbox")
    return out, t


def _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm=0, npr=256):
    return YoloCfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr)


def conv_transpose2x2(x, w, bias):
    """nn.ConvTranspose2d(ic, oc, 2, 2): x [n, ic, h, w], w [ic, oc, 2, 2]."""
    x, w, b = _f32(x), _f32(w), _f32(bias)
    n, ic, h, wd = x.shape
    oc = w.shape[1]
    y = np.empty((n, oc, 2 * h, 2 * wd), np.float32)
    lib().or_conv_transpose2x2(_p(x), n, ic, h, wd, _p(w), _p(b), oc, _p(y))
    return y


def _layout(fn, cfg):
    n = fn(ctypes.byref(cfg), None, 0)
    buf = (ctypes.c_int * (6 * n))()
    fn(ctypes.byref(cfg), buf, n)
    return np.frombuffer(buf, dtype=np.int32).reshape(n, 6).copy()


def _forward(fn, cfg, params, x, nm):
    params, x = _f32(params), _f32(x)
    batch, _, h, w = x.shape
    anchors = (h // 8) * (w // 8) + (h // 16) * (w // 16) + (h // 32) * (w // 32)
    out = np.empty((batch, cfg.nc + 4 + nm, anchors), np.float32)
    proto = np.empty((batch, nm, h // 4, w // 4), np.float32) if nm else None
    rc = fn(ctypes.byref(cfg), _p(params), ctypes.c_size_t(params.size), _p(x), batch, h, w, _p(out),
            ctypes.c_size_t(out.size), _p(proto) if nm else None)
    if rc:
        raise ValueError(f"oracle forward failed ({rc})")
    return (out, proto) if nm else out


def yolov8_layout(depth=0.33, width=0.25, max_channels=1024, nc=80, reg_max=16, bn_eps=1e-3, nm=0, npr=256):
    return _layout(lib().or_yolov8_layout, _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr))


def yolov8_forward(params, x, depth=0.33, width=0.25, max_channels=1024, nc=80, reg_max=16, bn_eps=1e-3, nm=0,
                   npr=256):
    """Head [B, nc+4, A]; with nm > 0 (Segment head) (head [B, nc+4+nm, A], protos [B, nm, H/4, W/4])."""
    return _forward(lib().or_yolov8_forward, _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr),
                    params, x, nm)


CF_IMPLICIT, CF_WINOGRAD4, CF_WINOGRAD2, CF_DEPTHWISE = range(4)


def _cf_lib():
    L = lib()
    L.cf_conv_create.restype = ctypes.c_void_p
    L.cf_conv_create.argtypes = [_f32p, _f32p] + [ctypes.c_int] * 6
    L.cf_conv_run.argtypes = [ctypes.c_void_p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _i32p, _i32p]
    L.cf_conv_algorithm.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    L.cf_conv_destroy.argtypes = [ctypes.c_void_p]
    return L


def cpu_fast_conv(x, w, bias=None, stride=1, groups=1, silu=False):
    """(y, algorithm) of one convolution (padding k // 2) on the CPU-baseline
    restatement (oracle/cpu_fast.c)."""
    L = _cf_lib()
    x, w = _f32(x), _f32(w)
    n, ic, h, wd = x.shape
    oc, _, k, _ = w.shape
    b = _f32(bias) if bias is not None else None
    c = L.cf_conv_create(_p(w), _p(b) if b is not None else None, oc, ic, k, stride, groups, int(silu))
    try:
        oh, ow = ctypes.c_int(), ctypes.c_int()
        L.cf_conv_run(c, _p(x), n, h, wd, None, ctypes.byref(oh), ctypes.byref(ow))
        y = np.empty((n, oc, oh.value, ow.value), np.float32)
        L.cf_conv_run(c, _p(x), n, h, wd, _p(y), None, None)
        return y, L.cf_conv_algorithm(c, h, wd)
    finally:
        L.cf_conv_destroy(c)


class FastYolov8:
    """CPU baseline: the YOLOv8 detect forward with its convolutions on the
    restatement of the reference's FP32 CPU algorithms (oracle/cpu_fast.c),
    weights loaded and planned once.  Timed by bench.py's cpu_baseline leg;
    tests/test_cpu_fast.py checks it against yolov8_forward."""

    def __init__(self, params, depth=0.33, width=0.25, max_channels=1024, nc=80, reg_max=16, bn_eps=1e-3):
        L = lib()
        L.or_fast_yolov8_create.restype = ctypes.c_void_p
        L.or_fast_yolov8_create.argtypes = [ctypes.POINTER(YoloCfg), _f32p, ctypes.c_size_t]
        L.or_fast_yolov8_forward.argtypes = [ctypes.c_void_p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p,
                                             ctypes.c_size_t]
        L.or_fast_yolov8_destroy.argtypes = [ctypes.c_void_p]
        self.cfg = _cfg(depth, width, max_channels, nc, reg_max, bn_eps)
        p = _f32(params)
        self.handle = L.or_fast_yolov8_create(ctypes.byref(self.cfg), _p(p), ctypes.c_size_t(p.size))
        if not self.handle:
            raise ValueError("parameter vector does not match the YOLOv8 layout")

    @staticmethod
    def threads() -> int:
        return int(lib().or_fast_threads())

    def forward(self, x):
        x = _f32(x)
        batch, _, h, w = x.shape
        anchors = (h // 8) * (w // 8) + (h // 16) * (w // 16) + (h // 32) * (w // 32)
        out = np.empty((batch, self.cfg.nc + 4, anchors), np.float32)
        rc = lib().or_fast_yolov8_forward(self.handle, _p(x), batch, h, w, _p(out), ctypes.c_size_t(out.size))
        if rc:
            raise ValueError(f"CPU baseline forward failed ({rc})")
        return out

    def close(self):
        if self.handle:
            lib().or_fast_yolov8_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


def yolo11_layout(depth=0.50, width=0.25, max_channels=1024, nc=80, reg_max=16, bn_eps=1e-3, nm=0, npr=256):
    return _layout(lib().or_yolo11_layout, _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr))


def yolo11_forward(params, x, depth=0.50, width=0.25, max_channels=1024, nc=80, reg_max=16, bn_eps=1e-3, nm=0,
                   npr=256):
    return _forward(lib().or_yolo11_forward, _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr),
                    params, x, nm)


def yolo26_layout(depth=0.50, width=0.25, max_channels=1024, nc=80, reg_max=1, bn_eps=1e-3, nm=0, npr=256):
    return _layout(lib().or_yolo26_layout, _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr))


def yolo26_forward(params, x, depth=0.50, width=0.25, max_channels=1024, nc=80, reg_max=1, bn_eps=1e-3, nm=0,
                   npr=256):
    """Head before the end-to-end selection, [B, nc+4(+nm), A] with x1 y1 x2 y2
    boxes; with nm > 0 also the prototypes [B, nm, H/4, W/4]."""
    return _forward(lib().or_yolo26_forward, _cfg(depth, width, max_channels, nc, reg_max, bn_eps, nm, npr),
                    params, x, nm)
