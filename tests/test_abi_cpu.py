"""CPU-side checks of the C-ABI library: it loads, exports every symbol the
header declares, and its host-only functions (BN fold, letterbox, detection
decoder, parameter layout) agree with the oracle.  No GPU calls."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from simdyolo_amd import _native as N
from simdyolo_amd import synth
from simdyolo_amd.detector import DetectorOptions, decode_detections

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_symbols():
    text = open(os.path.join(ROOT, "include", "simdyolo_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sy_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    declared = _header_symbols()
    assert len(declared) >= 40
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(N.EXPORTS) == declared


def test_device_count_without_gpu_is_clean():
    n = ctypes.c_int(-1)
    N.check(N.lib().sy_device_count(ctypes.byref(n)))
    assert n.value >= 0


def test_null_arguments_are_rejected():
    lib = N.lib()
    assert lib.sy_create(0, None) == N.SY_EINVAL
    assert lib.sy_frame_begin(None, None) == N.SY_EINVAL
    assert b"null" in lib.sy_last_error()


@pytest.mark.parametrize("scale", ["n", "s", "m"])
def test_layout_matches_oracle(scale):
    cfg = synth.config(scale)
    d, w, mc = synth.SCALES[scale]
    assert np.array_equal(synth.layout(cfg), oracle.yolov8_layout(d, w, mc))


@pytest.mark.parametrize("scale", ["n", "s", "m", "l"])
def test_yolo11_layout_matches_oracle(scale):
    cfg = synth.config(scale, arch="yolo11")
    d, w, mc = synth.SCALES_11[scale]
    assert np.array_equal(synth.layout(cfg), oracle.yolo11_layout(d, w, mc))


@pytest.mark.parametrize("arch", ["yolov8", "yolo11"])
@pytest.mark.parametrize("scale", ["n", "s"])
def test_segment_layout_matches_oracle(arch, scale):
    cfg = synth.config(scale, arch=arch, nm=32, npr=256)
    if arch == "yolov8":
        d, w, mc = synth.SCALES[scale]
        exp = oracle.yolov8_layout(d, w, mc, nm=32, npr=256)
    else:
        d, w, mc = synth.SCALES_11[scale]
        exp = oracle.yolo11_layout(d, w, mc, nm=32, npr=256)
    assert np.array_equal(synth.layout(cfg), exp)


@pytest.mark.parametrize("nm", [0, 32])
@pytest.mark.parametrize("scale", ["n", "s", "m"])
def test_yolo26_layout_matches_oracle(scale, nm):
    cfg = synth.config(scale, arch="yolo26", nm=nm, npr=256)
    d, w, mc = synth.SCALES_11[scale]
    assert np.array_equal(synth.layout(cfg), oracle.yolo26_layout(d, w, mc, reg_max=1, nm=nm, npr=256))


def test_fold_bn_bit_exact():
    r = np.random.Generator(np.random.PCG64(1))
    w = r.standard_normal((8, 3, 3, 3)).astype(np.float32)
    cb = r.standard_normal(8).astype(np.float32)
    g, b = r.uniform(.5, 1.5, 8).astype(np.float32), r.standard_normal(8).astype(np.float32)
    m, v = r.standard_normal(8).astype(np.float32), r.uniform(.1, 2, 8).astype(np.float32)
    wo, bo = np.empty_like(w), np.empty(8, np.float32)
    N.lib().sy_fold_bn(N.fptr(w), 8, 27, N.fptr(cb), N.fptr(g), N.fptr(b), N.fptr(m), N.fptr(v),
                       ctypes.c_float(1e-3), N.fptr(wo), N.fptr(bo))
    ew, eb = oracle.fold_bn(w, cb, g, b, m, v, 1e-3)
    assert np.array_equal(wo.view(np.uint32), ew.view(np.uint32))
    assert np.array_equal(bo.view(np.uint32), eb.view(np.uint32))


@pytest.mark.parametrize("src,dst", [((2, 1), (4, 4)), ((640, 480), (640, 640)), ((333, 517), (320, 320)),
                                     ((64, 64), (64, 64))])
def test_letterbox_bit_exact(src, dst):
    w, h = src
    r = np.random.Generator(np.random.PCG64(w * h))
    px = r.integers(0, 256, (h, w, 3), dtype=np.uint8)
    for bgr in (False, True):
        exp, et = oracle.letterbox(px, w, h, dst[0], dst[1], bgr=bgr)
        got = np.empty_like(exp)
        t = N.LetterboxT()
        N.check(N.lib().sy_letterbox_rgb(px.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), w, h, dst[0], dst[1],
                                         int(bgr), 0, N.fptr(got), ctypes.byref(t)))
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
        assert (t.pad_x, t.pad_y, t.scale_x, t.scale_y) == (et.pad_x, et.pad_y, et.scale_x, et.scale_y)


@pytest.mark.parametrize("seed", range(4))
def test_decode_detections_matches_oracle(seed):
    r = np.random.Generator(np.random.PCG64(seed))
    n, nc = 2000, 7
    head = np.zeros((4 + nc, n), np.float32)
    head[:2] = r.uniform(0, 640, (2, n))
    head[2:4] = r.uniform(-2, 90, (2, n))
    head[4:] = r.uniform(0, 0.6, (nc, n))
    head[4:, ::17] = head[4, ::17]  # exact class ties
    head[0, 5] = np.nan
    tx = N.LetterboxT(500, 400, 640, 640, 1.28, 1.28, 0, 64)
    o = DetectorOptions(class_count=nc)
    got = decode_detections(head, o, tx)
    exp = oracle.nms_decode(head, layout=0, class_count=nc,
                            transform=oracle.Letterbox(500, 400, 640, 640, 1.28, 1.28, 0, 64))
    assert [(d.anchor, d.class_id) for d in got] == [(d.anchor, d.class_id) for d in exp]
    for a, b in zip(got, exp):
        assert (a.x, a.y, a.width, a.height, a.confidence) == (b.x, b.y, b.width, b.height, b.confidence)


def test_decode_detections_reference_kat():
    out = np.array([10, 10, 10, 10, .9, .1, 10, 10, 10, 10, .8, .1, 10, 10, 10, 10, .1, .95], np.float32)
    o = DetectorOptions(output_layout=N.LAYOUT_NCHW + 1, width=20, height=20)  # channels-last
    assert len(decode_detections(out.reshape(3, 6), o)) == 2
    end = np.array([1, 1, 10, 10, .9, 0, 1, 1, 10, 10, .8, 0], np.float32).reshape(2, 6)
    o.output_layout = 3
    assert len(decode_detections(end, o)) == 2


def _compute(op, inputs, lengths, params, items, out_len):
    lib = N.lib()
    ptrs = (ctypes.c_void_p * 3)(*[ctypes.c_void_p(p) if p else None for p in inputs])
    lens = (ctypes.c_size_t * 3)(*lengths)
    block = (ctypes.c_uint32 * 32)(*params)
    out = ctypes.c_void_p(0x1000)  # never dereferenced: every case is refused on the host
    return lib.sy_compute(None, op, ptrs, lens, block, ctypes.c_int64(items), out, ctypes.c_size_t(out_len))


def test_compute_refuses_zero_length_binding_before_launch():
    """A bound input with length 0 is refused (it holds no element to read),
    before the context is even looked at; the same call with the binding
    absent passes the argument checks and only then fails on the null
    context."""
    p = [0] * 32
    p[0] = 8
    dummy = 0x2000
    assert _compute(32, [dummy, dummy, dummy], [64, 9, 0], p, 8, 64) == N.SY_EINVAL
    assert b"length 0" in N.lib().sy_last_error()
    assert _compute(10, [dummy, dummy, None], [64, 0, 0], p, 8, 64) == N.SY_EINVAL
    assert b"length 0" in N.lib().sy_last_error()
    assert _compute(1, [dummy, None, None], [64, 0, 0], p, 8, 64) == N.SY_EINVAL
    assert b"null context" in N.lib().sy_last_error()
    assert _compute(17, [dummy, None, None], [64, 0, 0], p, 8, 64) == N.SY_EUNSUPPORTED
