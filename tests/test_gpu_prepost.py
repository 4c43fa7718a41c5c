"""Device pre/post-processing against the host restatements of the reference.

* sy_letterbox_device must equal the oracle letterbox (itself pinned to the
  reference's KAT and identity case) bit for bit, for scaled, padded, BGR and
  strided images.
* sy_decode_detections_device (GPU candidates + host greedy NMS) must return
  exactly the oracle's DecodeIndexed result, including score ties (stable
  order), NaN/inf scores and boxes, non-positive sizes and truncation to
  max_candidates.
"""
import ctypes

import numpy as np
import pytest

import oracle
from simdyolo_amd import _native as N

pytestmark = pytest.mark.gpu


def _device_letterbox(hip, img, w, h, tw, th, bgr, row_stride):
    raw = np.ascontiguousarray(img, dtype=np.uint8)
    src = hip.malloc(raw.nbytes)
    dst = hip.malloc(3 * tw * th * 4)
    try:
        hip.h2d(src, raw)
        t = N.LetterboxT()
        N.check(N.lib().sy_letterbox_device(hip.handle, src, w, h, tw, th, int(bgr), row_stride, dst,
                                            ctypes.byref(t)))
        out = hip.d2h(dst, (1, 3, th, tw))
    finally:
        hip.free(src)
        hip.free(dst)
    return out, t


LETTERBOX_CASES = [
    # (width, height, tw, th, bgr, row padding bytes)
    (640, 640, 640, 640, False, 0),
    (500, 375, 640, 640, False, 0),
    (1280, 720, 640, 640, True, 0),
    (33, 47, 64, 96, False, 5),
    (719, 1283, 320, 320, True, 3),
    (1, 1, 32, 32, False, 0),
]


@pytest.mark.parametrize("case", LETTERBOX_CASES, ids=lambda c: "x".join(map(str, c)))
def test_letterbox_device_bit_exact(hip, case):
    w, h, tw, th, bgr, pad = case
    stride = w * 3 + pad
    rng = np.random.Generator(np.random.PCG64(w * 7 + h))
    img = rng.integers(0, 256, size=(h, stride), dtype=np.uint8)
    got, t = _device_letterbox(hip, img, w, h, tw, th, bgr, stride)
    exp, te = oracle.letterbox(img, w, h, tw, th, bgr=bgr, row_stride=stride)
    assert np.array_equal(got, exp)
    assert (t.scale_x, t.scale_y, t.pad_x, t.pad_y) == (te.scale_x, te.scale_y, te.pad_x, te.pad_y)


def _head(batch, nc, anchors, seed):
    """Heads with many exact score ties, some NaN/inf and degenerate boxes."""
    rng = np.random.Generator(np.random.PCG64(seed))
    h = np.empty((batch, 4 + nc, anchors), np.float32)
    h[:, 0] = rng.uniform(0, 640, (batch, anchors))
    h[:, 1] = rng.uniform(0, 640, (batch, anchors))
    h[:, 2] = rng.uniform(-5, 120, (batch, anchors))
    h[:, 3] = rng.uniform(-5, 120, (batch, anchors))
    h[:, 4:] = np.floor(rng.uniform(0, 1, (batch, nc, anchors)) * 64) / 64
    k = anchors // 50
    idx = rng.choice(anchors, k, replace=False)
    h[0, 4 + 3, idx[: k // 3]] = np.nan
    h[0, 4 + 5, idx[k // 3: 2 * k // 3]] = np.inf
    h[min(1, batch - 1), 0, idx[2 * k // 3:]] = np.inf
    return h


def _device_decode(hip, head, opts, transforms, max_out):
    b, c, a = head.shape
    dev = hip.malloc(head.nbytes)
    try:
        hip.h2d(dev, np.ascontiguousarray(head))
        out = (N.DetectionT * (b * max_out))()
        counts = (ctypes.c_int * b)()
        lbs = (N.LetterboxT * b)(*transforms)
        N.check(N.lib().sy_decode_detections_device(hip.handle, dev, b, c, a, ctypes.byref(opts), lbs, out,
                                                    max_out, counts))
    finally:
        hip.free(dev)
    return [[out[i * max_out + j] for j in range(counts[i])] for i in range(b)]


def _key(d):
    return (d.anchor, d.class_id, d.confidence, d.x, d.y, d.width, d.height)


@pytest.mark.parametrize("conf,iou,max_cand,agnostic", [(0.5, 0.45, 30000, 0), (0.25, 0.7, 30000, 1),
                                                         (0.8, 0.45, 100, 0), (0.0, 0.45, 30000, 0)])
def test_decode_device_equals_oracle(hip, conf, iou, max_cand, agnostic):
    nc, anchors = 80, 8400
    head = _head(3, nc, anchors, seed=int(conf * 100) + max_cand)
    lb = oracle.Letterbox(500, 375, 640, 640, 1.28, 1.28, 0, 80)
    opts = N.DecodeOptions(conf, iou, 300, max_cand, nc, agnostic, 1)
    tr = [N.LetterboxT(500, 375, 640, 640, 1.28, 1.28, 0, 80)] * 3
    got = _device_decode(hip, head, opts, tr, 300)
    for b in range(3):
        exp = oracle.nms_decode(head[b], layout=1, confidence=conf, iou=iou, max_candidates=max_cand,
                                agnostic=bool(agnostic), class_count=nc, transform=lb)
        assert [_key(d) for d in got[b]] == [_key(d) for d in exp], f"image {b}"
        assert len(exp) > 0


@pytest.mark.parametrize("conf,max_cand", [(0.0, 30000), (0.3, 30000), (0.0, 20000)])
def test_decode_device_1280(hip, conf, max_cand):
    """33600 anchors (a 1280x1280 input): with a low threshold more than 16384
    candidates pass, so the sort runs through the global work buffer; the
    30000 / 20000 candidate cut keeps ties in anchor order."""
    nc, anchors = 80, 33600
    head = _head(2, nc, anchors, seed=1280 + int(conf * 10) + max_cand)
    lb = oracle.Letterbox(1280, 1280, 1280, 1280, 1.0, 1.0, 0, 0)
    opts = N.DecodeOptions(conf, 0.45, 300, max_cand, nc, 0, 1)
    tr = [N.LetterboxT(1280, 1280, 1280, 1280, 1.0, 1.0, 0, 0)] * 2
    got = _device_decode(hip, head, opts, tr, 300)
    for b in range(2):
        exp = oracle.nms_decode(head[b], layout=1, confidence=conf, iou=0.45, max_candidates=max_cand,
                                class_count=nc, transform=lb)
        assert [_key(d) for d in got[b]] == [_key(d) for d in exp], f"image {b}"
        assert len(exp) > 0


def test_nms_candidates_1280_count(hip):
    """The candidate stage alone at 33600 anchors: count and order equal a
    stable descending sort of the passing anchors (more than one LDS block)."""
    nc, anchors, batch = 80, 33600, 1
    head = _head(batch, nc, anchors, seed=77)
    opts = N.DecodeOptions(0.0, 0.45, 300, 30000, nc, 0, 1)
    dev = hip.malloc(head.nbytes)
    cand = hip.malloc(batch * 30000 * ctypes.sizeof(N.DetectionT))
    cnt = hip.malloc(4 * batch)
    try:
        hip.h2d(dev, head)
        N.check(N.lib().sy_nms_candidates(hip.handle, dev, batch, 4 + nc, anchors, ctypes.byref(opts), cand, cnt))
        hip.flush()
        n = int(hip.d2h(cnt, (batch,), np.int32)[0])
        raw = hip.d2h(cand, (30000 * ctypes.sizeof(N.DetectionT) // 4,), np.float32)
    finally:
        for ptr in (dev, cand, cnt):
            hip.free(ptr)
    rec = np.frombuffer(raw.tobytes(), dtype=np.dtype([("cls", "<i4"), ("conf", "<f4"), ("x", "<f4"), ("y", "<f4"),
                                                         ("w", "<f4"), ("h", "<f4"), ("anchor", "<i4")]))[:n]
    scores = head[0, 4:]
    with np.errstate(invalid="ignore"):
        best = np.where(np.isnan(scores), -np.inf, scores).max(0)
    boxes_ok = np.isfinite(head[0, :4]).all(0) & (head[0, 2] > 0) & (head[0, 3] > 0)
    passing = np.nonzero(np.isfinite(best) & (best >= 0.0) & boxes_ok)[0]
    order = passing[np.argsort(-best[passing], kind="stable")][:30000]
    assert n == len(order) and n > 16384
    np.testing.assert_array_equal(rec["anchor"], order)


def test_decode_device_rejects_end_to_end_layout(hip):
    from simdyolo_amd import SyError
    head = np.zeros((1, 6, 300), np.float32)
    opts = N.DecodeOptions(0.25, 0.45, 300, 30000, 0, 0, 3)
    with pytest.raises(SyError):
        _device_decode(hip, head, opts, [N.LetterboxT(640, 640, 640, 640, 1.0, 1.0, 0, 0)], 300)
