"""Instance mask decode on the GPU vs the oracle (CpuMaskDecoder semantics).
Probabilities within 2e-6 absolute; crops identical."""
import numpy as np
import pytest

import oracle
from simdyolo_amd import _native as N
from simdyolo_amd import synth

pytestmark = pytest.mark.gpu


def run(hip, proto, coeffs, boxes, W, H, ld_extra=0):
    nm = proto.shape[0]
    _, tr = oracle.letterbox(np.zeros((H, W, 3), np.uint8), W, H, 640, 640)
    t = N.LetterboxT(tr.source_width, tr.source_height, tr.target_width, tr.target_height, tr.scale_x, tr.scale_y,
                     tr.pad_x, tr.pad_y)
    exp = [oracle.mask_decode(proto, coeffs[i], b, tr) for i, b in enumerate(boxes)]
    cap = sum(e[0].size for e in exp)
    hip.begin_frame()
    try:
        pv = hip.upload(proto[None])
        ld = nm + ld_extra
        rows = np.zeros((len(boxes), ld), np.float32)
        rows[:, ld_extra:] = coeffs
        cbuf = hip.malloc(rows.nbytes)
        out = hip.malloc(max(4, cap * 4))
        try:
            hip.h2d(cbuf, rows)
            info = hip.mask_decode(pv, cbuf + 4 * ld_extra, ld, boxes, t, out, cap)
            flat = hip.d2h(out, (cap,))
        finally:
            hip.free(cbuf)
            hip.free(out)
    finally:
        hip.end_frame()
    for (m, crop), (left, top, w, h, off) in zip(exp, info):
        assert (left, top, w, h) == crop
        got = flat[off:off + w * h].reshape(h, w)
        assert np.abs(got - m).max() <= 2e-6


@pytest.mark.parametrize("cfg", [(257, 193, 13, 11, 32), (19, 307, 9, 7, 32), (17, 19, 1, 1, 4),
                                 (101, 83, 17, 13, 8)])
def test_mask_decode_reference_shapes(hip, cfg):
    # Shapes of MaskPipelineTests.cs:12 (coefficient counts rounded to multiples of 4).
    W, H, P, Q, C = cfg
    r = np.random.Generator(np.random.PCG64(173))
    proto = (r.uniform(0, 4, (C, Q, P)) - 2).astype(np.float32)
    boxes = [(0.0, 0.0, float(W), float(H)), (0.2, 1.4, W * 0.73, H * 0.61), (W - 0.7, H - 0.6, 0.5, 0.4)]
    coeffs = (r.uniform(0, 1, (3, C)) - 0.5).astype(np.float32)
    run(hip, proto, coeffs, boxes, W, H)
    run(hip, proto, coeffs, boxes, W, H, ld_extra=6)  # rows of an end-to-end top-k output


def test_mask_decode_yolo26_scale(hip):
    r = np.random.Generator(np.random.PCG64(5))
    W, H, nm, k = 640, 480, 32, 300
    proto = synth.activations((nm, 160, 160), 6)
    coeffs = synth.activations((k, nm), 7) * np.float32(0.3)
    xy = r.uniform(0, 1, (k, 2)) * np.array([W - 40, H - 40])
    wh = r.uniform(4, 40, (k, 2))
    boxes = [(float(a), float(b), float(c), float(d)) for (a, b), (c, d) in zip(xy, wh)]
    run(hip, proto, coeffs, boxes, W, H, ld_extra=6)


def test_masks_from_segment_model_outputs(hip):
    """End to end: a YOLOv8n-seg forward, NMS on its head, then mask decode reading
    the model's own device prototype buffer (NCHW) and the head's coefficients,
    vs the oracle's forward + mask decode on the same detections."""
    from simdyolo_amd.detector import YoloDetector
    nm, size = 32, 320
    cfg = synth.config("n", nm=nm, npr=256)
    params = synth.params_for_layout(synth.layout(cfg), seed=synth.SEED + 41, cls_bias=0.0)
    x = synth.images(1, size, size, seed=43)
    exp_head, exp_proto = oracle.yolov8_forward(params, x, nm=nm, npr=256)
    tr = oracle.Letterbox(size, size, size, size, 1.0, 1.0, 0, 0)
    dets = oracle.nms_decode(exp_head[0][:84], layout=0, confidence=0.25, transform=tr)[:40]
    assert len(dets) >= 5
    boxes = []
    for d in dets:
        x0, y0 = max(0.0, d.x), max(0.0, d.y)
        x1, y1 = min(float(size), d.x + d.width), min(float(size), d.y + d.height)
        if x1 - x0 >= 1 and y1 - y0 >= 1:
            boxes.append((x0, y0, x1 - x0, y1 - y0, d.anchor))
    t = N.LetterboxT(size, size, size, size, 1.0, 1.0, 0, 0)
    with YoloDetector(cfg, params, ctx=hip) as det:
        head, _ = det.predict_seg(x)
        pptr, (c, ph, pw) = det.proto_buffer(1, size, size)
        assert (c, ph, pw) == (nm, size // 4, size // 4)
        rows = np.ascontiguousarray(np.stack([head[0, 84:, b[4]] for b in boxes]), np.float32)
        exp = [oracle.mask_decode(exp_proto[0], exp_head[0, 84:, b[4]], b[:4], tr) for b in boxes]
        cap = sum(e[0].size for e in exp)
        protos = N.Tensor(pptr, 1, nm, ph, pw, nm, N.LAYOUT_NCHW)
        cbuf = hip.malloc(rows.nbytes)
        out = hip.malloc(cap * 4)
        try:
            hip.h2d(cbuf, rows)
            info = hip.mask_decode(protos, cbuf, nm, [b[:4] for b in boxes], t, out, cap)
            flat = hip.d2h(out, (cap,))
        finally:
            hip.free(cbuf)
            hip.free(out)
    worst = 0.0
    for (m, crop), (left, top, w, h, off) in zip(exp, info):
        assert (left, top, w, h) == crop
        worst = max(worst, float(np.abs(flat[off:off + w * h].reshape(h, w) - m).max()))
    print(f"{len(boxes)} instances, max |p - p_ref| {worst:.2e}")
    assert worst <= 1e-3
