"""Whole-network parity: YOLOv8 forward on the HIP backend vs the CPU oracle
on the same seeded weights and images.

Bars (from the build target): raw head within max-rel 1e-3 (relative to
max(1, |ref|), as the reference's Near), detection index sets after NMS equal
except where scores tie within 1e-5, matched boxes IoU >= 0.999.
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import synth
from simdyolo_amd.detector import YoloDetector
from _parity import adaptive_threshold, check_detections, max_rel

pytestmark = pytest.mark.gpu

HEAD_TOL = 1e-3


@pytest.fixture(scope="module")
def v8n(hip):
    cfg = synth.config("n")
    params = synth.params(cfg)
    det = YoloDetector(cfg, params, ctx=hip)
    yield det, params
    det.close()


@pytest.mark.parametrize("batch,size", [(1, 640), (2, 320), (1, 256)])
def test_yolov8n_head_parity(v8n, batch, size):
    det, params = v8n
    x = synth.images(batch, size, size, seed=size + batch)
    got = det.predict_raw(x)
    exp = oracle.yolov8_forward(params, x)
    assert got.shape == exp.shape == (batch, 84, (size // 8) ** 2 + (size // 16) ** 2 + (size // 32) ** 2)
    err = max_rel(got, exp)
    print(f"v8n b{batch} {size}: max-rel {err:.3e}")
    assert err <= HEAD_TOL
    for b in range(batch):
        ng, ne = check_detections(got[b], exp[b])
        thr = adaptive_threshold(exp[b])
        ng2, ne2 = check_detections(got[b], exp[b], conf=thr)
        print(f"  image {b}: {ng} / {ne} detections @0.25, {ng2} / {ne2} @{thr:.5f} (gpu / oracle)")
        assert ng2 >= 10


@pytest.mark.parametrize("chunks", [3, 7])
def test_predict_raw_chunk_pipeline(v8n, monkeypatch, chunks):
    """PredictRaw from host buffers split into chunks (forced through
    SIMDYOLO_HIP_IO_CHUNKS): uploads, forwards and downloads of consecutive
    chunks overlap on separate threads and streams, and the staging buffers
    of chunk k are reused by chunk k + 2.  Seven images as 3 + 3 + 1 or as
    seven chunks of one: every image against the oracle, and a second call
    bit-identical to the first."""
    monkeypatch.setenv("SIMDYOLO_HIP_IO_CHUNKS", str(chunks))
    det, params = v8n
    x = synth.images(7, 320, 320, seed=77)
    got = det.predict_raw(x)
    again = det.predict_raw(x)
    assert again.tobytes() == got.tobytes()
    exp = oracle.yolov8_forward(params, x)
    assert got.shape == exp.shape == (7, 84, 2100)
    worst = max(max_rel(got[i], exp[i]) for i in range(7))
    print(f"v8n b7 320 in {chunks} chunks: worst max-rel {worst:.3e}")
    assert worst <= HEAD_TOL


@pytest.mark.parametrize("batch,h,w", [(32, 320, 448), (17, 256, 352)])
def test_predict_raw_default_chunks_match_resident(v8n, hip, batch, h, w):
    """PredictRaw from host buffers with the default chunking (two chunks from
    16 images: 16 + 16, or 9 + 8 on two chunk plans) at non-square sizes,
    whose head rows split unevenly over the staging pieces and the copy
    threads: every chunk's rows bit-equal to the same chunk plan run on
    resident buffers (the branch level does not change the bits)."""
    det, _ = v8n
    x = synth.images(batch, h, w, seed=batch + h)
    got = det.predict_raw(x)
    assert got.shape == det.output_shape(batch, h, w)
    chunk = (batch + 1) // 2
    for i0 in range(0, batch, chunk):
        n = min(chunk, batch - i0)
        inp, out = det.buffers(n, h, w)
        hip.h2d(inp, x[i0:i0 + n])
        det.run(n, h, w)
        hip.flush()
        np.testing.assert_array_equal(got[i0:i0 + n], hip.d2h(out, det.output_shape(n, h, w)))
    np.testing.assert_array_equal(det.predict_raw(x), got)


def test_predict_seg_default_chunks_match_resident(hip):
    """The same for a Segment model: two chunks of eight images, the head rows
    and then the prototypes of each chunk coming down through the staging,
    bit-equal to the chunk plan's resident head and prototype buffers."""
    cfg = synth.config("n", nm=32, npr=64)
    params = synth.params(cfg)
    batch, h, w = 16, 224, 288
    x = synth.images(batch, h, w, seed=16)
    with YoloDetector(cfg, params, ctx=hip) as det:
        head, protos = det.predict_seg(x)
        for i0 in (0, 8):
            inp, out = det.buffers(8, h, w)
            hip.h2d(inp, x[i0:i0 + 8])
            det.run(8, h, w)
            hip.flush()
            np.testing.assert_array_equal(head[i0:i0 + 8], hip.d2h(out, det.output_shape(8, h, w)))
            p, shape = det.proto_buffer(8, h, w)
            np.testing.assert_array_equal(protos[i0:i0 + 8], hip.d2h(p, (8,) + shape))


@pytest.mark.parametrize("arch,batch,h,w", [("yolov8", 3, 32, 32), ("yolov8", 2, 64, 96), ("yolo11", 2, 32, 64),
                                            ("yolov8", 40, 32, 32)])
def test_smallest_inputs(hip, arch, batch, h, w):
    """The smallest inputs: at 32x32 the stride-32 level is one pixel (SPPF
    pools a 1x1 plane, every Winograd tile is partial, the upsamples double
    1x1 maps); a batch of 40 such images also runs the host-buffer pipeline
    as two chunks.  Every image against the oracle."""
    cfg = synth.config("n", arch=arch)
    d, wd, mc = (synth.SCALES if arch == "yolov8" else synth.SCALES_11)["n"]
    params = synth.params(cfg)
    x = synth.images(batch, h, w, seed=h * w + batch)
    fwd = oracle.yolov8_forward if arch == "yolov8" else oracle.yolo11_forward
    with YoloDetector(cfg, params, ctx=hip) as det:
        got = det.predict_raw(x)
    for i in range(batch):
        exp = fwd(params, x[i:i + 1], depth=d, width=wd, max_channels=mc)[0]
        assert max_rel(got[i], exp) <= HEAD_TOL, f"image {i}"


def test_yolov8n_1280_head_and_device_decode(v8n):
    """A 1280x1280 input (33600 anchors, more than one LDS sort block):
    whole-network head parity, then the device candidate stage + host NMS
    equal to the oracle's decode of the oracle's head at a threshold that
    admits a few thousand candidates."""
    import ctypes
    from simdyolo_amd import _native as N
    det, params = v8n
    x = synth.images(1, 1280, 1280, seed=1280)
    got = det.predict_raw(x)
    exp = oracle.yolov8_forward(params, x)
    assert got.shape == (1, 84, 33600)
    assert max_rel(got, exp) <= HEAD_TOL
    conf = adaptive_threshold(exp[0], candidates=4000)
    hip = det.ctx
    dev = hip.malloc(got.nbytes)
    try:
        hip.h2d(dev, got)
        opts = N.DecodeOptions(conf, 0.45, 300, 30000, 80, 0, 1)
        lb = N.LetterboxT(1280, 1280, 1280, 1280, 1.0, 1.0, 0, 0)
        out = (N.DetectionT * 300)()
        cnt = (ctypes.c_int * 1)()
        N.check(N.lib().sy_decode_detections_device(hip.handle, dev, 1, 84, 33600, ctypes.byref(opts),
                                                    ctypes.byref(lb), out, 300, cnt))
    finally:
        hip.free(dev)
    dets = [(d.anchor, d.class_id) for d in out[:cnt[0]]]
    ref = oracle.nms_decode(got[0], layout=1, confidence=conf, transform=oracle.Letterbox(1280, 1280, 1280, 1280,
                                                                                          1.0, 1.0, 0, 0))
    assert dets == [(d.anchor, d.class_id) for d in ref] and len(dets) > 10
    n_got, n_exp = check_detections(got[0], exp[0], conf=conf, size=1280)
    assert n_exp > 10


def test_yolov8n_parity_with_zero_class_bias(hip):
    """Second seeded weight set with class bias 0 (scores spread over (0, 1)),
    so the default 0.25 threshold keeps many detections."""
    cfg = synth.config("n")
    params = synth.params_for_layout(synth.layout(cfg), seed=synth.SEED + 3, cls_bias=0.0)
    x = synth.images(2, 640, 640, seed=5)
    with YoloDetector(cfg, params, ctx=hip) as det:
        got = det.predict_raw(x)
    exp = oracle.yolov8_forward(params, x)
    err = max_rel(got, exp)
    print(f"v8n cls-bias 0, b2 640: max-rel {err:.3e}")
    assert err <= HEAD_TOL
    for b in range(2):
        ng, ne = check_detections(got[b], exp[b])
        print(f"  image {b}: {ng} / {ne} detections @0.25 (gpu / oracle)")
        assert ne >= 10


def test_graph_replay_and_eager_agree(v8n):
    det, _ = v8n
    x = synth.images(2, 320, 320, seed=99)
    first = det.predict_raw(x)       # captures the graph
    second = det.predict_raw(x)      # replays it
    det.set_graph(False)
    try:
        eager = det.predict_raw(x)
    finally:
        det.set_graph(True)
    np.testing.assert_array_equal(first, second)
    np.testing.assert_array_equal(first, eager)
    # A different input through the same graph must change the output.
    y = synth.images(2, 320, 320, seed=100)
    other = det.predict_raw(y)
    assert not np.array_equal(other, first)
    np.testing.assert_array_equal(det.predict_raw(x), first)


def test_public_outputs_are_independent(v8n):
    det, _ = v8n
    a = det.predict_raw(synth.images(1, 256, 256, seed=1))
    saved = a.copy()
    det.predict_raw(synth.images(1, 256, 256, seed=2))
    np.testing.assert_array_equal(a, saved)


def test_invalid_input_shape_rejected(v8n):
    from simdyolo_amd import SyError
    det, _ = v8n
    with pytest.raises(SyError):
        det.predict_raw(np.zeros((1, 3, 100, 100), np.float32))


@pytest.mark.parametrize("scale,batch,size", [("s", 1, 256), ("m", 2, 320)])
def test_scaled_yolov8_parity(hip, scale, batch, size):
    cfg = synth.config(scale)
    d, w, mc = synth.SCALES[scale]
    params = synth.params(cfg, seed=synth.SEED + 11)
    x = synth.images(batch, size, size, seed=17)
    with YoloDetector(cfg, params, ctx=hip) as det:
        got = det.predict_raw(x)
    exp = oracle.yolov8_forward(params, x, depth=d, width=w, max_channels=mc)
    err = max_rel(got, exp)
    print(f"v8{scale} b{batch} {size}: max-rel {err:.3e}")
    assert err <= HEAD_TOL


@pytest.mark.parametrize("scale,batch,size", [("n", 1, 640), ("n", 2, 320), ("s", 1, 256)])
def test_yolo11_parity(hip, scale, batch, size):
    """YOLO11 (C3k2, C2PSA attention, depthwise class branch) vs the oracle."""
    cfg = synth.config(scale, arch="yolo11")
    d, w, mc = synth.SCALES_11[scale]
    params = synth.params(cfg, seed=synth.SEED + 21)
    x = synth.images(batch, size, size, seed=23)
    with YoloDetector(cfg, params, ctx=hip) as det:
        got = det.predict_raw(x)
    exp = oracle.yolo11_forward(params, x, depth=d, width=w, max_channels=mc)
    err = max_rel(got, exp)
    print(f"yolo11{scale} b{batch} {size}: max-rel {err:.3e}")
    assert err <= HEAD_TOL
    if size == 640:
        conf = adaptive_threshold(exp[0])
        n_got, n_exp = check_detections(got[0], exp[0], conf)
        assert n_exp > 0 and abs(n_got - n_exp) <= 2


@pytest.mark.parametrize("arch,batch,size", [("yolov8", 1, 640), ("yolov8", 2, 320), ("yolo11", 1, 640),
                                             ("yolo11", 2, 256)])
def test_segment_parity(hip, arch, batch, size):
    """Segment head: detection head with nm mask coefficients appended, and the
    Proto output (3x3 conv, 2x2 stride-2 ConvTranspose, 3x3, 1x1) vs the oracle."""
    nm, npr = 32, 256
    cfg = synth.config("n", arch=arch, nm=nm, npr=npr)
    d, w, mc = (synth.SCALES if arch == "yolov8" else synth.SCALES_11)["n"]
    params = synth.params(cfg, seed=synth.SEED + 31)
    x = synth.images(batch, size, size, seed=37)
    with YoloDetector(cfg, params, ctx=hip) as det:
        got, protos = det.predict_seg(x)
        again, protos2 = det.predict_seg(x)   # graph replay
    fwd = oracle.yolov8_forward if arch == "yolov8" else oracle.yolo11_forward
    exp, exp_protos = fwd(params, x, depth=d, width=w, max_channels=mc, nm=nm, npr=npr)
    assert got.shape == exp.shape and got.shape[1] == 84 + nm
    assert protos.shape == exp_protos.shape == (batch, nm, size // 4, size // 4)
    e_head, e_proto = max_rel(got, exp), max_rel(protos, exp_protos)
    print(f"{arch}n-seg b{batch} {size}: head max-rel {e_head:.3e}, proto max-rel {e_proto:.3e}")
    assert e_head <= HEAD_TOL and e_proto <= HEAD_TOL
    np.testing.assert_array_equal(got, again)
    np.testing.assert_array_equal(protos, protos2)
    # The prototypes are not constant (a dead branch would pass a loose bar).
    assert float(exp_protos.std()) > 1e-2


def test_tuning_table_reproduces_choices(tmp_path):
    """A context that loads another's tuning table runs the same kernels:
    its forward is bit-identical, and no candidate is timed again."""
    from simdyolo_amd import SyError
    from simdyolo_amd.device import HipContext
    cfg = synth.config("n")
    params = synth.params(cfg)
    x = synth.images(2, 320, 320, seed=5)
    table = str(tmp_path / "tune.txt")
    with YoloDetector(cfg, params) as a:
        ref = a.predict_raw(x)
        a.ctx.tune_save(table)
    lines = open(table).read().splitlines()
    assert lines[0].startswith("simdyolo_hip tune") and len(lines) > 20
    ctx = HipContext(0)
    try:
        ctx.tune_load(table)
        with YoloDetector(cfg, params, ctx=ctx) as b:
            got = b.predict_raw(x)
        np.testing.assert_array_equal(got, ref)
        again = str(tmp_path / "again.txt")
        ctx.tune_save(again)
        assert sorted(open(again).read().splitlines()) == sorted(lines)
        bad = tmp_path / "bad.txt"
        bad.write_text("not a table\n")
        with pytest.raises(SyError):
            ctx.tune_load(str(bad))
    finally:
        ctx.close()


@pytest.mark.parametrize("arch,nm", [("yolov8", 0), ("yolov8", 32), ("yolo11", 0)])
def test_branch_levels_agree(hip, arch, nm):
    """The captured forward with the P3 (and P4) heads on a second stream
    computes the same head (and prototypes) as the eager single-stream pass,
    bit for bit, at every branch level and replay."""
    cfg = synth.config("n", arch=arch, nm=nm)
    params = synth.params(cfg)
    x = synth.images(2, 256, 320, seed=11)
    with YoloDetector(cfg, params, ctx=hip) as det:
        det.set_graph(False)
        eager = det.predict_raw(x)
        eager_proto = det.predict_seg(x)[1] if nm else None
        det.set_graph(True)
        assert det.branch_level(2, 256, 320) == -1
        for level in (0, 1, 2, -1):
            det.set_branch_level(level)
            for _ in range(2):
                np.testing.assert_array_equal(det.predict_raw(x), eager)
                if nm:
                    np.testing.assert_array_equal(det.predict_seg(x)[1], eager_proto)
            got = det.branch_level(2, 256, 320)
            assert got == level if level >= 0 else got in (0, 1, 2)
