"""Whole-network parity on the benchmarked path at the benchmarked sizes.

The throughput runs plan a batch on resident device buffers, tune every
convolution on the first (eager) pass, capture the forward as a graph at the
branch level that times fastest, and replay it.  These tests drive exactly
that sequence (sy_model_buffers, sy_model_run) and compare the head with the
oracle: every image of YOLOv8n and YOLO11n at batch 32, and images 0, 31 and
63 of YOLOv8m at batch 64.  The pattern follows the reference's whole-model
CPU-vs-device check (tests/SimdYolo.Tests/Program.cs:575-601).

Bar: max-rel 1e-3 on the raw head (relative to max(1, |ref|)); NMS index sets
equal except near-ties, matched boxes IoU >= 0.999.
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import synth
from simdyolo_amd.detector import YoloDetector
from _parity import adaptive_threshold, check_detections, max_rel

pytestmark = pytest.mark.gpu

HEAD_TOL = 1e-3


def bench_forward(det, x, replays=3):
    """Resident-buffer forward as the throughput run does it: the first run
    tunes eagerly and captures; later runs replay the graph."""
    b, _, h, w = x.shape
    inp, out = det.buffers(b, h, w)
    ctx = det.ctx
    ctx.h2d(inp, x)
    ctx.flush()
    for _ in range(replays):
        det.run(b, h, w)
    ctx.flush()
    level = det.branch_level(b, h, w)
    assert level in (0, 1, 2), "the forward did not run as a captured graph"
    return ctx.d2h(out, det.output_shape(b, h, w)), level


@pytest.mark.timeout(600)
@pytest.mark.parametrize("arch", ["yolov8", "yolo11"])
def test_nano_batch32_640_every_image(arch):
    cfg = synth.config("n", arch=arch)
    d, w, mc = (synth.SCALES if arch == "yolov8" else synth.SCALES_11)["n"]
    params = synth.params(cfg)
    x = synth.images(32, 640, 640)  # the throughput run's input
    with YoloDetector(cfg, params) as det:
        got, level = bench_forward(det, x)
    fwd = oracle.yolov8_forward if arch == "yolov8" else oracle.yolo11_forward
    worst = 0.0
    for i in range(32):
        exp = fwd(params, x[i:i + 1], depth=d, width=w, max_channels=mc)[0]
        err = max_rel(got[i], exp)
        worst = max(worst, err)
        assert err <= HEAD_TOL, f"image {i}: max-rel {err:.3e}"
        if i in (0, 31):
            n_got, n_exp = check_detections(got[i], exp, conf=adaptive_threshold(exp))
            assert n_exp >= 10
    print(f"{arch}n b32 640 (branch level {level}): worst max-rel {worst:.3e} over 32 images")


@pytest.mark.timeout(900)
def test_yolov8m_batch64_640():
    cfg = synth.config("m")
    d, w, mc = synth.SCALES["m"]
    params = synth.params(cfg)
    x = synth.images(64, 640, 640, seed=synth.SEED + 64)
    with YoloDetector(cfg, params) as det:
        got, level = bench_forward(det, x)
    for i in (0, 31, 63):
        exp = oracle.yolov8_forward(params, x[i:i + 1], depth=d, width=w, max_channels=mc)[0]
        err = max_rel(got[i], exp)
        print(f"v8m b64 640 (branch level {level}) image {i}: max-rel {err:.3e}")
        assert err <= HEAD_TOL
    assert np.isfinite(got).all()
