"""Pins the CPU baseline (oracle/cpu_fast.c), the restatement of the
reference's FP32 CPU convolution algorithms that bench.py times beside the
GPU numbers, before its figures are reported.

  * Routing: the Winograd F(4,3) / F(2,3) / implicit-GEMM choice per shape,
    restated from TensorOps.Conv (src/SimdYolo/Compute.cs:185-188) and
    CpuWinograd4.AdditionalHotShape (src/SimdYolo/CpuWinograd4.cs:28-32),
    checked against rules read off those lines (a mistaken bound flips a
    case).
  * Arithmetic: every route against the oracle's double-accumulating direct
    convolution at the reference's Winograd bar, 1e-4 relative
    (tests/SimdYolo.Tests/CpuWinogradPanelTests.cs:120), with inputs and
    weights scaled as there (0.1 and 0.3) on odd shapes with ragged tiles.
  * The whole YOLOv8n forward against the oracle's, within the 1e-3 head bar.
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import synth

F4, F2, IMPL, DW = oracle.CF_WINOGRAD4, oracle.CF_WINOGRAD2, oracle.CF_IMPLICIT, oracle.CF_DEPTHWISE


@pytest.mark.parametrize("ic,oc,hw,k,s,groups,expect", [
    (32, 32, 80, 3, 1, 1, F4),     # 32 <= ic <= 64, 32 <= oc <= 128, <= 160
    (64, 128, 160, 3, 1, 1, F4),
    (64, 144, 80, 3, 1, 1, F4),    # oc > 128: AdditionalHotShape (oc > 128)
    (16, 16, 160, 3, 1, 1, F2),    # ic < 32
    (128, 128, 20, 3, 1, 1, F4),   # AdditionalHotShape: ic >= 80, h >= 20
    (128, 128, 10, 3, 1, 1, F2),   # h < 20
    (256, 256, 20, 3, 1, 1, F4),   # ic + oc == 512
    (256, 320, 20, 3, 1, 1, F2),   # ic + oc > 512
    (64, 64, 200, 3, 1, 1, F2),    # h > 160
    (80, 80, 80, 3, 1, 1, F4),
    (8, 8, 16, 3, 1, 1, F2),       # ic >= 8, oc >= 8, oh*ow >= 64
    (8, 8, 7, 3, 1, 1, IMPL),      # oh*ow = 49 < 64
    (4, 8, 32, 3, 1, 1, IMPL),     # ic < 8
    (64, 128, 80, 3, 2, 1, IMPL),  # stride 2
    (128, 256, 40, 1, 1, 1, IMPL), # 1x1
    (64, 64, 20, 3, 1, 64, DW),    # depthwise
])
def test_routing(ic, oc, hw, k, s, groups, expect):
    x = np.zeros((1, ic, hw, hw), np.float32)
    w = np.zeros((oc, ic // groups, k, k), np.float32)
    _, alg = oracle.cpu_fast_conv(x, w, stride=s, groups=groups)
    assert alg == expect


@pytest.mark.parametrize("n,ic,h,w,oc,k,s,groups", [
    (2, 32, 23, 17, 40, 3, 1, 1),   # F(4,3), ragged tiles
    (1, 64, 41, 37, 144, 3, 1, 1),  # F(4,3) via AdditionalHotShape
    (2, 16, 19, 21, 24, 3, 1, 1),   # F(2,3)
    (1, 8, 9, 11, 12, 3, 1, 1),     # F(2,3), odd
    (2, 24, 17, 13, 40, 3, 2, 1),   # implicit, stride 2
    (1, 3, 33, 35, 16, 3, 2, 1),    # stem-like, ic = 3
    (2, 40, 13, 11, 72, 1, 1, 1),   # 1x1
    (1, 32, 15, 9, 32, 3, 1, 32),   # depthwise
    (1, 16, 10, 10, 16, 3, 2, 16),  # depthwise stride 2
])
@pytest.mark.parametrize("silu", [False, True])
def test_conv_matches_oracle(n, ic, h, w, oc, k, s, groups, silu):
    rng = np.random.Generator(np.random.PCG64(n * 1000 + ic * 10 + oc + k + s))
    x = (rng.standard_normal((n, ic, h, w)) * 0.1).astype(np.float32)
    wt = (rng.standard_normal((oc, ic // groups, k, k)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(oc) * 0.7).astype(np.float32)
    p = k // 2
    exp = oracle.conv2d(x, wt, b, (s, s), (p, p, p, p), groups=groups, silu=silu)
    got, _ = oracle.cpu_fast_conv(x, wt, b, stride=s, groups=groups, silu=silu)
    err = np.abs(got.astype(np.float64) - exp) / np.maximum(1.0, np.abs(exp))
    assert err.max() <= 1e-4, err.max()


def test_yolov8n_forward_matches_oracle():
    cfg = synth.config("n")
    params = synth.params(cfg)
    x = synth.images(2, 320, 320, seed=3)
    fast = oracle.FastYolov8(params)
    try:
        got = fast.forward(x)
        again = fast.forward(x)  # planned weights and pooled buffers reused
    finally:
        fast.close()
    exp = oracle.yolov8_forward(params, x)
    err = np.abs(got.astype(np.float64) - exp) / np.maximum(1.0, np.abs(exp))
    assert err.max() <= 1e-3, err.max()
    np.testing.assert_array_equal(got, again)
