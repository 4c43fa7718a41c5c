"""Per-kernel parity: HIP kernels through the C ABI vs the CPU oracle.

Tolerance for convolutions: |got - exp| <= 1e-4 * max(1, |exp|), the
reference's own kernel bar (tests/SimdYolo.Tests/Program.cs:13).  Pooling,
resize, copy and the bins=1 head coordinates are exact.
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import (CONV_DEPTHWISE, CONV_DIRECT, CONV_IGEMM, CONV_WINOGRAD, CONV_WINOGRAD2, CONV_WINOGRAD3,
                          synth)

pytestmark = pytest.mark.gpu

TOL = 1e-4


def near(got, exp, tol=TOL):
    err = np.abs(got.astype(np.float64) - exp) / np.maximum(1.0, np.abs(exp))
    assert np.isfinite(got).all()
    assert err.max() <= tol, f"max rel err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


def wide_view(hip, n, c, h, w, extra_before=4, extra_after=8):
    """A channel slice inside a wider NHWC buffer (offset pointer, ldc > c)."""
    buf = hip.alloc(n, c + extra_before + extra_after, h, w)
    return buf.slice(extra_before, c)


CONV_CASES = [
    # (n, ic, h, w, oc, k, s, algo)
    (2, 16, 20, 20, 16, 3, 1, CONV_WINOGRAD),
    (2, 32, 23, 17, 32, 3, 1, CONV_WINOGRAD),
    (1, 64, 40, 40, 64, 3, 1, CONV_WINOGRAD),
    (2, 128, 20, 20, 128, 3, 1, CONV_WINOGRAD),
    (1, 256, 20, 20, 256, 3, 1, CONV_WINOGRAD),
    (1, 64, 20, 20, 144, 3, 1, CONV_WINOGRAD),
    (2, 12, 13, 9, 20, 3, 1, CONV_WINOGRAD),
    (3, 80, 10, 10, 80, 3, 1, CONV_WINOGRAD),
    (2, 32, 23, 17, 32, 3, 1, CONV_WINOGRAD3),
    (1, 128, 20, 20, 128, 3, 1, CONV_WINOGRAD3),
    (2, 32, 23, 17, 32, 3, 1, CONV_IGEMM),
    (1, 64, 40, 40, 64, 3, 1, CONV_IGEMM),
    (1, 64, 80, 80, 128, 3, 2, CONV_IGEMM),
    (2, 16, 41, 37, 32, 3, 2, CONV_IGEMM),
    (1, 128, 40, 40, 256, 1, 1, CONV_IGEMM),
    (2, 384, 20, 20, 128, 1, 1, CONV_IGEMM),
    (1, 80, 20, 20, 80, 1, 1, CONV_IGEMM),
    (3, 12, 9, 11, 20, 1, 1, CONV_IGEMM),
    (2, 16, 20, 20, 16, 3, 1, CONV_WINOGRAD2),
    (2, 32, 23, 17, 32, 3, 1, CONV_WINOGRAD2),
    (1, 64, 40, 40, 64, 3, 1, CONV_WINOGRAD2),
    (2, 128, 20, 20, 128, 3, 1, CONV_WINOGRAD2),
    (1, 64, 20, 20, 144, 3, 1, CONV_WINOGRAD2),
    (3, 80, 10, 10, 80, 3, 1, CONV_WINOGRAD2),
    (1, 8, 13, 9, 20, 3, 1, CONV_WINOGRAD2),
    (1, 64, 80, 80, 144, 3, 1, CONV_WINOGRAD2),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("silu", [True, False])
def test_conv_parity(hip, case, silu):
    n, ic, h, w, oc, k, s, algo = case
    seed = n * 7919 + ic * 131 + h * 17 + oc + k + s + algo
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, k, k), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    p = k // 2
    exp = oracle.conv2d(x, wt, b, (s, s), (p, p, p, p), silu=silu)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (s, s), (p, p, p, p), silu=silu)
        hip.conv_set_algo(conv, algo)
        assert hip.conv_algo(conv) == algo
        xv = wide_view(hip, n, ic, h, w)
        hip.upload(x, xv)
        yv = wide_view(hip, n, oc, *exp.shape[2:], extra_before=8, extra_after=4)
        hip.conv(conv, xv, yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


@pytest.mark.parametrize("n,ic,h,w,oc", [(1, 64, 80, 80, 64), (2, 16, 13, 7, 8), (1, 32, 40, 40, 20),
                                         (1, 4, 3, 5, 4), (2, 96, 20, 20, 96)])
def test_conv_transpose2x2_parity(hip, n, ic, h, w, oc):
    """nn.ConvTranspose2d(ic, oc, 2, 2, bias) (the Proto upsample) through strided
    views on both sides vs the oracle."""
    seed = n * 31 + ic * 7 + h + w + oc
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((ic, oc, 2, 2), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    exp = oracle.conv_transpose2x2(x, wt, b)
    hip.begin_frame()
    try:
        conv = hip.conv_transpose2x2_create(wt, b)
        assert hip.conv_out_size(conv, h, w) == (2 * h, 2 * w)
        xv = wide_view(hip, n, ic, h, w)
        hip.upload(x, xv)
        yv = wide_view(hip, n, oc, 2 * h, 2 * w, extra_before=8, extra_after=4)
        hip.conv(conv, xv, yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


PW_CASES = [(1, 64, 40, 40, 64, False), (2, 48, 33, 17, 32, True), (1, 80, 20, 20, 80, False),
            (1, 16, 9, 7, 144, True), (2, 192, 20, 20, 64, False), (1, 256, 10, 10, 128, True),
            (1, 96, 5, 61, 256, False), (3, 32, 1, 1, 40, True)]


@pytest.mark.parametrize("nw", [1, 2, 3, 4])
@pytest.mark.parametrize("case", PW_CASES, ids=lambda c: "x".join(map(str, c)))
def test_pointwise_row_kernel_parity(hip, monkeypatch, case, nw):
    """1x1 conv on the weight-stationary row kernel (tile 32 + nw - 1; shapes
    whose weight slab does not fit fall back to the tiled GEMM), strided views,
    optional fused residual."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(32 + nw - 1))
    n, ic, h, w, oc, with_res = case
    seed = n + ic + h + w + oc + nw
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, 1, 1), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    r = synth.activations((n, oc, h, w), seed + 3)
    exp = oracle.conv2d(x, wt, b, (1, 1), (0, 0, 0, 0), silu=True)
    if with_res:
        exp = r + exp
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, silu=True)
        hip.conv_set_algo(conv, CONV_IGEMM)
        xv = wide_view(hip, n, ic, h, w)
        hip.upload(x, xv)
        yv = wide_view(hip, n, oc, h, w, extra_before=8, extra_after=4)
        rv = None
        if with_res:
            rv = wide_view(hip, n, oc, h, w, extra_before=4, extra_after=4)
            hip.upload(r, rv)
        hip.conv(conv, xv, yv, residual=rv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


C16_CASES = [(2, 37, 45, 16, 1, True), (1, 160, 160, 16, 1, False), (2, 41, 37, 32, 2, False),
             (1, 320, 320, 32, 2, False), (1, 9, 7, 32, 1, True), (3, 5, 66, 16, 2, True), (1, 1, 1, 16, 1, False)]


@pytest.mark.parametrize("case", C16_CASES, ids=lambda c: "x".join(map(str, c)))
def test_conv3x3_c16_kernel_parity(hip, monkeypatch, case):
    """3x3 conv with 16 input channels on the 16x16x4 MFMA kernel (tile 40),
    strided views, optional fused residual, stride 1 and 2."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", "40")
    n, h, w, oc, st, with_res = case
    seed = n + h + w + oc + st
    x = synth.activations((n, 16, h, w), seed)
    wt = synth.kaiming((oc, 16, 3, 3), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    exp = oracle.conv2d(x, wt, b, (st, st), (1, 1, 1, 1), silu=True)
    r = synth.activations(exp.shape, seed + 3)
    if with_res:
        exp = r + exp
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (st, st), (1, 1, 1, 1), silu=True)
        hip.conv_set_algo(conv, CONV_IGEMM)
        xv = wide_view(hip, n, 16, h, w)
        hip.upload(x, xv)
        yv = wide_view(hip, n, oc, *exp.shape[2:], extra_before=8, extra_after=4)
        rv = None
        if with_res:
            rv = wide_view(hip, n, oc, *exp.shape[2:], extra_before=4, extra_after=4)
            hip.upload(r, rv)
        hip.conv(conv, xv, yv, residual=rv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


@pytest.mark.parametrize("nw", [1, 2, 4])
@pytest.mark.parametrize("n,c,h,w,oc", [(2, 32, 19, 21, 32), (1, 64, 40, 40, 144), (1, 128, 20, 20, 128)])
def test_winograd_planes_on_row_kernel(hip, monkeypatch, n, c, h, w, oc, nw):
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(32 + nw - 1))
    x = synth.activations((n, c, h, w), c + h)
    wt = synth.kaiming((oc, c, 3, 3), c + w)
    b = synth.activations((oc,), oc) * np.float32(0.1)
    exp = oracle.conv2d(x, wt, b, (1, 1), (1, 1, 1, 1), silu=True)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (1, 1), (1, 1, 1, 1), silu=True)
        hip.conv_set_algo(conv, CONV_WINOGRAD3)
        xv = hip.upload(x)
        yv = hip.alloc(n, oc, h, w)
        hip.conv(conv, xv, yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


SPLIT_CASES = [
    # (n, ic, h, w, oc, k, s, tile, split, residual): im2col modes 1 (tap-aligned K tiles),
    # 0 (general) and 2 (1x1 rows); ragged last K chunk; fused residual through the reduce
    (1, 128, 40, 40, 128, 3, 2, 2, 4, False),
    (1, 128, 40, 40, 256, 3, 2, 11, 8, True),
    (1, 64, 20, 20, 64, 3, 1, 2, 16, True),
    (1, 24, 17, 19, 40, 3, 1, 2, 3, True),
    (2, 384, 20, 20, 256, 1, 1, 3, 4, False),
    (1, 512, 20, 20, 256, 1, 1, 12, 2, True),
    (1, 80, 9, 7, 80, 1, 1, 13, 16, False),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "x".join(map(str, c)))
def test_conv_split_k(hip, monkeypatch, case):
    """Implicit GEMM with K split over workgroups: raw partial tiles in scratch,
    then the reduce applies bias, SiLU and the residual in a fixed order."""
    n, ic, h, w, oc, k, st, tile, split, with_res = case
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(tile))
    monkeypatch.setenv("SIMDYOLO_HIP_SPLIT", str(split))
    seed = n + ic + h + oc + k + split
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, k, k), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    pd = k // 2
    exp = oracle.conv2d(x, wt, b, (st, st), (pd, pd, pd, pd), silu=True)
    r = synth.activations(exp.shape, seed + 3)
    if with_res:
        exp = r + exp
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (st, st), (pd, pd, pd, pd), silu=True)
        hip.conv_set_algo(conv, CONV_IGEMM)
        xv = wide_view(hip, n, ic, h, w)
        hip.upload(x, xv)
        yv = wide_view(hip, n, oc, *exp.shape[2:], extra_before=8, extra_after=4)
        rv = None
        if with_res:
            rv = wide_view(hip, n, oc, *exp.shape[2:], extra_before=4, extra_after=4)
            hip.upload(r, rv)
        hip.conv(conv, xv, yv, residual=rv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


@pytest.mark.parametrize("algo", [CONV_WINOGRAD, CONV_WINOGRAD3, CONV_WINOGRAD2, CONV_IGEMM])
def test_conv_residual_fused(hip, algo):
    # Bottleneck: y = x + SiLU(conv(x) + b)  (PtModel.cs:302-303 order).
    n, c, h, w = 2, 32, 19, 21
    x = synth.activations((n, c, h, w), 5)
    wt = synth.kaiming((c, c, 3, 3), 6)
    b = synth.activations((c,), 7) * np.float32(0.1)
    exp = x + oracle.conv2d(x, wt, b, (1, 1), (1, 1, 1, 1), silu=True)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (1, 1), (1, 1, 1, 1), silu=True)
        hip.conv_set_algo(conv, algo)
        buf = hip.alloc(n, 3 * c, h, w)
        xv, yv = buf.slice(0, c), buf.slice(2 * c, c)
        hip.upload(x, xv)
        hip.conv(conv, xv, yv, residual=xv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


@pytest.mark.parametrize("k", [1, 3])
def test_conv_inplace_residual_autotuned(hip, k):
    """y += SiLU(conv(x) + b) with the residual and the output the same view,
    under automatic algorithm choice: timing candidates must not re-run a conv
    that reads its own output."""
    n, c, h, w = 2, 32, 40, 40
    x = synth.activations((n, c, h, w), 15)
    r = synth.activations((n, c, h, w), 16)
    wt = synth.kaiming((c, c, k, k), 17)
    b = synth.activations((c,), 18) * np.float32(0.1)
    p = k // 2
    exp = r + oracle.conv2d(x, wt, b, (1, 1), (p, p, p, p), silu=True)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (1, 1), (p, p, p, p), silu=True)
        buf = hip.alloc(n, 2 * c, h, w)
        xv, yv = buf.slice(0, c), buf.slice(c, c)
        hip.upload(x, xv)
        hip.upload(r, yv)
        hip.conv(conv, xv, yv, residual=yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


@pytest.mark.parametrize("n,oc,h,w,shift", [(1, 16, 64, 64, 0), (2, 16, 33, 47, 0), (1, 48, 32, 32, 0),
                                            (1, 32, 130, 98, 0), (2, 64, 40, 72, 0), (1, 24, 32, 32, 0),
                                            (2, 16, 36, 64, 1)])
def test_stem_direct_nchw_input(hip, n, oc, h, w, shift):
    """Stem conv on a dense NCHW input: 16-byte patch loads when the row width
    is a multiple of 4 and the base is aligned; per-column loads otherwise
    (odd widths, and a base `shift` floats past an aligned address)."""
    x = synth.images(n, h, w, seed=h)
    wt = synth.kaiming((oc, 3, 3, 3), 9)
    b = synth.activations((oc,), 10) * np.float32(0.1)
    exp = oracle.conv2d(x, wt, b, (2, 2), (1, 1, 1, 1), silu=True)
    from simdyolo_amd._native import LAYOUT_NCHW, Tensor
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (2, 2), (1, 1, 1, 1), silu=True)
        assert hip.conv_algo(conv) == CONV_DIRECT
        raw = hip.alloc(n, 3, h, w + 1) if shift else hip.alloc(n, 3, h, w)
        xv = Tensor(raw.data + 4 * shift, n, 3, h, w, 3, LAYOUT_NCHW)
        hip.upload(x, xv)
        yv = hip.alloc(n, oc, *exp.shape[2:])
        hip.conv(conv, xv, yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    near(got, exp)


def test_conv_shape_mismatch_rejected(hip):
    from simdyolo_amd import SyError
    wt = synth.kaiming((16, 16, 3, 3), 1)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, None, (1, 1), (1, 1, 1, 1))
        xv = hip.alloc(1, 16, 8, 8)
        bad = hip.alloc(1, 16, 7, 8)
        with pytest.raises(SyError) as e:
            hip.conv(conv, xv, bad)
        assert e.value.code == 1
    finally:
        hip.end_frame()


@pytest.mark.parametrize("n,c,h,w", [(1, 128, 20, 20), (2, 8, 37, 29), (1, 64, 40, 40), (3, 16, 7, 5),
                                     (2, 12, 32, 32), (1, 4, 1, 13), (32, 128, 20, 20), (2, 48, 32, 32),
                                     (3, 16, 1, 1), (1, 32, 9, 31), (1, 16, 24, 24), (3, 48, 20, 20),
                                     (1, 24, 20, 20), (32, 256, 20, 20)])
def test_sppf_pool_exact(hip, n, c, h, w):
    x = synth.activations((n, c, h, w), h * w)
    # NaN propagates through every window that holds it (MathF.Max); zeros of
    # both signs tie.
    x.reshape(-1)[:: 97] = np.nan
    x.reshape(-1)[5:: 89] = 0.0
    x.reshape(-1)[7:: 89] = -0.0
    p1 = oracle.maxpool(x, (5, 5), (1, 1), (2, 2, 2, 2))
    p2 = oracle.maxpool(p1, (5, 5), (1, 1), (2, 2, 2, 2))
    p3 = oracle.maxpool(p2, (5, 5), (1, 1), (2, 2, 2, 2))
    hip.begin_frame()
    try:
        buf = hip.alloc(n, 4 * c, h, w)
        xs = [buf.slice(i * c, c) for i in range(4)]
        hip.upload(x, xs[0])
        hip.sppf_pool(*xs)
        got = [hip.download(v) for v in xs[1:]]
    finally:
        hip.end_frame()
    for g, e in zip(got, (p1, p2, p3)):
        np.testing.assert_array_equal(g, e)


@pytest.mark.parametrize("passes", [1, 3])
def test_pool5_20x20_register_kernel_any_view(hip, passes):
    """20x20 planes with whole 16-channel groups run the register kernel,
    which reads and writes single floats: channel slices at odd offsets in
    buffers of odd pixel stride, with ties, infinities and NaN in the input,
    against the oracle's chained clipped 5x5 pools."""
    n, c = 2, 32
    x = synth.activations((n, c, 20, 20), 4401)
    x[:, :, 3:9, 4:12] = np.round(x[:, :, 3:9, 4:12])   # ties
    x[0, 1, 0, 0] = np.inf
    x[1, 2, 19, 19] = -np.inf
    x[0, 3, 10, 7] = np.nan
    x[1, 5, :, :2] = np.nan                               # a window of NaN at the left edge
    exp = [x]
    for _ in range(passes):
        exp.append(oracle.maxpool(exp[-1], (5, 5), (1, 1), (2, 2, 2, 2)))
    hip.begin_frame()
    try:
        xv = hip.alloc(n, c + 5, 20, 20).slice(3, c)
        ys = [hip.alloc(n, c + 3, 20, 20).slice(1, c) for _ in range(3)]
        hip.upload(x, xv)
        names = set()
        hip.profile_enable(True)
        try:
            hip.profile_read()
            if passes == 3:
                hip.sppf_pool(xv, *ys)
            else:
                hip.maxpool(xv, ys[0], (5, 5), (1, 1), (2, 2, 2, 2))
            hip.flush()
            names = set(hip.profile_read())
        finally:
            hip.profile_enable(False)
        got = [hip.download(v) for v in ys[:passes]]
    finally:
        hip.end_frame()
    if passes == 3:
        assert "sppf_rows20" in names, sorted(names)
    for g, e in zip(got, exp[1:]):
        np.testing.assert_array_equal(g, e)


@pytest.mark.parametrize("stride", [1, 2])
def test_maxpool_generic_exact(hip, stride):
    x = np.sin(np.arange(2 * 3 * 9 * 13, dtype=np.float32)).reshape(2, 3, 9, 13).astype(np.float32)
    x.reshape(-1)[::41] = np.nan
    exp = oracle.maxpool(x, (5, 3), (stride, stride), (2, 1, 2, 1))
    hip.begin_frame()
    try:
        xv = hip.upload(x)
        yv = hip.alloc(*exp.shape)
        hip.maxpool(xv, yv, (5, 3), (stride, stride), (2, 1, 2, 1))
        got = hip.download(yv)
    finally:
        hip.end_frame()
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("c,k,st,pads,ceil", [(8, (5, 3), 1, (2, 1, 2, 1), False), (64, (5, 5), 1, (2, 2, 2, 2), False),
                                             (12, (3, 3), 2, (0, 1, 1, 0), True), (256, (2, 2), 2, (0, 0, 0, 0), False)])
def test_maxpool_vec4_exact(hip, c, k, st, pads, ceil):
    """Four-channel maxpool kernel on strided channel-slice views (16-byte aligned)."""
    x = synth.activations((2, c, 11, 13), c + st)
    x.reshape(-1)[::53] = np.nan
    exp = oracle.maxpool(x, k, (st, st), pads, ceil_mode=ceil)
    hip.begin_frame()
    try:
        xv = wide_view(hip, 2, c, 11, 13)
        hip.upload(x, xv)
        yv = wide_view(hip, *exp.shape, extra_before=8, extra_after=4)
        hip.maxpool(xv, yv, k, (st, st), pads, ceil_mode=ceil)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("h,w,k,st,pads,oh,ow", [(4, 34, 3, 2, (0, 0, 0, 0), 2, 17), (5, 33, 2, 2, (1, 1, 1, 1), 3, 17),
                                               (2, 35, 3, 2, (0, 0, 0, 0), 1, 17), (4, 36, 3, 2, (0, 1, 1, 0), 2, 18)])
def test_maxpool_ceil_mode_reference_cases(hip, h, w, k, st, pads, oh, ow):
    """MaxPoolCeilTests.cs:13-19: ceil mode keeps partial windows and drops
    windows that would start in padding; all-negative inputs show any padding
    value that leaked in.  Pads are (top, left, bottom, right)."""
    for frame in range(3):
        x = (-1.0 - ((np.arange(2 * 2 * h * w) * 73 + frame * 29) % 257)).astype(np.float32).reshape(2, 2, h, w)
        exp = oracle.maxpool(x, (k, k), (st, st), pads, ceil_mode=True)
        assert exp.shape == (2, 2, oh, ow)
        hip.begin_frame()
        try:
            xv = hip.upload(x)
            yv = hip.alloc(2, 2, oh, ow)
            hip.maxpool(xv, yv, (k, k), (st, st), pads, ceil_mode=True)
            got = hip.download(yv)
        finally:
            hip.end_frame()
        np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("c", [3, 64])
def test_resize_add_copy_exact(hip, c):
    x = synth.activations((2, c, 7, 5), 3)
    y = synth.activations((2, c, 7, 5), 4)
    up = oracle.resize_nearest(x, 14, 10)
    odd = oracle.resize_nearest(x, 4, 8)
    hip.begin_frame()
    try:
        xv, yv = hip.upload(x), hip.upload(y)
        u = wide_view(hip, 2, c, 14, 10)
        hip.resize_nearest(xv, u)
        o = hip.alloc(2, c, 4, 8)
        hip.resize_nearest(xv, o)
        s = hip.alloc(2, c, 7, 5)
        hip.add(xv, yv, s)
        cp = wide_view(hip, 2, c, 7, 5)
        hip.copy(xv, cp)
        got = [hip.download(t) for t in (u, o, s, cp)]
    finally:
        hip.end_frame()
    np.testing.assert_array_equal(got[0], up)
    np.testing.assert_array_equal(got[1], odd)
    np.testing.assert_array_equal(got[2], x + y)
    np.testing.assert_array_equal(got[3], x)


@pytest.mark.parametrize("bins,xyxy", [(16, False), (16, True), (1, False), (1, True)])
def test_detect_decode(hip, bins, xyxy):
    nc, batch = 80, 2
    shapes = [(12, 16), (6, 8), (3, 4)]
    strides = [8.0, 16.0, 32.0]
    levels = []
    for i, (h, w) in enumerate(shapes):
        raw = synth.activations((batch, 4 * bins + nc, h, w), 40 + i) * np.float32(3)
        levels.append(raw)
    exp = oracle.detect_decode([(r[:, :4 * bins], r[:, 4 * bins:], s) for r, s in zip(levels, strides)], bins, xyxy)
    total = exp.shape[2]
    hip.begin_frame()
    try:
        views = [hip.upload(r) for r in levels]
        out = hip.alloc(batch, nc + 4, 1, total)  # dense [B, nc+4, total] storage
        hip.detect_decode(views, strides, bins, nc, xyxy, out.data, total)
        hip.flush()
        got = hip.d2h(out.data, exp.shape)
    finally:
        hip.end_frame()
    if bins == 1:
        np.testing.assert_array_equal(got[:, :4], exp[:, :4])
    else:
        near(got[:, :4], exp[:, :4], 2e-5)
    near(got[:, 4:], exp[:, 4:], 1e-6)


def test_graph_replay_matches_eager(hip):
    x = synth.activations((2, 32, 20, 20), 77)
    wt = synth.kaiming((32, 32, 3, 3), 78)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, None, (1, 1), (1, 1, 1, 1), silu=True)
        xv = hip.upload(x)
        eager = hip.alloc(2, 32, 20, 20)
        hip.conv(conv, xv, eager)
        ref = hip.download(eager)
        yv = hip.alloc(2, 32, 20, 20)
        hip.graph_begin()
        hip.conv(conv, xv, yv)
        g = hip.graph_end()
        for _ in range(3):
            hip.graph_launch(g)
            hip.flush()
            np.testing.assert_array_equal(hip.download(yv), ref)
    finally:
        hip.end_frame()


DW_CASES = [
    # (n, c, h, w, k, s): DWConv of the YOLO11 class branch and C2PSA's pe
    (2, 64, 20, 20, 3, 1),
    (1, 80, 40, 40, 3, 1),
    (2, 30, 11, 13, 3, 1),  # c % 4 != 0: scalar path
    (1, 32, 21, 19, 3, 2),
    (1, 16, 9, 9, 5, 1),
    (1, 64, 7, 6, 3, 2),    # fewer output columns than a 4-column strip
    (3, 16, 1, 1, 3, 1),
    (1, 128, 13, 9, 3, 1),
    (2, 8, 80, 80, 3, 2),
    (2, 256, 20, 20, 3, 1),   # YOLO11n shapes: 32-channel blocks, 20-column tiles
    (1, 96, 41, 35, 3, 1),    # rows and columns past the last tile
]


# SIMDYOLO_HIP_TILE value of each 3x3 depthwise kernel, and the profile name
# it runs under (stride 2 and 16-byte-misaligned views: register / generic).
DW_KERNELS = {"register": "0", "tile": "1", "column4": "2", "column8": "3"}


def _dw_expected(kernel, c, w, s, aligned=True):
    if not aligned or c % 4:
        return "depthwise_conv"
    if s == 2 or kernel == "register":
        return f"depthwise_reg_s{s}"
    if kernel == "tile":
        return "depthwise_tile20" if w % 20 == 0 else "depthwise_tile32"
    return "depthwise_col4" if kernel == "column4" else "depthwise_col8"


def _aligned16(*views):
    return all(v.data % 16 == 0 and v.ldc % 4 == 0 for v in views)


def _dw_run(hip, conv, xv, yv, rv=None):
    """One depthwise conv with the algorithm pinned (no autotuning, so
    SIMDYOLO_HIP_TILE picks the kernel); returns the profile names seen."""
    hip.conv_set_algo(conv, CONV_DEPTHWISE)
    hip.profile_enable(True)
    try:
        hip.profile_read()
        hip.conv(conv, xv, yv, rv) if rv is not None else hip.conv(conv, xv, yv)
        hip.flush()
        return set(hip.profile_read())
    finally:
        hip.profile_enable(False)


@pytest.mark.parametrize("case", DW_CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("silu", [True, False])
@pytest.mark.parametrize("kernel", list(DW_KERNELS))
def test_depthwise_parity(hip, monkeypatch, case, silu, kernel):
    """3x3 stride-1 aligned views run the kernel SIMDYOLO_HIP_TILE pins: the
    register kernel (0), the LDS-tile kernel (1) or the column kernel with
    4- or 8-row segments (2, 3); other cases the generic one."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", DW_KERNELS[kernel])
    n, c, h, w, k, s = case
    seed = 4001 + n * 31 + c * 7 + h + k + s
    x = synth.activations((n, c, h, w), seed)
    wt = synth.kaiming((c, 1, k, k), seed + 1)
    b = synth.activations((c,), seed + 2) * np.float32(0.1)
    p = k // 2
    exp = oracle.conv2d(x, wt, b, (s, s), (p, p, p, p), groups=c, silu=silu)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (s, s), (p, p, p, p), groups=c, silu=silu)
        assert hip.conv_algo(conv) == CONV_DEPTHWISE
        xv = wide_view(hip, n, c, h, w)
        hip.upload(x, xv)
        yv = wide_view(hip, n, c, *exp.shape[2:], extra_before=8, extra_after=4)
        names = _dw_run(hip, conv, xv, yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    want = _dw_expected(kernel, c, exp.shape[3], s, aligned=_aligned16(xv, yv)) if k == 3 else "depthwise_conv"
    assert want in names, f"expected {want}, profile saw {sorted(names)}"
    near(got, exp)


@pytest.mark.parametrize("kernel", list(DW_KERNELS))
@pytest.mark.parametrize("h,w", [(20, 20), (13, 11)])
def test_depthwise_residual_fused(hip, monkeypatch, kernel, h, w):
    # C2PSA's pe: y = o + pe(v), pe = depthwise 3x3 without activation.
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", DW_KERNELS[kernel])
    n, c = 2, 64
    v = synth.activations((n, c, h, w), 4101)
    o = synth.activations((n, c, h, w), 4102)
    wt = synth.kaiming((c, 1, 3, 3), 4103)
    b = synth.activations((c,), 4104) * np.float32(0.1)
    exp = oracle.conv2d(v, wt, b, (1, 1), (1, 1, 1, 1), groups=c) + o
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (1, 1), (1, 1, 1, 1), groups=c)
        vv, ov, yv = wide_view(hip, n, c, h, w), wide_view(hip, n, c, h, w), hip.alloc(n, c, h, w)
        hip.upload(v, vv)
        hip.upload(o, ov)
        names = _dw_run(hip, conv, vv, yv, ov)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    want = _dw_expected(kernel, c, w, 1, aligned=_aligned16(vv, yv, ov))
    assert want in names, f"expected {want}, profile saw {sorted(names)}"
    near(got, exp)


def _attention_ref(qkv, heads, kd, hd, scale):
    """PSA Attention core in float64: qkv viewed [B, heads, 2kd+hd, N]."""
    b, _, h, w = qkv.shape
    n = h * w
    t = qkv.astype(np.float64).reshape(b, heads, 2 * kd + hd, n)
    q, k, v = t[:, :, :kd], t[:, :, kd:2 * kd], t[:, :, 2 * kd:]
    s = np.matmul(q.transpose(0, 1, 3, 2), k) * float(scale)
    s = np.exp(s - s.max(-1, keepdims=True))
    s /= s.sum(-1, keepdims=True)
    o = np.matmul(v, s.transpose(0, 1, 3, 2))
    return o.reshape(b, heads * hd, h, w), v.reshape(b, heads * hd, h, w)


ATTN_CASES = [
    # (batch, heads, key_dim, head_dim, h, w)
    (1, 2, 32, 64, 20, 20),   # YOLO11n C2PSA at 640x640
    (2, 1, 16, 32, 7, 9),     # N = 63: padded rows
    (2, 4, 32, 64, 4, 4),     # YOLO11m-like heads at 128x128
    (1, 2, 32, 64, 40, 40),   # 1280x1280 input
    (1, 2, 16, 20, 13, 13),   # N = 169 (K = 172, a ragged last chunk), head dim 20 (a ragged column tile)
]


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: "x".join(map(str, c)))
def test_attention_parity(hip, case):
    b, heads, kd, hd, h, w = case
    per = 2 * kd + hd
    qkv = synth.activations((b, heads * per, h, w), 4200 + h * w + heads)
    scale = np.float32(1.0) / np.sqrt(np.float32(kd))
    o_exp, v_exp = _attention_ref(qkv, heads, kd, hd, scale)
    hip.begin_frame()
    try:
        qv = wide_view(hip, b, heads * per, h, w)
        hip.upload(qkv, qv)
        ov = wide_view(hip, b, heads * hd, h, w, extra_before=8, extra_after=0)
        vv = hip.alloc(b, heads * hd, h, w)
        hip.attention(qv, heads, kd, hd, float(scale), ov, vv)
        o, v = hip.download(ov), hip.download(vv)
    finally:
        hip.end_frame()
    np.testing.assert_array_equal(v, v_exp.astype(np.float32))
    near(o, o_exp)
