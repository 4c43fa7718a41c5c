"""Every GEMM instantiation the autotuner can pick, forced one at a time, and
the per-layer microbench shapes at batch 1 and 32, against the oracle.

The tuner times all candidates and keeps the fastest per shape, so the
whole-network runs execute tiles that a size heuristic never picks.  Here each
of the 22 implicit-GEMM tiles runs in each A-row addressing mode (general
im2col, tap-aligned K tiles, plain 1x1 rows) and as the Winograd plane GEMM,
with and without split K and a fused residual, on ragged M, N and K.  The
profile name of the launch shows which instantiation ran.

The 3x3 s1 layer shapes of the per-layer microbench (C in {32, 64, 128, 256}
at 160, 80, 40, 20 pixels square) run through each Winograd form and through
the autotuned choice at batch 1 and 32.  At batch 32 the oracle checks images
0, 1 and 31; images 1..30 are the same picture, so their outputs must be
bit-identical (rows of the GEMMs do not interact).

Tolerance: |got - exp| <= 1e-4 * max(1, |exp|) (tests/SimdYolo.Tests/
Program.cs:13, the reference's kernel bar), except the Winograd forms at 256
channels: 2e-4.  F(4x4,3x3) in FP32 with the Lavin-Gray matrices the
reference uses (src/SimdYolo/CpuWinograd4.cs:36) amplifies the rounding of
the 36 plane products by up to 64 at output point (3, 3), and the plane sums
run over K = 256 channels.  A float32 emulation of the same transforms in the
same separable order, with a float32 BLAS product, reaches max-rel 0.89e-4
and 0.82e-4 on images 1 and 31 of the 256-channel 160x160 case, so 1e-4 sits
at the algorithm's own rounding there.  The reference checks its Winograd
paths at 1e-4 only at ic <= 80 with inputs and weights scaled by 0.1 and 0.3
(tests/SimdYolo.Tests/CpuWinogradPanelTests.cs:17-24).
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import CONV_IGEMM, CONV_WINOGRAD, CONV_WINOGRAD2, CONV_WINOGRAD3, synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
TOL_WINO_256 = 2e-4
# (bm, bn, wm, wn, bk, prefetch depth) of tiles 0..21, in the library's order.
TILES = [(128, 128, 2, 2, 16, 1), (128, 64, 2, 2, 16, 1), (64, 64, 2, 2, 16, 1), (128, 32, 4, 1, 16, 1),
         (64, 32, 2, 1, 16, 1), (256, 64, 4, 1, 16, 1), (128, 64, 2, 1, 16, 1), (128, 64, 2, 2, 32, 1),
         (128, 128, 2, 2, 32, 1), (256, 32, 4, 1, 16, 1), (256, 128, 4, 2, 16, 1), (64, 64, 2, 2, 32, 1),
         (128, 32, 4, 1, 32, 1), (64, 32, 2, 1, 32, 1), (64, 64, 2, 2, 32, 2), (128, 64, 2, 2, 32, 2),
         (64, 64, 2, 2, 16, 2), (128, 32, 4, 1, 16, 2), (256, 64, 4, 1, 16, 2), (128, 128, 2, 2, 16, 2),
         (64, 32, 2, 1, 32, 2), (128, 32, 4, 1, 32, 2), (64, 96, 2, 3, 16, 2), (64, 96, 2, 3, 32, 1)]


def near(got, exp, tol=TOL):
    err = np.abs(got.astype(np.float64) - exp) / np.maximum(1.0, np.abs(exp))
    assert np.isfinite(got).all()
    assert err.max() <= tol, f"max rel err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


def tile_name(t, kind, mode):
    bm, bn, wm, wn, bk, pf = TILES[t]
    suffix = f"_p{pf}" if pf > 1 else ""
    if kind == "wino":
        return f"wino_gemm_{bm}x{bn}_{wm}{wn}_k{bk}{suffix}"
    return f"igemm_m{mode}_{bm}x{bn}_{wm}{wn}_k{bk}{suffix}"


# (n, ic, h, w, oc, k, s): ragged M (pixels), N (oc) and K against every tile.
FORMS = {
    "rows1x1": (2, 40, 13, 11, 72, 1, 1),     # mode 2: K = 40, M = 286, N = 72
    "tap3x3s2": (1, 64, 19, 21, 40, 3, 2),    # mode 1: IC % BK == 0 for BK 16 and 32
    "im2col3x3": (2, 20, 11, 9, 24, 3, 1),    # mode 0: IC = 20 is no multiple of a K tile
    "winoplanes": (2, 48, 17, 15, 40, 3, 1),  # Winograd plane GEMM: K = 48, 40 tiles per plane
    # odd and single K-tile counts for the two-deep prefetch's unrolled loop
    "rows1x1_k72": (2, 72, 9, 7, 40, 1, 1),   # K = 72: 3 tiles of 32 (ragged), 5 of 16
    "rows1x1_k24": (1, 24, 7, 9, 24, 1, 1),   # K = 24: one tile of 32, two of 16
    "tap3x3s2_ic32": (1, 32, 15, 17, 72, 3, 2),  # K = 288: 9 tiles of 32, 18 of 16
}


def _mode(form, t):
    n, ic, h, w, oc, k, s = FORMS[form]
    if k == 1:
        return 2
    return 1 if ic % TILES[t][4] == 0 else 0


def _run_conv(hip, x, wt, b, stride, pad, algo, res=None, profile=False):
    n, ic, h, w = x.shape
    oc = wt.shape[0]
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (stride, stride), (pad, pad, pad, pad), silu=True)
        hip.conv_set_algo(conv, algo)
        oh, ow = hip.conv_out_size(conv, h, w)
        buf = hip.alloc(n, ic + 4, h, w)
        xv = buf.slice(4, ic)  # a channel slice of a wider buffer, as the model's views
        hip.upload(x, xv)
        ybuf = hip.alloc(n, oc + 12, oh, ow)
        yv = ybuf.slice(8, oc)
        rv = None
        if res is not None:
            rbuf = hip.alloc(n, oc + 8, oh, ow)
            rv = rbuf.slice(4, oc)
            hip.upload(res, rv)
        if profile:
            hip.profile_enable(True)
        hip.conv(conv, xv, yv, residual=rv)
        names = None
        if profile:
            hip.flush()
            names = set(hip.profile_read())
            hip.profile_enable(False)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    return got, names


@pytest.mark.parametrize("res", [False, True], ids=["plain", "res"])
@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("tile", range(len(TILES)))
def test_forced_tile(hip, monkeypatch, tile, form, res):
    """One GEMM instantiation forced through SIMDYOLO_HIP_TILE, checked
    against the oracle, and identified by its profile name."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(tile))
    n, ic, h, w, oc, k, s = FORMS[form]
    seed = 9000 + tile * 31 + len(form) + (7 if res else 0)
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, k, k), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    p = k // 2
    exp = oracle.conv2d(x, wt, b, (s, s), (p, p, p, p), silu=True)
    r = synth.activations(exp.shape, seed + 3) if res else None
    if res:
        exp = r + exp
    algo = CONV_WINOGRAD3 if form == "winoplanes" else CONV_IGEMM
    got, names = _run_conv(hip, x, wt, b, s, p, algo, r, profile=True)
    kind = "wino" if form == "winoplanes" else "conv"
    want = tile_name(tile, kind, _mode(form, tile))
    assert want in names, f"expected {want} to run, profile saw {sorted(names)}"
    near(got, exp)


# (tile, split, form): split K over 2-16 workgroups per output tile, every
# addressing mode, ragged last K chunk, residual through the reduce.
SPLITS = [(t, sp, f) for t in range(len(TILES)) for sp, f in ((2, "tap3x3s2"), (3, "im2col3x3"), (4, "rows1x1"))]


@pytest.mark.parametrize("tile,split,form", SPLITS, ids=lambda v: str(v))
def test_forced_tile_split_k(hip, monkeypatch, tile, split, form):
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(tile))
    monkeypatch.setenv("SIMDYOLO_HIP_SPLIT", str(split))
    n, ic, h, w, oc, k, s = FORMS[form]
    n = 1  # split K runs at batch 1
    seed = 9500 + tile * 13 + split
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, k, k), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    p = k // 2
    exp = oracle.conv2d(x, wt, b, (s, s), (p, p, p, p), silu=True)
    r = synth.activations(exp.shape, seed + 3)
    exp = r + exp
    got, names = _run_conv(hip, x, wt, b, s, p, CONV_IGEMM, r, profile=True)
    want = tile_name(tile, "conv", _mode(form, tile))
    assert any(nm.startswith(want + "_sk") for nm in names), f"no split-K {want} in {sorted(names)}"
    assert "splitk_reduce" in names
    near(got, exp)


KS_FORMS = {  # (ic, h, w, oc, k, s, mode, bk)
    "tap3x3s2": (64, 19, 21, 40, 3, 2, 1, 32),   # whole 32-deep chunks per tap
    "tap3x3_ic48": (48, 13, 11, 72, 3, 1, 1, 16),  # 16-deep chunks
    "rows1x1": (40, 13, 11, 72, 1, 1, 2, 32),     # K = 40: a ragged last chunk
    "rows1x1_deep": (512, 20, 20, 256, 1, 1, 2, 32),
}


@pytest.mark.parametrize("res", [False, True], ids=["plain", "res"])
@pytest.mark.parametrize("form", list(KS_FORMS))
@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("t16", [False, True], ids=["t32", "t16"])
def test_forced_in_workgroup_split_k(hip, monkeypatch, waves, form, res, t16):
    """The in-workgroup split-K kernels (one 32x32 tile per workgroup on
    32x32x2 MFMAs, or one 16x16 tile on 16x16x4 MFMAs with up to four K chunks
    per load round trip; the K chunks shared out over 4, 8 or 16 waves,
    partials summed in LDS) at batch 1, forced through SIMDYOLO_HIP_TILE,
    against the oracle."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str((52 if t16 else 48) + {4: 0, 8: 1, 16: 2}[waves]))
    ic, h, w, oc, k, s, mode, bk = KS_FORMS[form]
    seed = 9900 + waves + len(form) + (5 if res else 0)
    x = synth.activations((1, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, k, k), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    p = k // 2
    exp = oracle.conv2d(x, wt, b, (s, s), (p, p, p, p), silu=True)
    r = synth.activations(exp.shape, seed + 3) if res else None
    if res:
        exp = r + exp
    got, names = _run_conv(hip, x, wt, b, s, p, CONV_IGEMM, r, profile=True)
    want = f"igemm_ks{waves}_t16_m{mode}_k{bk}" if t16 else f"igemm_ks{waves}_m{mode}_k{bk}"
    assert want in names, f"expected {want} to run, profile saw {sorted(names)}"
    near(got, exp)


@pytest.mark.parametrize("form", ["tap3x3s2", "rows1x1"])
def test_split_k_repeats_and_replays(hip, monkeypatch, form):
    """Split K with its reduce: three eager runs on new inputs, then a captured
    graph replayed three times with new inputs uploaded between the replays,
    each against the oracle."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", "2")
    monkeypatch.setenv("SIMDYOLO_HIP_SPLIT", "4")
    n, ic, h, w, oc, k, s = FORMS[form]
    n = 1
    wt = synth.kaiming((oc, ic, k, k), 9700)
    b = synth.activations((oc,), 9701) * np.float32(0.1)
    p = k // 2
    xs = [synth.activations((n, ic, h, w), 9710 + i) for i in range(6)]
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (s, s), (p, p, p, p), silu=True)
        hip.conv_set_algo(conv, CONV_IGEMM)
        oh, ow = hip.conv_out_size(conv, h, w)
        xv = hip.alloc(n, ic, h, w)
        yv = hip.alloc(n, oc, oh, ow)
        for i in range(3):
            print(f"split-K {form}: eager run {i}", flush=True)
            hip.upload(xs[i], xv)
            hip.conv(conv, xv, yv)
            near(hip.download(yv), oracle.conv2d(xs[i], wt, b, (s, s), (p, p, p, p), silu=True))
        hip.graph_begin()
        hip.conv(conv, xv, yv)
        g = hip.graph_end()
        for i in range(3, 6):
            print(f"split-K {form}: graph replay {i - 3}", flush=True)
            hip.upload(xs[i], xv)
            hip.graph_launch(g)
            hip.flush()
            near(hip.download(yv), oracle.conv2d(xs[i], wt, b, (s, s), (p, p, p, p), silu=True))
    finally:
        hip.end_frame()


# ---------------------------------------------------------------- layer shapes

SHAPES = [(c, hw) for c in (32, 64, 128, 256) for hw in (160, 80, 40, 20)]
_cache = {}


def _shape_data(c, hw):
    """Images 0, 1 and 31 of a batch-32 input (1..30 are the same picture),
    the weights, and the oracle's output for those three images."""
    key = (c, hw)
    if key not in _cache:
        seed = 7000 + c + hw
        imgs = synth.activations((3, c, hw, hw), seed)
        wt = synth.kaiming((c, c, 3, 3), seed + 1)
        b = synth.activations((c,), seed + 2) * np.float32(0.1)
        exp = oracle.conv2d(imgs, wt, b, (1, 1), (1, 1, 1, 1), silu=True)
        _cache.clear()
        _cache[key] = (imgs, wt, b, exp)
    return _cache[key]


@pytest.mark.parametrize("algo", [CONV_WINOGRAD3, CONV_WINOGRAD2, -CONV_WINOGRAD2, CONV_WINOGRAD, 0],
                         ids=["wino3", "wino2", "wino2w8", "winofused", "autotuned"])
@pytest.mark.parametrize("batch", [1, 32])
@pytest.mark.parametrize("c,hw", SHAPES, ids=lambda v: str(v))
def test_layer_shape_winograd(hip, monkeypatch, c, hw, batch, algo):
    """Each Winograd form on the microbench shapes; wino2w8 is the planes +
    inverse kernel with four helper waves in the inverse transform."""
    if algo < 0:
        monkeypatch.setenv("SIMDYOLO_HIP_TILE", "1")
        algo = -algo
    imgs, wt, b, exp = _shape_data(c, hw)
    if batch == 1:
        x, want = imgs[:1], {0: exp[0]}
    else:
        x = np.concatenate([imgs[:1], np.repeat(imgs[1:2], 30, axis=0), imgs[2:3]])
        want = {0: exp[0], 1: exp[1], 31: exp[2]}
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (1, 1), (1, 1, 1, 1), silu=True)
        if algo:
            hip.conv_set_algo(conv, algo)
        xv = hip.upload(x)
        yv = hip.alloc(batch, c, hw, hw)
        hip.conv(conv, xv, yv)  # autotuned: times the candidates, then runs the pick
        if not algo:
            hip.conv(conv, xv, yv)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    for i, e in want.items():
        near(got[i], e, TOL if c < 256 else TOL_WINO_256)
    if batch == 32:
        for i in range(2, 31):
            np.testing.assert_array_equal(got[i], got[1])


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("n,ic,h,w,oc,res", [(2, 32, 23, 17, 32, True), (1, 64, 20, 20, 96, False),
                                             (3, 80, 10, 10, 80, True), (1, 64, 40, 40, 144, True),
                                             (2, 128, 13, 19, 160, False), (1, 8, 9, 7, 20, False)])
def test_wino_planes_inverse(hip, monkeypatch, n, ic, h, w, oc, res, waves):
    """Planes + inverse kernel in both wave layouts (four MFMA waves alone, or
    with four helper waves in the inverse transform): odd 32-channel block
    counts, one K chunk (ic = 8), ragged tiles, fused residual, strided
    views."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", "1" if waves == 8 else "0")
    seed = 9900 + n + ic + h + oc
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, 3, 3), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    exp = oracle.conv2d(x, wt, b, (1, 1), (1, 1, 1, 1), silu=True)
    r = synth.activations(exp.shape, seed + 3) if res else None
    if res:
        exp = r + exp
    got, names = _run_conv(hip, x, wt, b, 1, 1, CONV_WINOGRAD2, r, profile=True)
    assert ("wino_gemm_out_w8" if waves == 8 else "wino_gemm_out") in names, sorted(names)
    near(got, exp)


FUSED_NAMES = ["wino_fused", "wino_fused_ws", "wino_fused_g2"]


@pytest.mark.parametrize("n,ic,h,w,oc,res", [(2, 32, 23, 17, 32, True), (1, 64, 20, 20, 96, False),
                                             (3, 80, 10, 10, 80, True), (1, 64, 40, 40, 144, True),
                                             (2, 128, 13, 19, 160, False), (1, 8, 9, 7, 20, False),
                                             (4, 16, 6, 5, 32, True), (32, 32, 20, 20, 64, True),
                                             (2, 40, 12, 12, 32, True)])
@pytest.mark.parametrize("form", [0, 1, 2], ids=["fourwave", "specialized", "twogroups"])
def test_wino_fused_matches_two_kernel(hip, monkeypatch, n, ic, h, w, oc, res, form):
    """The fused Winograd kernels (input transform inside the plane GEMM:
    four waves doing both; four MFMA waves beside four transform waves; two
    four-wave groups over 64 output channels sharing each transform) compute
    the transform, the fragments and the sums of the two-kernel form in the
    same order: bit-identical outputs, and within tolerance of the oracle.
    Covers one K chunk, an odd chunk count, odd channel blocks (the two-group
    form's second group then stores nothing), a tile count below one block,
    ragged tiles, strided views and the fused residual."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(form))
    seed = 9950 + n + ic + h + oc
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, 3, 3), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    exp = oracle.conv2d(x, wt, b, (1, 1), (1, 1, 1, 1), silu=True)
    r = synth.activations(exp.shape, seed + 3) if res else None
    if res:
        exp = r + exp
    fused, names = _run_conv(hip, x, wt, b, 1, 1, CONV_WINOGRAD, r, profile=True)
    assert FUSED_NAMES[form] in names and "wino_input_blk" not in names, sorted(names)
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", "0")
    two, _ = _run_conv(hip, x, wt, b, 1, 1, CONV_WINOGRAD2, r)
    np.testing.assert_array_equal(fused, two)
    near(fused, exp)


@pytest.mark.parametrize("form", [0, 1, 2], ids=["fourwave", "specialized", "twogroups"])
@pytest.mark.parametrize("ic", [4, 12, 20])
def test_wino_fused_partial_chunk(hip, monkeypatch, ic, form):
    """Input channels that do not fill the last 8-channel K chunk (or the
    last 16 channels of the specialized form): the fused kernels read them
    as zero (their weights are zero-padded to the chunk)."""
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(form))
    n, h, w, oc = 2, 13, 9, 40
    seed = 9970 + ic
    x = synth.activations((n, ic, h, w), seed)
    wt = synth.kaiming((oc, ic, 3, 3), seed + 1)
    b = synth.activations((oc,), seed + 2) * np.float32(0.1)
    exp = oracle.conv2d(x, wt, b, (1, 1), (1, 1, 1, 1), silu=True)
    got, names = _run_conv(hip, x, wt, b, 1, 1, CONV_WINOGRAD, None, profile=True)
    assert FUSED_NAMES[form] in names, sorted(names)
    near(got, exp)


# ---------------------------------------------------------------- upsampled input part

def _upsampled_case(hip, n, ku, kr, h, w, oc, res, seed, profile=True):
    """sy_conv_run_upsampled of a 1x1 conv over concat(upsample2x(xu), rest)
    against the oracle's resize + concat + conv; returns (got, exp, names)."""
    xu = synth.activations((n, ku, h // 2, w // 2), seed)
    rest = synth.activations((n, kr, h, w), seed + 1)
    wt = synth.kaiming((oc, ku + kr, 1, 1), seed + 2)
    b = synth.activations((oc,), seed + 3) * np.float32(0.1)
    full = np.concatenate([oracle.resize_nearest(xu, h, w), rest], axis=1)
    exp = oracle.conv2d(full, wt, b, (1, 1), (0, 0, 0, 0), silu=True)
    r = synth.activations(exp.shape, seed + 4) if res else None
    if res:
        exp = r + exp
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, b, (1, 1), (0, 0, 0, 0), silu=True)
        xuv = hip.alloc(n, ku + 8, h // 2, w // 2).slice(4, ku)
        hip.upload(xu, xuv)
        xv = hip.alloc(n, ku + kr + 4, h, w).slice(4, ku + kr)
        hip.upload(rest, xv.slice(ku, kr))   # the leading ku channels stay unwritten
        yv = hip.alloc(n, oc + 12, h, w).slice(8, oc)
        rv = None
        if res:
            rv = hip.alloc(n, oc + 8, h, w).slice(4, oc)
            hip.upload(r, rv)
        names = set()
        if profile:
            hip.profile_enable(True)
            hip.profile_read()
        try:
            hip.conv_upsampled(conv, xuv, xv, yv, rv)
            hip.flush()
            if profile:
                names = set(hip.profile_read())
        finally:
            if profile:
                hip.profile_enable(False)
        got = hip.download(yv)
    finally:
        hip.end_frame()
    return got, exp, names


@pytest.mark.parametrize("res", [False, True], ids=["plain", "res"])
@pytest.mark.parametrize("tile", range(len(TILES)))
def test_upsampled_part_forced_tile(hip, monkeypatch, tile, res):
    """Every GEMM tile on the upsampled-part addressing (MODE 3): a 64-channel
    half-resolution part and a 32-channel full-resolution part (K tiles of 16
    and 32 both stay on one side), ragged M and N, residual fused."""
    monkeypatch.setenv("SIMDYOLO_HIP_AUTOTUNE", "0")
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", str(tile))
    got, exp, names = _upsampled_case(hip, 2, 64, 32, 14, 18, 40, res, 9900 + tile)
    want = tile_name(tile, "conv", 3)
    assert want in names, f"expected {want}, profile saw {sorted(names)}"
    assert "resize_nearest" not in names
    near(got, exp)


@pytest.mark.parametrize("split", [2, 4])
def test_upsampled_part_split_k(hip, monkeypatch, split):
    monkeypatch.setenv("SIMDYOLO_HIP_AUTOTUNE", "0")
    monkeypatch.setenv("SIMDYOLO_HIP_TILE", "2")
    monkeypatch.setenv("SIMDYOLO_HIP_SPLIT", str(split))
    got, exp, names = _upsampled_case(hip, 1, 128, 64, 20, 20, 64, True, 9950 + split)
    assert any(nm.startswith(tile_name(2, "conv", 3) + "_sk") for nm in names), sorted(names)
    near(got, exp)


def test_upsampled_part_autotuned_and_fallback(hip):
    """The tuner's pick on a YOLOv8n head shape, and a 16-channel upsampled
    part (not a whole number of 32-channel K tiles), which runs as the resize
    into the concat followed by the plain conv."""
    got, exp, names = _upsampled_case(hip, 2, 256, 128, 40, 40, 128, False, 9970)
    assert "resize_nearest" not in names and any(nm.startswith("igemm_m3_") for nm in names), sorted(names)
    near(got, exp)
    got, exp, names = _upsampled_case(hip, 1, 16, 32, 12, 10, 24, True, 9980)
    assert "resize_nearest" in names, sorted(names)
    near(got, exp)


def test_upsampled_part_rejects_mismatched_views(hip):
    """A source that is not a half-size NHWC view of the input's leading
    channels is refused before any launch."""
    from simdyolo_amd import SyError
    wt = synth.kaiming((16, 96, 1, 1), 9990)
    hip.begin_frame()
    try:
        conv = hip.conv_create(wt, None, (1, 1), (0, 0, 0, 0), silu=True)
        x = hip.alloc(1, 96, 8, 8)
        y = hip.alloc(1, 16, 8, 8)
        for xu in (hip.alloc(1, 64, 8, 8),      # not half size
                   hip.alloc(1, 64, 4, 3),      # width not half
                   hip.alloc(2, 64, 4, 4),      # batch differs
                   hip.alloc(1, 96, 4, 4)):     # no channels left for the rest
            with pytest.raises(SyError) as e:
                hip.conv_upsampled(conv, xu, x, y)
            assert e.value.code == 1, e.value
    finally:
        hip.end_frame()
