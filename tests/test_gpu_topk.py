"""End-to-end two-stage top-k on the GPU vs the oracle, bit-exact.

Inputs follow the reference's own generator (CpuPtEndToEndTests.cs:58-86:
NaN payloads, +-inf, +-0, +-denormal, exact ties) over its parameter grid,
plus YOLO26-scale heads (8400 anchors, 80 classes, 32 mask coefficients,
k = 300) with many exact ties."""
import numpy as np
import pytest

import oracle
from _inputs import special_input

pytestmark = pytest.mark.gpu


def run_gpu(hip, x, maximum, classes, onnx):
    x = np.ascontiguousarray(x, dtype=np.float32)
    batch, channels, anchors = x.shape
    k = min(maximum, anchors)
    fields = 6 + channels - classes - 4
    src = hip.malloc(max(1, x.nbytes))
    dst = hip.malloc(max(4, batch * k * fields * 4))
    try:
        hip.h2d(src, x)
        hip.e2e_topk(src, batch, channels, anchors, classes, maximum, onnx, dst)
        hip.flush()
        return hip.d2h(dst, (batch, k, fields))
    finally:
        hip.free(src)
        hip.free(dst)


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("onnx", [False, True])
def test_topk_reference_grid(hip, onnx):
    checked = 0
    for batch in (1, 2):
        for classes in (1, 3, 7):
            for anchors in (1, 7, 8, 9, 37):
                for maximum in (1, 8, 49):
                    if onnx and maximum > anchors:
                        continue
                    for frame in range(4):
                        x = special_input(batch, classes, anchors, frame)
                        exp = oracle.e2e_select(x, maximum, classes, onnx=onnx)
                        got = run_gpu(hip, x, maximum, classes, onnx)
                        assert same_bits(got, exp), (batch, classes, anchors, maximum, frame)
                        checked += 1
    assert checked > 100


@pytest.mark.parametrize("onnx", [False, True])
@pytest.mark.parametrize("seed", [0, 1])
def test_topk_yolo26_scale(hip, onnx, seed):
    r = np.random.Generator(np.random.PCG64(seed))
    batch, nc, extra, anchors = 2, 80, 32, 8400
    x = r.standard_normal((batch, 4 + nc + extra, anchors)).astype(np.float32)
    # Quantised sigmoid-like scores: many exact ties across anchors and classes.
    x[:, 4:4 + nc] = np.round(r.uniform(0, 1, (batch, nc, anchors)) * 256).astype(np.float32) / 256
    x[0, 4, ::97] = np.nan
    x[1, 4 + 3, ::131] = -0.0
    exp = oracle.e2e_select(x, 300, nc, onnx=onnx)
    got = run_gpu(hip, x, 300, nc, onnx)
    assert same_bits(got, exp)


@pytest.mark.parametrize("onnx", [False, True])
@pytest.mark.parametrize("anchors", [2049, 12000, 33600, 40000])
def test_topk_register_chunks_and_global_keys(hip, onnx, anchors):
    """Each stage-1 instantiation: 2049 anchors (3 register chunks per
    thread), 12000 (17 chunks), 1280x1280 heads (33600 anchors, the largest
    register instantiation) and 40000 (keys re-read from global memory on
    every radix pass); bit-exact with ties and a NaN column."""
    r = np.random.Generator(np.random.PCG64(anchors))
    batch, nc, extra = 2, 80, 32
    x = r.standard_normal((batch, 4 + nc + extra, anchors)).astype(np.float32)
    x[:, 4:4 + nc] = np.round(r.uniform(0, 1, (batch, nc, anchors)) * 512).astype(np.float32) / 512
    x[0, 4 + 7, ::211] = np.nan
    exp = oracle.e2e_select(x, 300, nc, onnx=onnx)
    got = run_gpu(hip, x, 300, nc, onnx)
    assert same_bits(got, exp)


def test_topk_zero_k_and_small_anchor_counts(hip):
    x = special_input(2, 5, 61, 0)
    assert run_gpu(hip, x, 0, 5, False).shape == (2, 0, 6)
    exp = oracle.e2e_select(x, 17, 5)
    assert same_bits(run_gpu(hip, x, 17, 5, False), exp)


@pytest.mark.parametrize("onnx", [False, True])
def test_topk_flood_of_ties(hip, onnx):
    """Every score equal: each selected anchor's whole class column reaches the
    stage-1 bound, so the candidate list overflows and the full pair set is
    ranked by tie index alone."""
    batch, nc, extra, anchors = 2, 80, 4, 8400
    x = np.full((batch, 4 + nc + extra, anchors), 0.5, np.float32)
    x[:, :4] = np.random.Generator(np.random.PCG64(3)).standard_normal((batch, 4, anchors)).astype(np.float32)
    exp = oracle.e2e_select(x, 300, nc, onnx=onnx)
    got = run_gpu(hip, x, 300, nc, onnx)
    assert same_bits(got, exp)


@pytest.mark.parametrize("onnx", [False, True])
@pytest.mark.parametrize("nc", [4, 5, 80])
def test_topk_columns_tied_at_the_bound(hip, onnx, nc):
    """A few anchors with more than four classes tied at the top score: their
    class columns are read in full; the rest come from the four-best lists."""
    r = np.random.Generator(np.random.PCG64(nc))
    batch, anchors = 2, 8400
    x = r.standard_normal((batch, 4 + nc, anchors)).astype(np.float32)
    top = np.float32(x[:, 4:].max() + 1)
    for b in range(batch):
        picks = r.choice(anchors, 25, replace=False)
        for a in picks:
            cls = r.choice(nc, min(nc, 6), replace=False)
            x[b, 4 + cls, a] = top
    x[0, 4 + nc - 1, 5] = -0.0
    exp = oracle.e2e_select(x, 300, nc, onnx=onnx)
    got = run_gpu(hip, x, 300, nc, onnx)
    assert same_bits(got, exp)


@pytest.mark.parametrize("prefix", [3, 11])
def test_topk_misaligned_head(hip, prefix):
    """A head view that starts a few floats into its buffer (GpuTopKTests.cs:159-169
    builds such views with a 3..11-float sentinel prefix)."""
    r = np.random.Generator(np.random.PCG64(prefix))
    batch, nc, extra, anchors = 2, 80, 32, 8400
    x = r.standard_normal((batch, 4 + nc + extra, anchors)).astype(np.float32)
    flat = np.concatenate([np.full(prefix, np.nan, np.float32), x.ravel()])
    k, fields = 300, 6 + extra
    src = hip.malloc(flat.nbytes)
    dst = hip.malloc(batch * k * fields * 4)
    try:
        hip.h2d(src, flat)
        hip.e2e_topk(src + 4 * prefix, batch, 4 + nc + extra, anchors, nc, k, False, dst)
        hip.flush()
        got = hip.d2h(dst, (batch, k, fields))
    finally:
        hip.free(src)
        hip.free(dst)
    assert same_bits(got, oracle.e2e_select(x, k, nc, onnx=False))
