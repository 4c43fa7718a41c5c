"""sy_e2e_topk_noalloc: the allocation-free top-k entry point.

It runs the same kernels as sy_e2e_topk over a fixed per-GPU scratch block
instead of the context's scratch, so its rows must be bit-identical to
sy_e2e_topk's.  Two calls in a row (the second on a smaller input) check that
the block's leftover contents from the first call do not leak into the second.
Oversized requests are refused on the host before any launch.
"""
import ctypes

import numpy as np
import pytest

from _inputs import special_input
from simdyolo_amd import SyError, _native as N
from simdyolo_amd.device import HipContext

pytestmark = pytest.mark.gpu


def _call(ctx, fn, src, x, maximum, classes, onnx, dst, k, fields):
    batch, channels, anchors = x.shape
    N.check(getattr(N.lib(), fn)(ctx.handle, ctypes.c_void_p(src), batch, channels, anchors, classes, maximum,
                                 onnx, ctypes.c_void_p(dst)))
    ctx.flush()
    return ctx.d2h(dst, (batch, k, fields))


def _both(ctx, x, maximum, classes, onnx):
    x = np.ascontiguousarray(x, dtype=np.float32)
    batch, channels, anchors = x.shape
    k = min(maximum, anchors)
    fields = 6 + channels - classes - 4
    src = ctx.malloc(x.nbytes)
    dst = ctx.malloc(max(4, batch * k * fields * 4))
    try:
        ctx.h2d(src, x)
        ref = _call(ctx, "sy_e2e_topk", src, x, maximum, classes, onnx, dst, k, fields)
        # Poison the output so a call that writes nothing cannot pass.
        ctx.h2d(dst, np.full((batch, k, fields), np.nan, np.float32))
        got = _call(ctx, "sy_e2e_topk_noalloc", src, x, maximum, classes, onnx, dst, k, fields)
    finally:
        ctx.free(src)
        ctx.free(dst)
    return ref, got


def _yolo26_like(batch, anchors, classes, extra, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((batch, 4 + classes + extra, anchors)).astype(np.float32)
    # Exact ties at quantised scores.
    x[:, 4:4 + classes] = np.round(x[:, 4:4 + classes] * 8) / 8
    return x


@pytest.mark.parametrize("onnx", [0, 1])
def test_noalloc_topk_matches_topk_twice(onnx):
    with HipContext(0) as ctx:
        big = _yolo26_like(32, 8400, 80, 32, 11 + onnx)          # ~5.5 MB of scratch
        ref, got = _both(ctx, big, 300, 80, onnx)
        assert got.tobytes() == ref.tobytes()
        small = special_input(3, 6, 97, onnx)                     # special values, ties
        ref2, got2 = _both(ctx, small, 40, 6, onnx)
        assert got2.tobytes() == ref2.tobytes()


def test_noalloc_topk_refuses_oversize_before_launch():
    """A request whose scratch exceeds the fixed block is refused on the host.
    The head and output buffers are full-sized anyway, so the call stays in
    bounds even if the block ever grew enough to accept it."""
    with HipContext(0) as ctx:
        batch, classes, anchors = 512, 80, 8400                   # ~88 MB of scratch > 32 MiB
        src = ctx.malloc(batch * (classes + 4) * anchors * 4)
        dst = ctx.malloc(batch * 300 * 6 * 4)
        try:
            with pytest.raises(SyError) as e:
                N.check(N.lib().sy_e2e_topk_noalloc(ctx.handle, ctypes.c_void_p(src), batch, classes + 4, anchors,
                                                    classes, 300, 0, ctypes.c_void_p(dst)))
            assert e.value.code == N.SY_EUNSUPPORTED
            assert "fixed block" in str(e.value)
        finally:
            ctx.free(src)
            ctx.free(dst)


def _rows(ctx, fn, src, shape, maximum, classes, onnx, dst):
    batch, channels, anchors = shape
    N.check(getattr(N.lib(), fn)(ctx.handle, ctypes.c_void_p(src), batch, channels, anchors, classes, maximum,
                                 onnx, ctypes.c_void_p(dst)))


def test_noalloc_topk_first_call_under_capture():
    """On a fresh context (empty scratch) the first call ever is made inside a
    graph capture, where any allocation is refused (ensure_scratch returns
    SY_ESTATE while capturing): the capture must succeed, and each launch of
    the graph must give sy_e2e_topk's rows, which a second context computes
    afterwards."""
    x = _yolo26_like(4, 8400, 80, 32, 5)
    batch, channels, anchors = x.shape
    k, fields = 300, 6 + 32
    with HipContext(0) as ctx:
        src = ctx.malloc(x.nbytes)
        dst = ctx.malloc(batch * k * fields * 4)
        try:
            ctx.h2d(src, x)
            ctx.h2d(dst, np.full((batch, k, fields), np.nan, np.float32))
            ctx.graph_begin()
            try:
                _rows(ctx, "sy_e2e_topk_noalloc", src, x.shape, 300, 80, 0, dst)
            finally:
                g = ctx.graph_end()
            got = []
            for _ in range(2):
                ctx.graph_launch(g)
                ctx.flush()
                got.append(ctx.d2h(dst, (batch, k, fields)))
                ctx.h2d(dst, np.full((batch, k, fields), np.nan, np.float32))
        finally:
            ctx.free(src)
            ctx.free(dst)
    with HipContext(0) as ref_ctx:
        ref, _ = _both(ref_ctx, x, 300, 80, 0)
    for rows in got:
        assert rows.tobytes() == ref.tobytes()


def test_noalloc_topk_two_contexts_back_to_back():
    """Two contexts (two streams) enqueue calls on the shared block without
    waiting in between; the library orders them, so each gets its own
    input's rows.  Both requests have the same shape, so every index the
    kernels form stays inside the buffers whatever the ordering."""
    xs = [_yolo26_like(8, 8400, 80, 32, 21 + j) for j in range(2)]
    shape = xs[0].shape
    k, fields = 300, 6 + 32
    ctxs = [HipContext(0), HipContext(0)]
    bufs = []
    try:
        for ctx, x in zip(ctxs, xs):
            src, dst = ctx.malloc(x.nbytes), ctx.malloc(shape[0] * k * fields * 4)
            bufs.append((ctx, src, dst))
            ctx.h2d(src, x)
        for _ in range(3):
            for ctx, src, dst in bufs:
                _rows(ctx, "sy_e2e_topk_noalloc", src, shape, 300, 80, 0, dst)
        got = []
        for ctx, src, dst in bufs:
            ctx.flush()
            got.append(ctx.d2h(dst, (shape[0], k, fields)))
    finally:
        for ctx, src, dst in bufs:
            ctx.free(src)
            ctx.free(dst)
        for ctx in ctxs:
            ctx.close()
    with HipContext(0) as ref_ctx:
        for x, rows in zip(xs, got):
            ref, _ = _both(ref_ctx, x, 300, 80, 0)
            assert rows.tobytes() == ref.tobytes()
