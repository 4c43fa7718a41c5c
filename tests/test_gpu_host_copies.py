"""Host <-> device copies through the context's pinned staging.

sy_memcpy (and sy_upload_nchw / sy_download_nchw, which use it) sends host
copies of 1 MiB or more through three 8 MiB pinned slots that host threads
fill or empty while the DMA of the slot before runs.  Bars: every copy
bit-exact, at sizes around the staging threshold and with ragged last pieces;
back-to-back uploads that reuse the slot ring before the first one's DMA is
waited for; an upload whose host buffer is overwritten as soon as the call
returns (the call must have read it); uploads and downloads through the
layout-converting entry points (NCHW host <-> NHWC device view).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MiB = 1 << 20


def _data(nbytes, seed):
    n = nbytes // 4
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


@pytest.mark.parametrize("nbytes", [MiB - 4, MiB, MiB + 4, 5 * MiB + 12, 24 * MiB, 33 * MiB + 4, 80 * MiB + 256])
def test_round_trip(hip, nbytes):
    x = _data(nbytes, nbytes)
    p = hip.malloc(x.nbytes)
    try:
        hip.h2d(p, x)
        y = hip.d2h(p, x.shape)
    finally:
        hip.free(p)
    np.testing.assert_array_equal(y, x)


def test_back_to_back_uploads_reuse_the_ring(hip):
    """Five uploads (more pieces than slots) before any download, then each
    buffer read back; the host array is overwritten after every call."""
    sizes = [3 * MiB + 8, 17 * MiB, 2 * MiB - 4, 9 * MiB + 4, 26 * MiB]
    ptrs, sent = [], []
    buf = np.empty(max(sizes) // 4, np.float32)
    try:
        for i, n in enumerate(sizes):
            x = _data(n, 100 + i)
            buf[:x.size] = x
            p = hip.malloc(n)
            ptrs.append(p)
            hip.h2d(p, buf[:x.size])
            buf[:x.size] = -1.0  # the call has read the host buffer by now
            sent.append(x)
        for p, x in zip(ptrs, sent):
            np.testing.assert_array_equal(hip.d2h(p, x.shape), x)
    finally:
        for p in ptrs:
            hip.free(p)


@pytest.mark.parametrize("shape", [(1, 3, 640, 640), (2, 64, 80, 80), (4, 24, 96, 112)])
def test_layout_converting_copies(hip, shape):
    """sy_upload_nchw into an NHWC frame tensor and sy_download_nchw back."""
    x = np.random.default_rng(sum(shape)).standard_normal(shape).astype(np.float32)
    hip.begin_frame()
    try:
        t = hip.upload(x)
        np.testing.assert_array_equal(hip.download(t), x)
    finally:
        hip.end_frame()
