"""Parity of the generic device ops through the C ABI: ``sy_compute`` (the
reference's IDeviceBackend.Compute over shaders/tensor.comp) and ``sy_matmul``
(IDeviceBackend.DeviceMatMul) against the oracle's restatement, on the cases
whose parameter blocks are built as the reference's callers build them.

Data movement, comparisons and single roundings of +, -, *, / are bit-exact;
ops that evaluate exp or pow, or add taps, are held to each case's stated
relative tolerance (to the largest output magnitude); matrix products to
2e-5 of the largest output magnitude (FP32 accumulation over k <= 64 against
the oracle's float64).
"""
import numpy as np
import pytest

from simdyolo_amd import SyError, _native as N
from oracle import tensor_ops
from _tensor_cases import assert_close, batch_strides, cases, matmul_cases
from _tensor_params import binary, block, unary

pytestmark = pytest.mark.gpu
CASES = cases()


class _Buffers:
    """Device copies of host arrays, freed together."""

    def __init__(self, hip):
        self.hip, self.ptrs, self.keep = hip, [], []

    def put(self, host):
        if host is None:
            return None
        host = np.ascontiguousarray(host, np.float32).reshape(-1)
        self.keep.append(host)
        ptr = self.hip.malloc(max(host.nbytes, 4))
        self.hip.h2d(ptr, host)
        self.ptrs.append(ptr)
        return ptr, host.size

    def free(self):
        self.hip.flush()
        for p in self.ptrs:
            self.hip.free(p)


def _device_run(hip, c, out_len=None):
    bufs = _Buffers(hip)
    try:
        out_len = c["out_len"] if out_len is None else out_len
        init = c["prefill"] if c["prefill"] is not None else np.zeros(out_len, np.float32)
        out_ptr, _ = bufs.put(init)
        hip.compute(c["op"], [bufs.put(c["a"]), bufs.put(c["b"]), bufs.put(c["d"])], c["params"], c["items"],
                    out_ptr, out_len)
        return hip.d2h(out_ptr, (out_len,))
    finally:
        bufs.free()


@pytest.mark.parametrize("c", CASES, ids=lambda c: c["name"])
def test_compute_matches_oracle(hip, c):
    print(f"sy_compute op {c['op']} case {c['name']}", flush=True)
    got = _device_run(hip, c)
    exp = tensor_ops.run(c["op"], c["a"], c["b"], c["d"], c["params"], c["out_len"], c["prefill"])
    assert_close(got, exp, c["tol"])


def test_compute_offsets_and_large(hip):
    """Element offsets P(28..31) shift every binding, and a launch of more
    than 2^20 work items covers every item."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal(3 * 1024 * 1024 + 7).astype(np.float32)
    b = rng.standard_normal(1 << 20).astype(np.float32)
    op, p, n, _ = binary(12, (3, 1024, 1024), (1024, 1024))
    p[28], p[29], p[30] = 7, 0, 5
    c = dict(op=op, params=p, items=n, out_len=n + 5, prefill=None, a=a, b=b, d=None, tol=0)
    got = _device_run(hip, c)
    exp = tensor_ops.run(op, a, b, None, p, n + 5)
    assert_close(got, exp, 0)
    assert got[:5].tolist() == [0.0] * 5


def test_compute_refuses_bad_blocks(hip):
    bufs = _Buffers(hip)
    try:
        x = bufs.put(np.ones(64, np.float32))
        out, _ = bufs.put(np.zeros(64, np.float32))
        op, p, n, _ = unary(1, (64,))
        with pytest.raises(SyError) as e:  # P(0) differs from the work items
            hip.compute(op, [x, None, None], p, n - 1, out, 64)
        assert e.value.code == N.SY_EINVAL
        with pytest.raises(SyError) as e:
            hip.compute(17, [x, None, None], p, n, out, 64)
        assert e.value.code == N.SY_EUNSUPPORTED
        with pytest.raises(SyError) as e:  # work items past the output
            hip.compute(op, [x, None, None], p, n, out, 32)
        assert e.value.code == N.SY_EINVAL
        op, p, n, _ = binary(10, (8, 8), (8, 8))
        p[7] = 64  # a stride reaching past input A
        with pytest.raises(SyError) as e:
            hip.compute(op, [x, x, None], p, n, out, 64)
        assert e.value.code == N.SY_EINVAL
        with pytest.raises(SyError) as e:  # binary without its second input
            hip.compute(10, [x, None, None], binary(10, (8, 8), (8, 8))[1], 64, out, 64)
        assert e.value.code == N.SY_EINVAL
        zero = block(0)
        hip.compute(1, [x, None, None], zero, 0, out, 64)  # zero work items: no launch
    finally:
        bufs.free()


@pytest.mark.parametrize("name,m,n,k,batch,ab,bb", matmul_cases(), ids=[c[0] for c in matmul_cases()])
def test_matmul_matches_oracle(hip, name, m, n, k, batch, ab, bb):
    print(f"sy_matmul {name} m={m} n={n} k={k} batch={batch}", flush=True)
    rng = np.random.default_rng(11)
    a = rng.standard_normal(tuple(ab) + (m, k)).astype(np.float32)
    b = rng.standard_normal(tuple(bb) + (k, n)).astype(np.float32)
    count = int(np.prod(batch)) if batch else 1
    sa, sb = batch_strides(batch, ab), batch_strides(batch, bb)
    bufs = _Buffers(hip)
    try:
        (pa, la), (pb, lb) = bufs.put(a), bufs.put(b)
        pc, lc = bufs.put(np.zeros(count * m * n, np.float32))
        hip.matmul(pa, pb, pc, m, n, k, batch, sa, sb, la, lb, lc)
        got = hip.d2h(pc, (count * m * n,))
    finally:
        bufs.free()
    exp = tensor_ops.matmul(a, b, m, n, k, batch, sa, sb)
    assert_close(got, exp, 2e-5)


def test_matmul_refusals(hip):
    bufs = _Buffers(hip)
    try:
        (pa, la) = bufs.put(np.ones(64, np.float32))
        with pytest.raises(SyError) as e:
            hip.matmul(pa, pa, pa, 0, 8, 8, (), (), (), la, la, la)
        assert e.value.code == N.SY_EUNSUPPORTED
        with pytest.raises(SyError) as e:  # second batch matrix past the buffer
            hip.matmul(pa, pa, pa, 8, 8, 8, (2,), (1,), (0,), la, la, 128)
        assert e.value.code == N.SY_EINVAL
    finally:
        bufs.free()
