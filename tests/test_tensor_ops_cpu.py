"""Pins of the oracle's restatement of the generic device ops (tensor.comp) and
of the batched device matrix product, on the CPU: each case's parameter block
is built as the reference's callers build it, and the oracle's result must
equal what a library routine gives for the same operation (torch.nn.functional,
numpy).  A wrong index, stride slot or broadcast rule in the oracle fails here.
"""
import numpy as np
import pytest

import oracle
from oracle import tensor_ops
from _tensor_cases import assert_close, batch_strides, cases, matmul_cases
from _tensor_params import decode_head, decode_pose

CASES = cases()


def _run(c):
    return tensor_ops.run(c["op"], c["a"], c["b"], c["d"], c["params"], c["out_len"], c["prefill"])


@pytest.mark.parametrize("c", [c for c in CASES if c["expect"] is not None], ids=lambda c: c["name"])
def test_oracle_matches_library(c):
    assert_close(_run(c), c["expect"], c["tol"])


@pytest.mark.parametrize("bins,xyxy", [(16, False), (16, True), (1, True), (1, False)])
def test_oracle_decode_matches_c_oracle(bins, xyxy):
    """Op 30 against the C oracle's head decode (itself pinned on the
    reference's golden detections)."""
    c = next(c for c in CASES if c["name"] == f"decode_b{bins}_x{int(xyxy)}")
    boxes = c["a"].reshape(2, 4 * bins, 5, 6)
    scores = c["b"].reshape(2, 7, 5, 6)
    exp = oracle.detect_decode([(boxes, scores, 16.0)], bins, xyxy)
    assert_close(_run(c), exp, 2e-6)


def test_oracle_decode_level_offset():
    c = next(c for c in CASES if c["name"] == "decode_level_offset")
    got = _run(c).reshape(2, 9, 40)
    exp = oracle.detect_decode([(c["a"].reshape(2, 64, 4, 3), c["b"].reshape(2, 5, 4, 3), 32.0)], 16, False)
    assert_close(got[:, :, 25:37], exp, 2e-6)
    assert not got[:, :, :25].any() and not got[:, :, 37:].any()


@pytest.mark.parametrize("y26", [False, True])
def test_oracle_pose_rules(y26):
    """Op 31: keypoint x, y = (v * 2 + grid) * stride for YOLOv8 and
    (v + grid + 0.5) * stride for YOLO26, confidence = sigmoid(v)."""
    c = next(c for c in CASES if c["name"] == f"pose_y26{int(y26)}")
    kp = c["a"].reshape(2, 17, 3, 4, 5).astype(np.float64)
    gy, gx = np.meshgrid(np.arange(4), np.arange(5), indexing="ij")
    exp = np.empty_like(kp)
    if y26:
        exp[:, :, 0] = (kp[:, :, 0] + gx + 0.5) * 8
        exp[:, :, 1] = (kp[:, :, 1] + gy + 0.5) * 8
    else:
        exp[:, :, 0] = (kp[:, :, 0] * 2 + gx) * 8
        exp[:, :, 1] = (kp[:, :, 1] * 2 + gy) * 8
    exp[:, :, 2] = 1 / (1 + np.exp(-kp[:, :, 2]))
    assert_close(_run(c), exp, 1e-6)


def test_oracle_dfl_closed_forms():
    """DFL of one-hot logits is the hot bin; of equal logits, (bins - 1) / 2."""
    from _tensor_params import dfl
    op, p, n, out = dfl((1, 64, 10), 16)
    x = np.full((1, 4, 16, 10), -80.0, np.float32)
    hot = np.arange(40).reshape(4, 10) % 16
    for s in range(4):
        for a in range(10):
            x[0, s, hot[s, a], a] = 80.0
    assert_close(tensor_ops.run(op, x.reshape(-1), None, None, p, 40), hot.astype(np.float32), 1e-6)
    flat = np.zeros((1, 64, 10), np.float32)
    assert_close(tensor_ops.run(op, flat.reshape(-1), None, None, p, 40), np.full(40, 7.5, np.float32), 1e-7)


@pytest.mark.parametrize("name,m,n,k,batch,ab,bb", matmul_cases(), ids=[c[0] for c in matmul_cases()])
def test_oracle_matmul_matches_numpy(name, m, n, k, batch, ab, bb):
    rng = np.random.default_rng(7)
    a = rng.standard_normal(tuple(ab) + (m, k)).astype(np.float32)
    b = rng.standard_normal(tuple(bb) + (k, n)).astype(np.float32)
    exp = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    got = tensor_ops.matmul(a, b, m, n, k, batch, batch_strides(batch, ab), batch_strides(batch, bb))
    assert_close(got, np.broadcast_to(exp, tuple(batch) + (m, n)) if batch else exp, 1e-6)


def test_oracle_params_builders_cover_every_op():
    """Every op the HIP entry accepts has at least one case."""
    ops = {c["op"] for c in CASES}
    assert ops == {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 20, 21, 22, 23, 24, 25, 26, 30, 31, 32,
                   33, 34, 35, 36, 37}
    assert decode_head(1, 2, 2, 16, 3, 8.0, True)[1][0] == 4
    assert decode_pose((1, 6, 2, 2), 2, 3, 8.0, False)[2] == 24
