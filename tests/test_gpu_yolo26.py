"""YOLO26 end to end on the GPU against the oracle: the decoded head before
selection, the two-stage top-k rows with the mask coefficients as extras, the
Proto26 prototypes and the instance masks (PtModel.cs:345-359, 444-570;
CpuMaskDecoder.cs:18-81).

Bars: head and prototypes within max-rel 1e-3 (relative to max(1, |ref|)),
the head's boxes compared as the raw distances (grid cells) they decode from;
the device selection bit-exact against the oracle's selection on the same
(device) head; against the oracle's own head, (anchor, class) pairs equal
except pairs whose score lies within 1e-4 of a selection boundary, and shared
rows within max-rel 1e-3; identical mask crops; probabilities against the oracle's decode of the
device's own prototypes and coefficients within the FP32 forward-error bound
of the coefficient dot product, and against the oracle's model outputs within
the first-order bound that the measured prototype/coefficient differences
allow.
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import _native as N
from simdyolo_amd import synth
from simdyolo_amd.detector import YoloDetector
from _parity import max_rel

pytestmark = pytest.mark.gpu
NM, NC, K = 32, 80, 300


def _grid(size):
    """Anchor centres (grid units) and strides of the 8/16/32 levels."""
    cx, cy, st = [], [], []
    for s in (8, 16, 32):
        n = size // s
        yy, xx = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
        cx.append(xx.ravel() + 0.5)
        cy.append(yy.ravel() + 0.5)
        st.append(np.full(n * n, float(s)))
    return np.concatenate(cx), np.concatenate(cy), np.concatenate(st)


def _raw(head, size):
    """The head in the units of the raw one2one outputs: the four box
    distances in grid cells (x1 = (cx - d0) * stride, ...), then the scores
    and extras unchanged.  Decoding multiplies a distance by the stride, so a
    bar relative to max(1, |x|) is applied before that scaling."""
    cx, cy, st = _grid(size)
    h = head.astype(np.float64).copy()
    h[..., 0, :] = cx - h[..., 0, :] / st
    h[..., 1, :] = cy - h[..., 1, :] / st
    h[..., 2, :] = h[..., 2, :] / st - cx
    h[..., 3, :] = h[..., 3, :] / st - cy
    return h


def _anchor_of(head, rows):
    """Anchor of every selected row: the column whose x1 y1 x2 y2 and class
    score the row carries."""
    keys = {tuple(head[0:4, a].tolist()): a for a in range(head.shape[1])}
    out = []
    for r in rows:
        a = keys[tuple(r[0:4].tolist())]
        assert head[4 + int(r[5]), a] == r[4]
        out.append((a, int(r[5])))
    return out


def _boundaries(head, k):
    """Stage-1 (per-anchor max score) and stage-2 (pair score) k-th values."""
    best = head[4:4 + NC].max(0)
    s1 = float(np.sort(best)[-k])
    top = np.argsort(-best, kind="stable")[:k]
    s2 = float(np.sort(head[4:4 + NC, top].ravel())[-k])
    return best, s1, s2


def _check_selection(rows, head, exp_rows, exp_head, k, size):
    got = _anchor_of(head, rows)
    exp = _anchor_of(exp_head, exp_rows)
    best, s1, s2 = _boundaries(exp_head, k)
    for a, c in set(got) ^ set(exp):
        near = abs(float(exp_head[4 + c, a]) - s2) <= 1e-4 or abs(float(best[a]) - s1) <= 1e-4
        assert near, f"pair (anchor {a}, class {c}) score {exp_head[4 + c, a]} only on one side"
    ei = {p: i for i, p in enumerate(exp)}
    shared = [(i, ei[p]) for i, p in enumerate(got) if p in ei]
    assert len(shared) >= 0.9 * k
    gi, xi = zip(*shared)
    # Shared rows: scores and extras as they are, boxes as grid distances.
    anchors = np.array([got[i][0] for i in gi])
    cx, cy, st = (g[anchors] for g in _grid(size))

    def dist(r):
        r = r.astype(np.float64)
        return np.stack([cx - r[:, 0] / st, cy - r[:, 1] / st, r[:, 2] / st - cx, r[:, 3] / st - cy], 1)
    a, b = rows[list(gi)], exp_rows[list(xi)]
    assert max_rel(a[:, 4:], b[:, 4:]) <= 1e-3
    assert max_rel(dist(a), dist(b)) <= 1e-3
    return shared


@pytest.fixture(scope="module")
def seg_model():
    cfg = synth.config("n", arch="yolo26", nm=NM, npr=256)
    lay = synth.layout(cfg)
    # Class bias 0 spreads the scores, so the selection decides real cases.
    params = synth.params_for_layout(lay, seed=synth.SEED + 26, cls_bias=0.0)
    return cfg, params


def test_yolo26n_seg_640_head_rows_and_masks(hip, seg_model):
    cfg, params = seg_model
    size = 640
    x = synth.images(1, size, size, seed=synth.SEED + 27)
    print("YOLO26n-seg B=1 640: oracle forward", flush=True)
    exp_head, exp_proto = oracle.yolo26_forward(params, x, nm=NM, npr=256)
    with YoloDetector(cfg, params, ctx=hip) as det:
        assert det.output_shape(1, size, size) == (1, K, 6 + NM)
        for rep in range(2):  # eager (tuning) pass, then the captured graph
            print(f"YOLO26n-seg B=1 640: device forward {rep}", flush=True)
            rows, proto = det.predict_seg(x)
            hptr, (c, a) = det.head_buffer(1, size, size)
            assert (c, a) == (NC + 4 + NM, 8400)
            head = hip.d2h(hptr, (1, c, a))
            assert max_rel(_raw(head, size), _raw(exp_head, size)) <= 1e-3
            assert max_rel(proto, exp_proto) <= 1e-3
            # The device selection with extras, bit-exact on its own head.
            np.testing.assert_array_equal(rows, oracle.e2e_select(head, K, NC))
            exp_rows = oracle.e2e_select(exp_head, K, NC)
            shared = _check_selection(rows[0], head[0], exp_rows[0], exp_head[0], K, size)
        # Masks of 40 shared rows from the model's own prototype buffer and the
        # coefficient rows of its output buffer.
        pptr, (pc, ph, pw) = det.proto_buffer(1, size, size)
        _, out_ptr = det.buffers(1, size, size)
    picks = []
    for gi, xi in shared:
        x1, y1, x2, y2 = (float(v) for v in rows[0, gi, :4])
        x1, y1, x2, y2 = max(0.0, x1), max(0.0, y1), min(float(size), x2), min(float(size), y2)
        if x2 - x1 >= 1 and y2 - y1 >= 1:
            picks.append((gi, xi, (x1, y1, x2 - x1, y2 - y1)))
        if len(picks) == 40:
            break
    assert len(picks) >= 20
    tr = oracle.Letterbox(size, size, size, size, 1.0, 1.0, 0, 0)
    t = N.LetterboxT(size, size, size, size, 1.0, 1.0, 0, 0)
    gpu_coeffs = [rows[0, gi, 6:] for gi, _, _ in picks]
    ref_coeffs = [exp_rows[0, xi, 6:] for _, xi, _ in picks]
    # The oracle's mask decode on the device's own prototypes and rows (the
    # kernel's parity), and on the oracle's model outputs.
    same = [oracle.mask_decode(proto[0], c, box, tr) for c, (_, _, box) in zip(gpu_coeffs, picks)]
    exp = [oracle.mask_decode(exp_proto[0], c, box, tr) for c, (_, _, box) in zip(ref_coeffs, picks)]
    cap = sum(e[0].size for e in exp)
    protos = N.Tensor(pptr, 1, pc, ph, pw, pc, N.LAYOUT_NCHW)
    ld = 6 + NM
    coeffs = np.ascontiguousarray(np.stack(gpu_coeffs), np.float32)
    cbuf = hip.malloc(coeffs.nbytes)
    out = hip.malloc(cap * 4)
    try:
        hip.h2d(cbuf, coeffs)
        info = hip.mask_decode(protos, cbuf, NM, [b for _, _, b in picks], t, out, cap)
        flat = hip.d2h(out, (cap,))
        # The same rows read in place from the model output (ld = 6 + nm).
        info2 = hip.mask_decode(protos, out_ptr + 4 * (picks[0][0] * ld + 6), ld, [picks[0][2]], t, out, cap)
        first = hip.d2h(out, (info2[0][2] * info2[0][3],))
    finally:
        hip.free(cbuf)
        hip.free(out)
    np.testing.assert_array_equal(first, flat[:first.size])
    # First-order bound of the mask-logit difference that the prototype and
    # coefficient differences allow (the bilinear resample is a convex
    # combination; sigmoid is 1/4-Lipschitz).
    dproto = np.abs(proto[0].astype(np.float64) - exp_proto[0]).reshape(NM, -1).max(1)
    pmax = np.abs(exp_proto[0].astype(np.float64)).reshape(NM, -1).max(1)
    pmax_gpu = np.abs(proto[0].astype(np.float64)).reshape(NM, -1).max(1)
    worst_same = worst = 0.0
    for i, ((m, crop), (ms, crop_s), (left, top, w, h, off)) in enumerate(zip(exp, same, info)):
        assert (left, top, w, h) == crop == crop_s
        got = flat[off:off + w * h].reshape(h, w)
        # Same inputs: the FP32 forward-error bound of the nm-term dot product
        # and the 4-tap resample (40 roundings of 2^-24 relative to
        # sum |c| max|p|), through the 1/4-Lipschitz sigmoid.
        e_same = float(np.abs(got - ms).max())
        b_same = 0.25 * 40 * 2.0 ** -24 * float((np.abs(gpu_coeffs[i]) * pmax_gpu).sum()) + 2e-6
        assert e_same <= b_same, (i, e_same, b_same)
        worst_same = max(worst_same, e_same)
        dc = np.abs(gpu_coeffs[i].astype(np.float64) - ref_coeffs[i])
        bound = 0.25 * float((np.abs(ref_coeffs[i]) * dproto + dc * pmax + dc * dproto).sum()) + 1e-5
        err = float(np.abs(got - m).max())
        assert err <= bound, (i, err, bound)
        worst = max(worst, err)
    print(f"{len(picks)} instances, max |p - p_ref| {worst:.2e} (same inputs {worst_same:.2e})")


def test_yolo26n_detect_batch2(hip):
    """YOLO26n detect (no Segment head), batch 2 at 320x320: the per-image
    selection of a batched head."""
    cfg = synth.config("n", arch="yolo26")
    params = synth.params_for_layout(synth.layout(cfg), seed=synth.SEED + 28, cls_bias=0.0)
    x = synth.images(2, 320, 320, seed=synth.SEED + 29)
    exp_head = oracle.yolo26_forward(params, x)
    with YoloDetector(cfg, params, ctx=hip) as det:
        for rep in range(2):
            print(f"YOLO26n B=2 320: device forward {rep}", flush=True)
            rows = det.predict_raw(x)
            assert rows.shape == (2, K, 6)
            hptr, (c, a) = det.head_buffer(2, 320, 320)
            head = hip.d2h(hptr, (2, c, a))
            assert max_rel(_raw(head, 320), _raw(exp_head, 320)) <= 1e-3
            np.testing.assert_array_equal(rows, oracle.e2e_select(head, K, NC))
            exp_rows = oracle.e2e_select(exp_head, K, NC)
            for b in range(2):
                _check_selection(rows[b], head[b], exp_rows[b], exp_head[b], K, 320)


def _raw_hw(head, h, w):
    """_raw for an h x w image: box distances in grid cells of each level."""
    cx, cy, st = [], [], []
    for s in (8, 16, 32):
        yy, xx = np.meshgrid(np.arange(h // s), np.arange(w // s), indexing="ij")
        cx.append(xx.ravel() + 0.5)
        cy.append(yy.ravel() + 0.5)
        st.append(np.full(xx.size, float(s)))
    cx, cy, st = np.concatenate(cx), np.concatenate(cy), np.concatenate(st)
    r = head.astype(np.float64).copy()
    r[..., 0, :] = cx - r[..., 0, :] / st
    r[..., 1, :] = cy - r[..., 1, :] / st
    r[..., 2, :] = r[..., 2, :] / st - cx
    r[..., 3, :] = r[..., 3, :] / st - cy
    return r


@pytest.mark.parametrize("batch,h,w", [(3, 32, 32), (2, 64, 96)])
def test_yolo26_fewer_anchors_than_k(hip, seg_model, batch, h, w):
    """Images with fewer anchors than the 300 rows kept (21 at 32x32, 126 at
    64x96): every anchor's best pair is selected, k = anchors.  The device
    selection with extras bit-exact against the oracle's selection on the
    device's own head; that head (boxes as grid distances) and the
    prototypes against the oracle's."""
    cfg, params = seg_model
    anchors = (h // 8) * (w // 8) + (h // 16) * (w // 16) + (h // 32) * (w // 32)
    x = synth.images(batch, h, w, seed=h + w + batch)
    with YoloDetector(cfg, params, ctx=hip) as det:
        assert det.output_shape(batch, h, w) == (batch, anchors, 6 + NM)
        rows, proto = det.predict_seg(x)
        hptr, (c, a) = det.head_buffer(batch, h, w)
        assert (c, a) == (NC + 4 + NM, anchors)
        head = hip.d2h(hptr, (batch, c, a))
    np.testing.assert_array_equal(rows, oracle.e2e_select(head, anchors, NC))
    exp_head, exp_proto = oracle.yolo26_forward(params, x, nm=NM, npr=256)
    assert max_rel(_raw_hw(head, h, w), _raw_hw(exp_head, h, w)) <= 1e-3
    assert max_rel(proto, exp_proto) <= 1e-3
