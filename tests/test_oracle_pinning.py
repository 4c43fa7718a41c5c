"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (dropped term,
wrong sign or index, transposed operand) fails it:
  * textbook ops against torch.nn.functional in this container (a third-party
    implementation, not the reference);
  * the reference's own known-answer tests (file:line cited per test);
  * invariants the mathematics fixes (closed forms, full-sort equivalence,
    parameter/FLOP counts published for the architecture).
"""
import math

import numpy as np
import pytest

import oracle
from _inputs import special_input

torch = pytest.importorskip("torch")
F = torch.nn.functional


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ------------------------------------------------------------------ conv


@pytest.mark.parametrize("n,c,h,w,oc,k,s,pad,dil,groups", [
    (2, 17, 9, 11, 19, 3, 1, (1, 1, 1, 1), 1, 1),   # Program.cs:210-221 shape
    (1, 3, 33, 31, 16, 3, 2, (1, 1, 1, 1), 1, 1),    # stem-like, odd sizes
    (2, 8, 16, 16, 12, 1, 1, (0, 0, 0, 0), 1, 1),    # pointwise
    (1, 6, 12, 10, 6, 3, 2, (2, 1, 0, 3), 2, 6),     # depthwise, asymmetric pads, dilation
    (1, 8, 10, 10, 4, 3, 1, (1, 1, 1, 1), 1, 2),     # grouped
])
@pytest.mark.parametrize("silu", [False, True])
def test_conv_matches_torch(n, c, h, w, oc, k, s, pad, dil, groups, silu):
    r = _rng(n * 100 + c)
    x = r.standard_normal((n, c, h, w)).astype(np.float32)
    wt = (r.standard_normal((oc, c // groups, k, k)) * 0.3).astype(np.float32)
    b = r.standard_normal(oc).astype(np.float32)
    y = oracle.conv2d(x, wt, b, (s, s), pad, (dil, dil), groups, silu)
    xt = F.pad(torch.from_numpy(x).double(), (pad[1], pad[3], pad[0], pad[2]))
    ref = F.conv2d(xt, torch.from_numpy(wt).double(), torch.from_numpy(b).double(), stride=s, dilation=dil,
                   groups=groups)
    if silu:
        ref = ref.float().double()
        ref = ref * torch.sigmoid(ref)
    np.testing.assert_allclose(y, ref.numpy(), rtol=2e-6, atol=2e-6)


def test_bn_fold_closed_form():
    # PtModel.cs:135-143.  mean 0, var 1 => b' = beta, w' = w * gamma / sqrt(1 + eps).
    r = _rng(3)
    w = r.standard_normal((4, 2, 3, 3)).astype(np.float32)
    g = r.uniform(0.5, 1.5, 4).astype(np.float32)
    beta = r.standard_normal(4).astype(np.float32)
    wo, bo = oracle.fold_bn(w, None, g, beta, np.zeros(4, np.float32), np.ones(4, np.float32), 1e-3)
    scale = g / np.sqrt(np.float32(1.0 + 1e-3), dtype=np.float32)
    np.testing.assert_array_equal(bo, beta)
    np.testing.assert_array_equal(wo, w * scale[:, None, None, None])
    # Non-trivial mean/var/conv-bias: matches the double formula to float rounding.
    mean = r.standard_normal(4).astype(np.float32)
    var = r.uniform(0.2, 3, 4).astype(np.float32)
    cb = r.standard_normal(4).astype(np.float32)
    wo, bo = oracle.fold_bn(w, cb, g, beta, mean, var, 1e-5)
    sc = g.astype(np.float64) / np.sqrt(var.astype(np.float64) + 1e-5)
    np.testing.assert_allclose(bo, beta + (cb - mean) * sc, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(wo, w * sc[:, None, None, None], rtol=1e-6)


# ------------------------------------------------------------------ pooling / resize


@pytest.mark.parametrize("stride", [1, 2])
def test_maxpool_matches_torch(stride):
    # Program.cs:135-148: kernel [5,3], pads [2,1,2,1] on sin(i) data.
    x = np.sin(np.arange(2 * 3 * 9 * 13, dtype=np.float32)).reshape(2, 3, 9, 13).astype(np.float32)
    y = oracle.maxpool(x, (5, 3), (stride, stride), (2, 1, 2, 1))
    ref = F.max_pool2d(torch.from_numpy(x), (5, 3), stride=stride, padding=(2, 1)).numpy()
    np.testing.assert_array_equal(y, ref)


def test_maxpool_ceil_and_sppf_chain():
    r = _rng(5)
    x = r.standard_normal((1, 4, 20, 20)).astype(np.float32)
    y = oracle.maxpool(x, (3, 3), (2, 2), (0, 0, 0, 0), ceil_mode=True)
    ref = F.max_pool2d(torch.from_numpy(x), 3, stride=2, ceil_mode=True).numpy()
    np.testing.assert_array_equal(y, ref)
    # Chained 5x5 pools == 9x9 / 13x13 windows (used by the fused SPPF kernel).
    p1 = oracle.maxpool(x, (5, 5), (1, 1), (2, 2, 2, 2))
    p2 = oracle.maxpool(p1, (5, 5), (1, 1), (2, 2, 2, 2))
    p3 = oracle.maxpool(p2, (5, 5), (1, 1), (2, 2, 2, 2))
    np.testing.assert_array_equal(p2, oracle.maxpool(x, (9, 9), (1, 1), (4, 4, 4, 4)))
    np.testing.assert_array_equal(p3, oracle.maxpool(x, (13, 13), (1, 1), (6, 6, 6, 6)))


@pytest.mark.parametrize("width", [3, 19])
def test_resize_nearest_reference_kat(width):
    # Program.cs:149-164: out[p][y][x] == in[p][y*7/h][x*width/w].
    x = (-np.arange(2 * 3 * 7 * width, dtype=np.float32) * 0.25).reshape(2, 3, 7, width)
    for h, w in [(14, 2 * width), (4, width + 3)]:
        y = oracle.resize_nearest(x, h, w)
        for yy in range(h):
            for xx in range(w):
                assert np.array_equal(y[:, :, yy, xx], x[:, :, yy * 7 // h, xx * width // w])
    up = oracle.resize_nearest(x, 14, 2 * width)
    np.testing.assert_array_equal(up, F.interpolate(torch.from_numpy(x), scale_factor=2, mode="nearest").numpy())


# ------------------------------------------------------------------ head decode


@pytest.mark.parametrize("width", [1, 3, 19, 80])
@pytest.mark.parametrize("bins", [1, 16])
@pytest.mark.parametrize("xyxy", [False, True])
def test_head_coordinates_reference_kat(width, bins, xyxy):
    # CpuHeadCoordinatesTests.cs:12-57: all-equal logits (0.2) give d = 7.5 for
    # 16 bins; 1 bin takes sin(a + side*.3 + b)*4 as the distance, bit-exact.
    batch, height, classes = 2, 3, 3
    spatial = width * height
    boxes = np.zeros((batch, 4 * bins, height, width), np.float32)
    for b in range(batch):
        for side in range(4):
            for r in range(bins):
                for a in range(spatial):
                    v = np.float32(math.sin(a + side * 0.3 + b) * 4) if bins == 1 else np.float32(0.2)
                    boxes[b, side * bins + r].flat[a] = v
    scores = np.zeros((batch, classes, height, width), np.float32)
    out = oracle.detect_decode([(boxes, scores, 8.0)], bins, xyxy)
    for b in range(batch):
        for a in range(spatial):
            def dist(side):
                return boxes[b, side * bins].flat[a] if bins == 1 else np.float32(7.5)
            f = np.float32
            cx, cy = f(a % width) + f(.5), f(a // width) + f(.5)
            x1, y1 = (cx - dist(0)) * f(8), (cy - dist(1)) * f(8)
            x2, y2 = (cx + dist(2)) * f(8), (cy + dist(3)) * f(8)
            exp = [x1, y1, x2, y2] if xyxy else [(x1 + x2) * f(.5), (y1 + y2) * f(.5), x2 - x1, y2 - y1]
            exp += [f(.5)] * classes
            got = out[b, :, a]
            if bins == 1:
                assert np.array_equal(got.view(np.uint32), np.array(exp, np.float32).view(np.uint32))
            else:
                np.testing.assert_allclose(got, np.array(exp, np.float32), rtol=2e-5, atol=2e-5)


def test_dfl_expectation_matches_softmax():
    # Program.cs:534-555: distance = sum(softmax(x) * r) over bins.
    r = _rng(9)
    boxes = r.standard_normal((1, 4 * 16, 2, 3)).astype(np.float32) * 3
    scores = r.standard_normal((1, 2, 2, 3)).astype(np.float32)
    out = oracle.detect_decode([(boxes, scores, 1.0)], 16, xyxy=True)
    t = torch.from_numpy(boxes).double().reshape(1, 4, 16, 6)
    d = (torch.softmax(t, 2) * torch.arange(16).double().reshape(1, 1, 16, 1)).sum(2)[0].numpy()
    cx = np.arange(6) % 3 + 0.5
    cy = np.arange(6) // 3 + 0.5
    np.testing.assert_allclose(out[0, 0], cx - d[0], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(out[0, 3], cy + d[3], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(out[0, 4:], 1 / (1 + np.exp(-scores.reshape(2, 6).astype(np.float64))), rtol=1e-6)


def test_yolo26_single_bin_kat():
    # Yolo26Tests.cs:45-48: a single-bin head takes the raw distances.
    boxes = np.array([1, 2, 3, 4], np.float32).reshape(1, 4, 1, 1)
    scores = np.zeros((1, 1, 1, 1), np.float32)
    out = oracle.detect_decode([(boxes, scores, 8.0)], 1, xyxy=True)
    np.testing.assert_array_equal(out[0, :4, 0], [(0.5 - 1) * 8, (0.5 - 2) * 8, (0.5 + 3) * 8, (0.5 + 4) * 8])


# ------------------------------------------------------------------ E2E top-k


def _net_max(a, b):
    # .NET MathF.Max: NaN propagates, +0 > -0.
    if a != b:
        if not math.isnan(a):
            return a if b < a else b
        return a
    return a if math.copysign(1.0, b) < 0 else b


def _desc_key_pt(score):
    # OrderByDescending with Single.CompareTo: NaN is the smallest value.
    return (1, 0.0) if math.isnan(score) else (0, -score)


def _full_sort_pt(x, maximum, classes):
    # CpuPtEndToEndTests.cs:93-121, as an independent full sort.
    batch, _, anchors = x.shape
    k = min(maximum, anchors)
    out = np.zeros((batch, k, 6), np.float32)
    for b in range(batch):
        maxima = [-math.inf] * anchors
        for c in range(classes):
            for a in range(anchors):
                maxima[a] = _net_max(maxima[a], float(x[b, 4 + c, a]))
        sel = sorted(range(anchors), key=lambda a: (_desc_key_pt(maxima[a]), a))[:k]
        cand = [(a, c, x[b, 4 + c, a]) for a in sel for c in range(classes)]
        cand.sort(key=lambda t: (_desc_key_pt(float(t[2])), t[0], t[1]))
        for i, (a, c, s) in enumerate(cand[:k]):
            out[b, i, :4] = x[b, :4, a]
            out[b, i, 4] = s
            out[b, i, 5] = c
    return out


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("classes", [1, 3, 7])
@pytest.mark.parametrize("anchors", [1, 7, 8, 9, 37])
@pytest.mark.parametrize("maximum", [1, 8, 49])
def test_e2e_pt_matches_full_sort(batch, classes, anchors, maximum):
    for frame in range(4):
        x = special_input(batch, classes, anchors, frame)
        got = oracle.e2e_select(x, maximum, classes)
        exp = _full_sort_pt(x, maximum, classes)
        assert got.shape == exp.shape
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (frame,)


def _full_sort_onnx(x, maximum, classes):
    # SelectOnnx semantics (CpuEndToEnd.cs:147-241): NaN first; ties by rank*C+c.
    batch, _, anchors = x.shape
    out = np.zeros((batch, maximum, 6), np.float32)

    def key(s):
        return (0, 0.0) if math.isnan(s) else (1, -s)
    for b in range(batch):
        maxima = [-math.inf] * anchors
        for c in range(classes):
            for a in range(anchors):
                maxima[a] = _net_max(maxima[a], float(x[b, 4 + c, a]))
        ranks = sorted(range(anchors), key=lambda a: (key(maxima[a]), a))[:maximum]
        cand = [(float(x[b, 4 + c, ranks[r]]), r * classes + c) for r in range(maximum) for c in range(classes)]
        cand.sort(key=lambda t: (key(t[0]), t[1]))
        for i, (s, idx) in enumerate(cand[:maximum]):
            a = ranks[idx // classes]
            out[b, i, :4] = x[b, :4, a]
            out[b, i, 4] = x[b, 4 + idx % classes, a]
            out[b, i, 5] = idx % classes
    return out


@pytest.mark.parametrize("classes,anchors,maximum", [(1, 9, 8), (3, 37, 8), (7, 37, 37), (5, 61, 17)])
def test_e2e_onnx_matches_full_sort(classes, anchors, maximum):
    for frame in range(4):
        x = special_input(2, classes, anchors, frame)
        got = oracle.e2e_select(x, maximum, classes, onnx=True)
        exp = _full_sort_onnx(x, maximum, classes)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_e2e_extras_gathered_at_anchor():
    r = _rng(11)
    x = r.standard_normal((1, 4 + 3 + 2, 50)).astype(np.float32)
    got = oracle.e2e_select(x, 10, 3)
    for row in got[0]:
        a = int(row[0]) if False else None
        idx = np.where((x[0, :4].T == row[:4]).all(1))[0]
        assert len(idx) == 1
        np.testing.assert_array_equal(row[6:], x[0, 7:, idx[0]])


# ------------------------------------------------------------------ NMS / letterbox


def test_nms_reference_kat():
    # Program.cs:227-234: class-aware NMS keeps 2 of 3; end-to-end skips NMS.
    out = np.array([10, 10, 10, 10, .9, .1, 10, 10, 10, 10, .8, .1, 10, 10, 10, 10, .1, .95], np.float32)
    tx = oracle.Letterbox(20, 20, 20, 20, 1.0, 1.0, 0, 0)
    dets = oracle.nms_decode(out.reshape(3, 6), layout=2, transform=tx)
    assert len(dets) == 2
    end = np.array([1, 1, 10, 10, .9, 0, 1, 1, 10, 10, .8, 0], np.float32).reshape(2, 6)
    assert len(oracle.nms_decode(end, layout=3, transform=tx)) == 2


def test_nms_greedy_against_brute_force():
    r = _rng(21)
    n, nc = 400, 4
    head = np.zeros((4 + nc, n), np.float32)
    head[0] = r.uniform(0, 600, n)
    head[1] = r.uniform(0, 600, n)
    head[2] = r.uniform(5, 120, n)
    head[3] = r.uniform(5, 120, n)
    head[4:] = r.uniform(0, 1, (nc, n))
    tx = oracle.Letterbox(640, 640, 640, 640, 1.0, 1.0, 0, 0)
    dets = oracle.nms_decode(head, layout=1, class_count=nc, transform=tx)
    # Independent greedy NMS in float64 box math (IoU computed the same way).
    conf = head[4:].max(0)
    cls = head[4:].argmax(0)
    keep = [a for a in range(n) if conf[a] >= 0.25]
    keep.sort(key=lambda a: -conf[a])
    boxes = {a: (head[0, a] - head[2, a] * 0.5, head[1, a] - head[3, a] * 0.5, head[2, a], head[3, a])
             for a in keep}

    def iou(p, q):
        w = max(0.0, min(p[0] + p[2], q[0] + q[2]) - max(p[0], q[0]))
        h = max(0.0, min(p[1] + p[3], q[1] + q[3]) - max(p[1], q[1]))
        i = w * h
        return i / max(1e-45, p[2] * p[3] + q[2] * q[3] - i)
    kept = []
    for a in keep:
        if any(cls[k] == cls[a] and iou(boxes[k], boxes[a]) > 0.45 for k in kept):
            continue
        kept.append(a)
        if len(kept) >= 300:
            break
    assert [d.anchor for d in dets] == kept


def test_letterbox_reference_kat():
    # Program.cs:222-226: 2x1 BGR image into 4x4 -> pad rows, value mapping.
    px = np.array([0, 0, 255, 0, 255, 0], np.uint8)
    out, t = oracle.letterbox(px, 2, 1, 4, 4, bgr=True)
    assert abs(out.flat[4] - 1) < 1e-6
    assert abs(out.flat[0] - 114 / 255) < 1e-6
    assert t.pad_y == 1


def test_letterbox_identity_at_network_size():
    r = _rng(4)
    img = r.integers(0, 256, (32, 48, 3), dtype=np.uint8)
    out, t = oracle.letterbox(img, 48, 32, 48, 32)
    np.testing.assert_array_equal(out[0], img.transpose(2, 0, 1).astype(np.float32) / np.float32(255))
    assert (t.pad_x, t.pad_y, t.scale_x, t.scale_y) == (0, 0, 1.0, 1.0)


# ------------------------------------------------------------------ topology


def _counts(layout):
    fused = sum(int(np.prod(e[1:5])) for e in layout if e[0] == 0)
    fused += sum(int(e[1]) for e in layout if e[0] in (2, 5, 6, 7))
    return fused + 16  # + the fixed DFL 1x1 conv


def _unfused(layout):
    # conv weights + BN gamma/beta + Conv2d biases + DFL (running stats are buffers)
    return sum(int(np.prod(e[1:5])) for e in layout if e[0] in (0, 1, 2, 5, 6, 7)) + 16


@pytest.mark.parametrize("scale,fused,unfused", [
    ((0.33, 0.25, 1024), 3151904, 3157200),     # YOLOv8n
    ((0.33, 0.50, 1024), 11156544, 11166560),   # YOLOv8s
    ((0.67, 0.75, 768), 25886080, 25902640),    # YOLOv8m
])
def test_yolov8_parameter_counts(scale, fused, unfused):
    # ultralytics' published model summaries (fused and unfused parameter counts).
    lay = oracle.yolov8_layout(*scale)
    assert _counts(lay) == fused
    assert _unfused(lay) == unfused


@pytest.mark.parametrize("fn,scale,unfused,fused", [
    # ultralytics' printed model summaries (parameters incl. the 16 fixed DFL weights)
    ("yolov8_layout", (0.33, 0.25, 1024), 3409968, 3404320),   # YOLOv8n-seg
    ("yolo11_layout", (0.50, 0.25, 1024), 2876848, 2868664),   # YOLO11n-seg
])
def test_segment_parameter_counts(fn, scale, unfused, fused):
    lay = getattr(oracle, fn)(*scale, nm=32, npr=256)
    assert _unfused(lay) == unfused
    assert _counts(lay) == fused


@pytest.mark.parametrize("fn,scale,millions", [
    # ultralytics' model tables (fused parameters, rounded to 0.1 M)
    ("yolov8_layout", (0.33, 0.50, 1024), 11.8), ("yolov8_layout", (0.67, 0.75, 768), 27.3),
    ("yolov8_layout", (1.00, 1.00, 512), 46.0), ("yolov8_layout", (1.00, 1.25, 512), 71.8),
    ("yolo11_layout", (0.50, 0.50, 1024), 10.1), ("yolo11_layout", (0.50, 1.00, 512), 22.4),
    ("yolo11_layout", (1.00, 1.00, 512), 27.6), ("yolo11_layout", (1.00, 1.50, 512), 62.1),
])
def test_segment_parameter_counts_rounded(fn, scale, millions):
    lay = getattr(oracle, fn)(*scale, nm=32, npr=256)
    assert round(_counts(lay) / 1e6, 1) == millions


def test_conv_transpose_matches_torch():
    r = np.random.Generator(np.random.PCG64(11))
    x = r.standard_normal((2, 12, 7, 5)).astype(np.float32)
    w = r.standard_normal((12, 20, 2, 2)).astype(np.float32)
    b = r.standard_normal(20).astype(np.float32)
    got = oracle.conv_transpose2x2(x, w, b)
    exp = F.conv_transpose2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                             torch.from_numpy(b).double(), stride=2).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)


def test_yolov8_segment_matches_torch_restatement():
    """YOLOv8n-seg at 64x64: head with appended mask coefficients and the
    Proto output against the torch restatement."""
    import simdyolo_amd.synth as S
    lay = oracle.yolov8_layout(nm=32, npr=256)
    params = S.params_for_layout(lay, seed=17)
    x = S.images(2, 64, 64, seed=18)
    got, proto = oracle.yolov8_forward(params, x, nm=32, npr=256)
    exp, exp_proto = _torch_yolov8(params, lay, x, nm=32, npr=256)
    assert got.shape == (2, 84 + 32, 84) and proto.shape == (2, 32, 16, 16)
    np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(proto, exp_proto, rtol=1e-4, atol=1e-4)


def test_yolov8_forward_matches_torch_restatement():
    """Whole-network cross-check at 64x64 against a torch.nn.functional
    restatement of yolov8.yaml (independent code path, double precision)."""
    import simdyolo_amd.synth as S  # only for the seeded parameter scheme
    lay = oracle.yolov8_layout()
    params = S.params_for_layout(lay, seed=7)
    x = S.images(2, 64, 64, seed=8)
    got = oracle.yolov8_forward(params, x)
    exp = _torch_yolov8(params, lay, x)
    np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-4)


def _torch_yolov8(params, lay, x, width=0.25, depth=0.33, max_ch=1024, nc=80, reg=16, eps=1e-3, nm=0, npr=256):
    it = iter(lay)
    pos = [0]

    def take(e):
        n = int(np.prod(e[1:5]))
        v = torch.from_numpy(params[pos[0]:pos[0] + n].astype(np.float64)).reshape(*[int(d) for d in e[1:5]])
        pos[0] += n
        return v

    def conv_mod():
        w = take(next(it)); g = take(next(it)).flatten(); b = take(next(it)).flatten()
        m = take(next(it)).flatten(); v = take(next(it)).flatten()
        s = g / torch.sqrt(v + eps)
        return ("c", w * s[:, None, None, None], b - m * s)

    def conv2d_mod():
        w = take(next(it)); b = take(next(it)).flatten()
        return ("p", w, b)

    def run(mod, t, stride=1):
        kind, w, b = mod
        y = F.conv2d(t, w, b, stride=stride, padding=w.shape[-1] // 2)
        return y * torch.sigmoid(y) if kind == "c" else y

    def ch(c):
        return int(math.ceil(min(c, max_ch) * width / 8) * 8)

    def rep(n):
        return max(round(n * depth), 1) if n > 1 else n

    def c2f_mods(n):
        cv1 = conv_mod(); cv2 = conv_mod()
        ms = [(conv_mod(), conv_mod()) for _ in range(n)]
        return cv1, cv2, ms

    def c2f(mods, t, add):
        cv1, cv2, ms = mods
        y = run(cv1, t)
        ys = list(y.chunk(2, 1))
        for a, b in ms:
            z = run(b, run(a, ys[-1]))
            ys.append(ys[-1] + z if add else z)
        return run(cv2, torch.cat(ys, 1))

    c = [ch(v) for v in (64, 128, 256, 512, 1024)]
    m0 = conv_mod(); m1 = conv_mod(); f2 = c2f_mods(rep(3)); m3 = conv_mod(); f4 = c2f_mods(rep(6))
    m5 = conv_mod(); f6 = c2f_mods(rep(6)); m7 = conv_mod(); f8 = c2f_mods(rep(3))
    s1 = conv_mod(); s2 = conv_mod()
    f12 = c2f_mods(rep(3)); f15 = c2f_mods(rep(3)); m16 = conv_mod(); f18 = c2f_mods(rep(3))
    m19 = conv_mod(); f21 = c2f_mods(rep(3))
    box = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    cls = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    if nm:
        pcv1 = conv_mod()
        up_w = take(next(it)); up_b = take(next(it)).flatten()
        pcv2 = conv_mod(); pcv3 = conv_mod()
        cv4 = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    assert pos[0] == params.size
    t = torch.from_numpy(x.astype(np.float64))
    l1 = run(m1, run(m0, t, 2), 2)
    l2 = c2f(f2, l1, True)
    l4 = c2f(f4, run(m3, l2, 2), True)
    l6 = c2f(f6, run(m5, l4, 2), True)
    l8 = c2f(f8, run(m7, l6, 2), True)
    a = run(s1, l8)
    p1 = F.max_pool2d(a, 5, 1, 2); p2 = F.max_pool2d(p1, 5, 1, 2); p3 = F.max_pool2d(p2, 5, 1, 2)
    l9 = run(s2, torch.cat([a, p1, p2, p3], 1))
    up = lambda z: F.interpolate(z, scale_factor=2, mode="nearest")
    l12 = c2f(f12, torch.cat([up(l9), l6], 1), False)
    l15 = c2f(f15, torch.cat([up(l12), l4], 1), False)
    l18 = c2f(f18, torch.cat([run(m16, l15, 2), l12], 1), False)
    l21 = c2f(f21, torch.cat([run(m19, l18, 2), l9], 1), False)
    outs = []
    for i, (feat, s) in enumerate(zip((l15, l18, l21), (8, 16, 32))):
        bx = run(box[i][2], run(box[i][1], run(box[i][0], feat)))
        cl = run(cls[i][2], run(cls[i][1], run(cls[i][0], feat)))
        B, _, h, w = bx.shape
        d = (torch.softmax(bx.reshape(B, 4, reg, h * w), 2) *
             torch.arange(reg, dtype=torch.float64).reshape(1, 1, reg, 1)).sum(2)
        gx = (torch.arange(h * w) % w).double() + 0.5
        gy = (torch.arange(h * w) // w).double() + 0.5
        x1, y1, x2, y2 = gx - d[:, 0], gy - d[:, 1], gx + d[:, 2], gy + d[:, 3]
        xywh = torch.stack([(x1 + x2) / 2, (y1 + y2) / 2, x2 - x1, y2 - y1], 1) * s
        outs.append(torch.cat([xywh, torch.sigmoid(cl.reshape(B, nc, h * w))], 1))
    head = torch.cat(outs, 2)
    if not nm:
        return head.numpy()
    proto = run(pcv3, run(pcv2, F.conv_transpose2d(run(pcv1, l15), up_w, up_b, stride=2)))
    mc = [run(cv4[i][2], run(cv4[i][1], run(cv4[i][0], f))).flatten(2) for i, f in enumerate((l15, l18, l21))]
    return torch.cat([head, torch.cat(mc, 2)], 1).numpy(), proto.numpy()


# ------------------------------------------------------------------ masks


def test_mask_reference_kat_all_ones_prototype():
    # Program.cs:235-240: all-ones prototypes, coefficients (20, 0) -> sigmoid(20) ~ 1.
    proto = np.ones((2, 4, 4), np.float32)
    tx = oracle.Letterbox(12, 12, 12, 12, 1.0, 1.0, 0, 0)
    out, info = oracle.mask_decode(proto, np.array([20, 0], np.float32), (2, 2, 4, 4), tx)
    assert info == (2, 2, 4, 4)
    assert abs(out[0, 0] - 1.0) < 1e-4


@pytest.mark.parametrize("cfg", [(257, 193, 13, 11), (19, 307, 9, 7), (101, 83, 17, 13)])
def test_mask_bilinear_exact_on_linear_prototype(cfg):
    """A prototype that is linear in (x, y) is reproduced exactly by bilinear
    sampling, so every probability has a closed form: sigmoid(a*px + b*py + c)
    at the half-pixel-mapped prototype coordinate (CpuMaskDecoder.cs:33-38)."""
    W, H, P, Q = cfg
    _, tr = oracle.letterbox(np.zeros((H, W, 3), np.uint8), W, H, 640, 640)
    a, b, c = 0.37, -0.21, 0.5
    xs, ys = np.meshgrid(np.arange(P, dtype=np.float64), np.arange(Q, dtype=np.float64))
    proto = (a * xs + b * ys + c)[None].astype(np.float32)
    box = (0.2, 1.4, W * 0.73, H * 0.61)
    out, (left, top, width, height) = oracle.mask_decode(proto, np.ones(1, np.float32), box, tr)
    assert (left, top) == (0, 1) and width == int(np.ceil(box[0] + box[2])) and height == int(np.ceil(box[1] + box[3])) - 1
    rl = min(max(int(round(tr.pad_x * P / 640)), 0), P - 1)
    rt = min(max(int(round(tr.pad_y * Q / 640)), 0), Q - 1)
    rr = min(max(int(round((tr.pad_x + W * tr.scale_x) * P / 640)), rl + 1), P)
    rb = min(max(int(round((tr.pad_y + H * tr.scale_y) * Q / 640)), rt + 1), Q)
    for y in range(top, top + height):
        for x in range(left, left + width):
            got = out[y - top, x - left]
            if x < np.ceil(box[0]) or y < np.ceil(box[1]):
                assert got == 0.0
                continue
            px = np.clip(np.float32(rl) + (np.float32(x) + np.float32(.5)) * np.float32(rr - rl) / np.float32(W) - np.float32(.5), rl, rr - 1)
            py = np.clip(np.float32(rt) + (np.float32(y) + np.float32(.5)) * np.float32(rb - rt) / np.float32(H) - np.float32(.5), rt, rb - 1)
            exp = 1 / (1 + np.exp(-(a * float(px) + b * float(py) + c)))
            assert abs(got - exp) < 2e-6, (x, y, got, exp)


@pytest.mark.parametrize("scale,fused,unfused", [
    ((0.50, 0.25, 1024), 2616248, 2624080),     # YOLO11n
    ((0.50, 0.50, 1024), 9443760, 9458752),     # YOLO11s
    ((0.50, 1.00, 512), 20091712, 20114688),    # YOLO11m (all C3k2 use C3k)
    ((1.00, 1.00, 512), 25340992, 25372160),    # YOLO11l
    ((1.00, 1.50, 512), 56919424, 56966176),    # YOLO11x
])
def test_yolo11_parameter_counts(scale, fused, unfused):
    # ultralytics' published YOLO11 model summaries.
    lay = oracle.yolo11_layout(*scale)
    assert _counts(lay) == fused
    assert _unfused(lay) == unfused


def test_yolo11_segment_matches_torch_restatement():
    import simdyolo_amd.synth as S
    lay = oracle.yolo11_layout(nm=32, npr=256)
    params = S.params_for_layout(lay, seed=19)
    x = S.images(1, 128, 128, seed=20)
    got, proto = oracle.yolo11_forward(params, x, nm=32, npr=256)
    exp, exp_proto = _torch_yolo11(params, lay, x, nm=32, npr=256)
    np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(proto, exp_proto, rtol=1e-4, atol=1e-4)


def test_yolo11_forward_matches_torch_restatement():
    """YOLO11n at 128x128 (16 attention tokens at P5) against an independent
    torch.nn.functional restatement of yolo11.yaml in double precision."""
    import simdyolo_amd.synth as S
    lay = oracle.yolo11_layout()
    params = S.params_for_layout(lay, seed=9)
    x = S.images(2, 128, 128, seed=10)
    got = oracle.yolo11_forward(params, x)
    exp = _torch_yolo11(params, lay, x)
    np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-4)


def _torch_yolo11(params, lay, x, width=0.25, depth=0.50, max_ch=1024, nc=80, reg=16, eps=1e-3, nm=0, npr=256):
    it = iter(lay)
    pos = [0]

    def take(e):
        n = int(np.prod(e[1:5]))
        v = torch.from_numpy(params[pos[0]:pos[0] + n].astype(np.float64)).reshape(*[int(d) for d in e[1:5]])
        pos[0] += n
        return v

    def conv_mod(act=True, groups=1):
        w = take(next(it)); g = take(next(it)).flatten(); b = take(next(it)).flatten()
        m = take(next(it)).flatten(); v = take(next(it)).flatten()
        s = g / torch.sqrt(v + eps)
        return (act, w * s[:, None, None, None], b - m * s, groups)

    def conv2d_mod():
        w = take(next(it)); b = take(next(it)).flatten()
        return (False, w, b, 1)

    def run(mod, t, stride=1):
        act, w, b, g = mod
        y = F.conv2d(t, w, b, stride=stride, padding=w.shape[-1] // 2, groups=g)
        return y * torch.sigmoid(y) if act else y

    def ch(c):
        return int(math.ceil(min(c, max_ch) * width / 8) * 8)

    def rep(n):
        return max(round(n * depth), 1) if n > 1 else n

    def bneck_mods():
        return (conv_mod(), conv_mod())

    def bneck(mods, t):
        return t + run(mods[1], run(mods[0], t))

    def c3k_mods():
        return (conv_mod(), conv_mod(), conv_mod(), [bneck_mods() for _ in range(2)])

    def c3k(mods, t):
        cv1, cv2, cv3, ms = mods
        a = run(cv1, t)
        for b in ms:
            a = bneck(b, a)
        return run(cv3, torch.cat([a, run(cv2, t)], 1))

    def c3k2_mods(n, c3k_):
        cv1 = conv_mod(); cv2 = conv_mod()
        return cv1, cv2, [(c3k_, c3k_mods() if c3k_ else bneck_mods()) for _ in range(n)]

    def c3k2(mods, t):
        cv1, cv2, ms = mods
        ys = list(run(cv1, t).chunk(2, 1))
        for is_c3k, m in ms:
            ys.append(c3k(m, ys[-1]) if is_c3k else bneck(m, ys[-1]))
        return run(cv2, torch.cat(ys, 1))

    def attn_mods(c):
        return (conv_mod(False), conv_mod(False), conv_mod(False, groups=c))

    def attention(mods, t, heads):
        qkv_m, proj_m, pe_m = mods
        B, C, H, W = t.shape
        N = H * W
        hd = C // heads
        kd = hd // 2
        qkv = run(qkv_m, t).view(B, heads, 2 * kd + hd, N)
        q, k, v = qkv.split([kd, kd, hd], dim=2)
        a = (q.transpose(-2, -1) @ k) * (kd ** -0.5)
        a = a.softmax(dim=-1)
        o = (v @ a.transpose(-2, -1)).view(B, C, H, W) + run(pe_m, v.reshape(B, C, H, W))
        return run(proj_m, o)

    c = [ch(v) for v in (64, 128, 256, 512, 1024)]
    n2 = rep(2)
    m0 = conv_mod(); m1 = conv_mod(); f2 = c3k2_mods(n2, False); m3 = conv_mod(); f4 = c3k2_mods(n2, False)
    m5 = conv_mod(); f6 = c3k2_mods(n2, True); m7 = conv_mod(); f8 = c3k2_mods(n2, True)
    s1 = conv_mod(); s2 = conv_mod()
    p_cv1 = conv_mod(); p_cv2 = conv_mod()
    psa = [(attn_mods(c[4] // 2), conv_mod(), conv_mod(False)) for _ in range(n2)]
    f13 = c3k2_mods(n2, False); f16 = c3k2_mods(n2, False); m17 = conv_mod(); f19 = c3k2_mods(n2, False)
    m20 = conv_mod(); f22 = c3k2_mods(n2, True)
    box = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    feats_c = (c[2], c[3], c[4])
    cls = [[conv_mod(groups=feats_c[i]), conv_mod(), conv_mod(groups=80), conv_mod(), conv2d_mod()] for i in range(3)]
    if nm:
        pcv1 = conv_mod()
        up_w = take(next(it)); up_b = take(next(it)).flatten()
        pcv2 = conv_mod(); pcv3 = conv_mod()
        cv4 = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    assert pos[0] == params.size
    t = torch.from_numpy(x.astype(np.float64))
    l2 = c3k2(f2, run(m1, run(m0, t, 2), 2))
    l4 = c3k2(f4, run(m3, l2, 2))
    l6 = c3k2(f6, run(m5, l4, 2))
    l8 = c3k2(f8, run(m7, l6, 2))
    a = run(s1, l8)
    p1 = F.max_pool2d(a, 5, 1, 2); p2 = F.max_pool2d(p1, 5, 1, 2); p3 = F.max_pool2d(p2, 5, 1, 2)
    l9 = run(s2, torch.cat([a, p1, p2, p3], 1))
    ya, yb = run(p_cv1, l9).chunk(2, 1)
    for att, f0, f1 in psa:
        yb = yb + attention(att, yb, yb.shape[1] // 64)
        yb = yb + run(f1, run(f0, yb))
    l10 = run(p_cv2, torch.cat([ya, yb], 1))
    up = lambda z: F.interpolate(z, scale_factor=2, mode="nearest")
    l13 = c3k2(f13, torch.cat([up(l10), l6], 1))
    l16 = c3k2(f16, torch.cat([up(l13), l4], 1))
    l19 = c3k2(f19, torch.cat([run(m17, l16, 2), l13], 1))
    l22 = c3k2(f22, torch.cat([run(m20, l19, 2), l10], 1))
    outs = []
    for i, (feat, s) in enumerate(zip((l16, l19, l22), (8, 16, 32))):
        bx = run(box[i][2], run(box[i][1], run(box[i][0], feat)))
        cl = feat
        for mod in cls[i]:
            cl = run(mod, cl)
        B, _, h, w = bx.shape
        d = (torch.softmax(bx.reshape(B, 4, reg, h * w), 2) *
             torch.arange(reg, dtype=torch.float64).reshape(1, 1, reg, 1)).sum(2)
        gx = (torch.arange(h * w) % w).double() + 0.5
        gy = (torch.arange(h * w) // w).double() + 0.5
        x1, y1, x2, y2 = gx - d[:, 0], gy - d[:, 1], gx + d[:, 2], gy + d[:, 3]
        xywh = torch.stack([(x1 + x2) / 2, (y1 + y2) / 2, x2 - x1, y2 - y1], 1) * s
        outs.append(torch.cat([xywh, torch.sigmoid(cl.reshape(B, nc, h * w))], 1))
    head = torch.cat(outs, 2)
    if not nm:
        return head.numpy()
    proto = run(pcv3, run(pcv2, F.conv_transpose2d(run(pcv1, l16), up_w, up_b, stride=2)))
    mc = [run(cv4[i][2], run(cv4[i][1], run(cv4[i][0], f))).flatten(2) for i, f in enumerate((l16, l19, l22))]
    return torch.cat([head, torch.cat(mc, 2)], 1).numpy(), proto.numpy()


@pytest.mark.parametrize("h,w,k,st,pads,oh,ow", [(4, 34, 3, 2, (0, 0, 0, 0), 2, 17), (5, 33, 2, 2, (1, 1, 1, 1), 3, 17),
                                               (2, 35, 3, 2, (0, 0, 0, 0), 1, 17), (4, 36, 3, 2, (0, 1, 1, 0), 2, 18)])
def test_maxpool_ceil_mode_reference_cases(h, w, k, st, pads, oh, ow):
    """MaxPoolCeilTests.cs:13-19: the reference's output sizes, and its expected
    values (the max over in-image taps only) by brute force."""
    x = (-1.0 - ((np.arange(2 * 2 * h * w) * 73) % 257)).astype(np.float32).reshape(2, 2, h, w)
    got = oracle.maxpool(x, (k, k), (st, st), pads, ceil_mode=True)
    assert got.shape == (2, 2, oh, ow)
    ref = np.full((2, 2, oh, ow), -np.inf, np.float32)
    for y in range(oh):
        for xx in range(ow):
            for ky in range(k):
                for kx in range(k):
                    sy, sx = y * st + ky - pads[0], xx * st + kx - pads[1]
                    if 0 <= sy < h and 0 <= sx < w:
                        ref[:, :, y, xx] = np.maximum(ref[:, :, y, xx], x[:, :, sy, sx])
    np.testing.assert_array_equal(got, ref)


# YOLO26 (ultralytics yolo26.yaml / yolo26-seg.yaml, end-to-end).  The model
# summaries count every parameter of the training graph: besides the branches
# inference runs (one2one_cv2 / one2one_cv3 / one2one_cv4, which the layout
# lists), the one-to-many copies cv2 / cv3 / cv4 of identical shapes and the
# training-only Proto26.semseg = Conv(ch0, c_, 3), Conv(c_, c_, 3),
# Conv2d(c_, nc, 1).  reg_max 1 makes DFL an Identity (no weights).
_Y26_HEAD_ENTRIES = 3 * (12 + 22)   # per level box 5+5+2, class 5+5+5+5+2 entries
_Y26_PROTO_ENTRIES = 5 + 2 + 5 + 5 + 10 + 5   # cv1, upsample, cv2, cv3, feat_refine x2, feat_fuse
_Y26_CV4_ENTRIES = 3 * (5 + 5 + 2)


def _trainable(entries):
    return sum(int(np.prod(e[1:5])) for e in entries if e[0] in (0, 1, 2, 5, 6, 7))


@pytest.mark.parametrize("nm,published", [(0, 2572280), (32, 3126280)])
def test_yolo26_parameter_counts(nm, published):
    lay = oracle.yolo26_layout(nm=nm, npr=256)
    tail = _Y26_PROTO_ENTRIES + _Y26_CV4_ENTRIES if nm else 0
    head = lay[len(lay) - tail - _Y26_HEAD_ENTRIES:len(lay) - tail]
    extra = _trainable(head)
    if nm:
        extra += _trainable(lay[-_Y26_CV4_ENTRIES:])
        c0, c_, nc = 64, 64, 80   # P3 width and Proto width at the n scale
        extra += (c_ * c0 * 9 + 2 * c_) + (c_ * c_ * 9 + 2 * c_) + (nc * c_ + nc)
    assert _trainable(lay) + extra == published


@pytest.mark.parametrize("nm,batch", [(0, 2), (32, 1)])
def test_yolo26_forward_matches_torch_restatement(nm, batch):
    """YOLO26n(-seg) at 128x128 against an independent torch.nn.functional
    restatement of yolo26.yaml / yolo26-seg.yaml in double precision."""
    import simdyolo_amd.synth as S
    lay = oracle.yolo26_layout(nm=nm, npr=256)
    params = S.params_for_layout(lay, seed=29 + nm)
    x = S.images(batch, 128, 128, seed=30)
    if nm:
        got, proto = oracle.yolo26_forward(params, x, nm=nm, npr=256)
        exp, exp_proto = _torch_yolo26(params, lay, x, nm=nm)
        np.testing.assert_allclose(proto, exp_proto, rtol=1e-4, atol=1e-4)
    else:
        got = oracle.yolo26_forward(params, x)
        exp = _torch_yolo26(params, lay, x)
    np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-4)


def _torch_yolo26(params, lay, x, width=0.25, depth=0.50, max_ch=1024, nc=80, eps=1e-3, nm=0, npr=256):
    it = iter(lay)
    pos = [0]

    def take(e):
        n = int(np.prod(e[1:5]))
        v = torch.from_numpy(params[pos[0]:pos[0] + n].astype(np.float64)).reshape(*[int(d) for d in e[1:5]])
        pos[0] += n
        return v

    def conv_mod(act=True, groups=1):
        w = take(next(it)); g = take(next(it)).flatten(); b = take(next(it)).flatten()
        m = take(next(it)).flatten(); v = take(next(it)).flatten()
        s = g / torch.sqrt(v + eps)
        return (act, w * s[:, None, None, None], b - m * s, groups)

    def conv2d_mod():
        w = take(next(it)); b = take(next(it)).flatten()
        return (False, w, b, 1)

    def run(mod, t, stride=1):
        act, w, b, g = mod
        y = F.conv2d(t, w, b, stride=stride, padding=w.shape[-1] // 2, groups=g)
        return y * torch.sigmoid(y) if act else y

    def ch(c):
        return int(math.ceil(min(c, max_ch) * width / 8) * 8)

    def rep(n):
        return max(round(n * depth), 1) if n > 1 else n

    def bneck(mods, t):
        return t + run(mods[1], run(mods[0], t))

    def c3k(mods, t):
        cv1, cv2, cv3, ms = mods
        a = run(cv1, t)
        for b in ms:
            a = bneck(b, a)
        return run(cv3, torch.cat([a, run(cv2, t)], 1))

    def attention(mods, t, heads):
        qkv_m, proj_m, pe_m = mods
        B, C, H, W = t.shape
        N = H * W
        hd = C // heads
        kd = hd // 2
        q, k, v = run(qkv_m, t).view(B, heads, 2 * kd + hd, N).split([kd, kd, hd], dim=2)
        a = ((q.transpose(-2, -1) @ k) * (kd ** -0.5)).softmax(dim=-1)
        o = (v @ a.transpose(-2, -1)).view(B, C, H, W) + run(pe_m, v.reshape(B, C, H, W))
        return run(proj_m, o)

    def psa_mods(c):
        return ((conv_mod(False), conv_mod(False), conv_mod(False, groups=c)), conv_mod(), conv_mod(False))

    def psa(mods, t):
        att, f0, f1 = mods
        t = t + attention(att, t, max(t.shape[1] // 64, 1))
        return t + run(f1, run(f0, t))

    # kind: "b" Bottleneck(e=0.5), "k" C3k(n=2), "a" Bottleneck then PSABlock
    def c3k2_mods(n, kind, c):
        cv1 = conv_mod(); cv2 = conv_mod()
        ms = []
        for _ in range(n):
            if kind == "k":
                ms.append((kind, (conv_mod(), conv_mod(), conv_mod(), [(conv_mod(), conv_mod()) for _ in range(2)])))
            elif kind == "a":
                ms.append((kind, ((conv_mod(), conv_mod()), psa_mods(c))))
            else:
                ms.append((kind, (conv_mod(), conv_mod())))
        return cv1, cv2, ms

    def c3k2(mods, t):
        cv1, cv2, ms = mods
        ys = list(run(cv1, t).chunk(2, 1))
        for kind, m in ms:
            y = ys[-1]
            if kind == "k":
                y = c3k(m, y)
            elif kind == "a":
                y = psa(m[1], bneck(m[0], y))
            else:
                y = bneck(m, y)
            ys.append(y)
        return run(cv2, torch.cat(ys, 1))

    c = [ch(v) for v in (64, 128, 256, 512, 1024)]
    n2 = rep(2)
    m0 = conv_mod(); m1 = conv_mod(); f2 = c3k2_mods(n2, "b", 0); m3 = conv_mod(); f4 = c3k2_mods(n2, "b", 0)
    m5 = conv_mod(); f6 = c3k2_mods(n2, "k", 0); m7 = conv_mod(); f8 = c3k2_mods(n2, "k", 0)
    s1 = conv_mod(False); s2 = conv_mod()
    p_cv1 = conv_mod(); p_cv2 = conv_mod()
    psa10 = [psa_mods(c[4] // 2) for _ in range(n2)]
    f13 = c3k2_mods(n2, "k", 0); f16 = c3k2_mods(n2, "k", 0); m17 = conv_mod(); f19 = c3k2_mods(n2, "k", 0)
    m20 = conv_mod(); f22 = c3k2_mods(rep(1), "a", c[4] // 2)
    box = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    feats_c = (c[2], c[3], c[4])
    c3w = max(feats_c[0], min(nc, 100))
    cls = [[conv_mod(groups=feats_c[i]), conv_mod(), conv_mod(groups=c3w), conv_mod(), conv2d_mod()] for i in range(3)]
    if nm:
        pcv1 = conv_mod()
        up_w = take(next(it)); up_b = take(next(it)).flatten()
        pcv2 = conv_mod(); pcv3 = conv_mod()
        refine = [conv_mod(), conv_mod()]
        fuse = conv_mod()
        cv4 = [[conv_mod(), conv_mod(), conv2d_mod()] for _ in range(3)]
    assert pos[0] == params.size
    t = torch.from_numpy(x.astype(np.float64))
    l2 = c3k2(f2, run(m1, run(m0, t, 2), 2))
    l4 = c3k2(f4, run(m3, l2, 2))
    l6 = c3k2(f6, run(m5, l4, 2))
    l8 = c3k2(f8, run(m7, l6, 2))
    a = run(s1, l8)
    p1 = F.max_pool2d(a, 5, 1, 2); p2 = F.max_pool2d(p1, 5, 1, 2); p3 = F.max_pool2d(p2, 5, 1, 2)
    l9 = run(s2, torch.cat([a, p1, p2, p3], 1)) + l8
    ya, yb = run(p_cv1, l9).chunk(2, 1)
    for m in psa10:
        yb = psa(m, yb)
    l10 = run(p_cv2, torch.cat([ya, yb], 1))
    up = lambda z, f=2: F.interpolate(z, scale_factor=f, mode="nearest")
    l13 = c3k2(f13, torch.cat([up(l10), l6], 1))
    l16 = c3k2(f16, torch.cat([up(l13), l4], 1))
    l19 = c3k2(f19, torch.cat([run(m17, l16, 2), l13], 1))
    l22 = c3k2(f22, torch.cat([run(m20, l19, 2), l10], 1))
    outs = []
    for i, (feat, s) in enumerate(zip((l16, l19, l22), (8, 16, 32))):
        d = run(box[i][2], run(box[i][1], run(box[i][0], feat)))
        cl = feat
        for mod in cls[i]:
            cl = run(mod, cl)
        B, _, h, w = d.shape
        d = d.reshape(B, 4, h * w)
        gx = (torch.arange(h * w) % w).double() + 0.5
        gy = (torch.arange(h * w) // w).double() + 0.5
        xyxy = torch.stack([gx - d[:, 0], gy - d[:, 1], gx + d[:, 2], gy + d[:, 3]], 1) * s
        outs.append(torch.cat([xyxy, torch.sigmoid(cl.reshape(B, nc, h * w))], 1))
    head = torch.cat(outs, 2)
    if not nm:
        return head.numpy()
    r = l16 + up(run(refine[0], l19), 2) + up(run(refine[1], l22), 4)
    proto = run(pcv3, run(pcv2, F.conv_transpose2d(run(pcv1, run(fuse, r)), up_w, up_b, stride=2)))
    mc = [run(cv4[i][2], run(cv4[i][1], run(cv4[i][0], f))).flatten(2) for i, f in enumerate((l16, l19, l22))]
    return torch.cat([head, torch.cat(mc, 2)], 1).numpy(), proto.numpy()
