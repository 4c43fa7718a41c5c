"""numpy restatement of the reference's generic device ops (shaders/tensor.comp)
and of its batched device matrix product (VulkanExecution.cs:499-541).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP
``sy_compute`` / ``sy_matmul`` entry points.  The shipped package never
imports it.

``run(op, a, b, d, params, out_len, out)`` evaluates one dispatch: work item i in
[0, P(0)) computes what tensor.comp's ``main`` computes for
gl_GlobalInvocationID.x == i, with A/B/C/D(k) addressing element k + P(28..31)
of the bound buffers.  Elements of the output that no work item writes keep
their value in ``out`` (zeros when it is None).  Each branch cites
the shader lines it follows.  Vectorised over work items with int64 index
arithmetic; sums over kernel taps run in float64, so the device result is
compared within a stated tolerance, not bit for bit, for ops that add.

Pinned in tests/test_tensor_ops_cpu.py against library routines (torch.nn
functional ops, numpy broadcasting, transposes, pixel shuffle, softmax) on
parameter blocks built as the reference's DeviceOps builds them
(src/SimdYolo/DeviceExecution.cs:107-190) and as its callers do.
"""
from __future__ import annotations

import numpy as np


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x.astype(np.float64)))


def _f(u):
    return np.array([u], np.uint32).view(np.float32)[0].astype(np.float64)


def run(op: int, a, b, d, params, out_len: int, out=None) -> np.ndarray:
    P = [int(v) for v in params] + [0] * (32 - len(params))
    # Slot 27 flags a bound bias input (VulkanExecution.cs:265).
    P[27] = 0 if d is None else 1
    n = P[0]
    i = np.arange(n, dtype=np.int64)
    c = np.zeros(out_len, np.float64) if out is None else np.asarray(out, np.float64).reshape(-1).copy()
    A = lambda k: np.asarray(a, np.float64)[np.asarray(k, np.int64) + P[28]]
    B = lambda k: np.asarray(b, np.float64)[np.asarray(k, np.int64) + P[29]]
    D = lambda k: np.asarray(d, np.float64)[np.asarray(k, np.int64) + P[31]]

    def C(k, v):
        c[np.asarray(k, np.int64) + P[30]] = v

    if op < 10:  # tensor.comp:18-29
        x = A(i)
        # The shader computes in FP32; round the input once so exp/sqrt/sigmoid
        # are evaluated on the same value.
        y = {1: lambda: x * _sigmoid(x), 2: lambda: _sigmoid(x), 3: lambda: np.maximum(x, 0),
             4: lambda: x * _f(P[1]), 5: lambda: np.exp(x), 6: lambda: np.sqrt(x), 7: lambda: -x,
             8: lambda: np.abs(x), 9: lambda: np.where(x >= 0, x, x * _f(P[1]))}[op]()
        C(i, y)
    elif op < 20:  # tensor.comp:30-41
        t, ai, bi = i.copy(), np.zeros_like(i), np.zeros_like(i)
        for j in range(3, -1, -1):
            coord = t % P[1 + j]
            t //= P[1 + j]
            ai += coord * P[5 + j]
            bi += coord * P[9 + j]
        x, y = A(ai), B(bi)
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            r = {10: x + y, 11: x - y, 12: x * y, 13: x / y, 14: np.power(x, y), 15: np.maximum(x, y),
                 16: np.minimum(x, y)}[op]
        C(i, r)
    elif op == 20:  # tensor.comp:42-44, nearest resize
        plane = P[3] * P[4]
        ch, oy, ox = i // plane, i % plane // P[4], i % P[4]
        C(i, A((ch * P[1] + oy * P[1] // P[3]) * P[2] + ox * P[2] // P[4]))
    elif op in (21, 22):  # tensor.comp:45-54, max / average pool
        h, w, oh, ow, kh, kw = P[1:7]
        plane = oh * ow
        ch, oy, ox = i // plane, i % plane // ow, i % ow
        sy, sx = oy * P[7] - P[9], ox * P[8] - P[10]
        v = np.full(n, -np.inf) if op == 21 else np.zeros(n)
        count = np.zeros(n, np.int64)
        for ky in range(kh):
            for kx in range(kw):
                y, x = sy + ky, sx + kx
                ok = (y >= 0) & (x >= 0) & (y < h) & (x < w)
                e = np.where(ok, A(np.where(ok, (ch * h + y) * w + x, -P[28])), 0.0)
                v = np.where(ok, np.maximum(v, e) if op == 21 else v + e, v)
                count += ok
        C(i, v if op == 21 else v / (kh * kw if P[11] == 1 else count))
    elif op == 23:  # tensor.comp:55-58, transpose by input strides
        t, src = i.copy(), np.zeros_like(i)
        for j in range(3, -1, -1):
            src += t % P[1 + j] * P[5 + j]
            t //= P[1 + j]
        C(i, A(src))
    elif op == 24:  # tensor.comp:59-61, slice
        inner = P[3]
        outer, rem = i // (P[2] * inner), i % (P[2] * inner)
        C(i, A(outer * P[1] * inner + P[4] * inner + rem))
    elif op == 25:  # tensor.comp:62-67, softmax along an axis, one work item per row
        size, inner = P[1], P[2]
        base = i // inner * size * inner + i % inner
        rows = np.stack([A(base + j * inner) for j in range(size)], 1)
        e = np.exp(rows - rows.max(1, keepdims=True))
        y = e / e.sum(1, keepdims=True)
        for j in range(size):
            C(base + j * inner, y[:, j])
    elif op == 26:  # tensor.comp:68-70, concat write
        size = P[1] * P[3]
        C(i // size * P[2] * P[3] + P[4] * P[3] + i % size, A(i))
    elif op in (30, 34):  # tensor.comp:71-89 (30) and 107-112 (34)
        spatial = P[1]
        bins = P[3] if op == 30 else P[2]

        def dfl(base):
            if bins == 1:
                return A(base)
            rows = np.stack([A(base + j * spatial) for j in range(bins)], 1)
            e = np.exp(rows - rows.max(1, keepdims=True))
            return (e * np.arange(bins)).sum(1) / e.sum(1)

        if op == 34:
            C(i, dfl(i // spatial * bins * spatial + i % spatial))
        else:
            width, nc = P[2], P[4]
            batch, anchor = i // spatial, i % spatial
            dist = [dfl((batch * 4 + s) * bins * spatial + anchor) for s in range(4)]
            stride = _f(P[5])
            cx, cy = (anchor % width) + 0.5, (anchor // width) + 0.5
            x1, y1 = (cx - dist[0]) * stride, (cy - dist[1]) * stride
            x2, y2 = (cx + dist[2]) * stride, (cy + dist[3]) * stride
            os_ = spatial if P[7] == 0 else P[7]
            dst = batch * (nc + 4) * os_ + P[8] + anchor
            xyxy = P[6] == 1
            C(dst, x1 if xyxy else (x1 + x2) * 0.5)
            C(dst + os_, y1 if xyxy else (y1 + y2) * 0.5)
            C(dst + 2 * os_, x2 if xyxy else x2 - x1)
            C(dst + 3 * os_, y2 if xyxy else y2 - y1)
            for j in range(nc):
                C(dst + (4 + j) * os_, _sigmoid(B((batch * nc + j) * spatial + anchor)))
    elif op == 31:  # tensor.comp:90-94, pose keypoints
        spatial, width, dim = P[1], P[2], P[3]
        axis, anchor = i // spatial % dim, i % spatial
        v, stride = A(i), _f(P[4])
        factor, offset = (1.0, 0.5) if P[5] == 1 else (2.0, 0.0)
        C(i, np.where(axis == 0, (v * factor + (anchor % width + offset)) * stride,
                      np.where(axis == 1, (v * factor + (anchor // width + offset)) * stride, _sigmoid(v))))
    elif op == 32:  # tensor.comp:95-103, depthwise conv
        ic, ih, iw = P[1:4]
        oh, ow, kh, kw = P[5:9]
        spatial = oh * ow
        bc = i // spatial
        ch, oy, ox = bc % ic, i % spatial // ow, i % ow
        v = D(ch) if P[27] == 1 else np.zeros(n)
        for ky in range(kh):
            for kx in range(kw):
                y = oy * P[9] - P[11] + ky * P[13]
                x = ox * P[10] - P[12] + kx * P[14]
                ok = (y >= 0) & (x >= 0) & (y < ih) & (x < iw)
                e = np.where(ok, A(np.where(ok, (bc * ih + y) * iw + x, -P[28])), 0.0)
                v = v + e * B((ch * kh + ky) * kw + kx)
        C(i, v * _sigmoid(v) if P[16] == 1 else v)
    elif op == 33:  # tensor.comp:135-150, transposed conv, weights [ic][oc/groups][kh][kw]
        ic, ih, iw, oc, oh, ow, kh, kw = P[1:9]
        groups = P[15]
        spatial = oh * ow
        co, batch = i // spatial % oc, i // (spatial * oc)
        cog, cig = oc // groups, ic // groups
        grp, oy, ox = co // cog, i % spatial // ow, i % ow
        v = D(co) if P[27] == 1 else np.zeros(n)
        for ky in range(kh):
            for kx in range(kw):
                yn = oy + P[11] - ky * P[13]
                xn = ox + P[12] - kx * P[14]
                ok = (yn >= 0) & (xn >= 0) & (yn % P[9] == 0) & (xn % P[10] == 0)
                y, x = yn // P[9], xn // P[10]
                ok &= (y < ih) & (x < iw)
                for q in range(cig):
                    ci = grp * cig + q
                    e = np.where(ok, A(np.where(ok, ((batch * ic + ci) * ih + y) * iw + x, -P[28])), 0.0)
                    v = v + e * B(((ci * cog + co % cog) * kh + ky) * kw + kx)
        C(i, v)
    elif op == 35:  # tensor.comp:104-106, depth to space by 2
        h, w, channels = P[1:4]
        plane = h * w
        co, batch, y, x = i // plane % channels, i // (plane * channels), i % plane // w, i % w
        C(i, A(((batch * channels * 4 + co * 4 + y % 2 * 2 + x % 2) * (h // 2) + y // 2) * (w // 2) + x // 2))
    elif op == 36:  # tensor.comp:113-123, row maximum with MathF.Max semantics
        size = P[1]
        rows = np.stack([A(i * size + j) for j in range(size)], 1) if n else np.zeros((0, size))
        out = np.empty(n)
        for r in range(n):
            m = -np.inf
            for v in rows[r]:
                if np.isnan(v):
                    m = v
                    break
                if v > m or (v == 0.0 and m == 0.0 and not np.signbit(v)):
                    m = v
            out[r] = m
        C(i, out)
    elif op == 37:  # tensor.comp:124-134, gather along axis P(9), indices from B
        t, src = i.copy(), np.zeros_like(i)
        for dim in range(3, -1, -1):
            coord = t % P[1 + dim]
            t //= P[1 + dim]
            if dim == P[9]:
                idx = B(i).astype(np.int64)
                coord = np.where(idx < 0, idx + P[10], idx)
            src += coord * P[5 + dim]
        C(i, A(src))
    else:
        raise NotImplementedError(op)
    return c.astype(np.float32)


def matmul(a, b, m: int, n: int, k: int, batch_shape=(), a_strides=(), b_strides=()) -> np.ndarray:
    """c[z] = a[za] @ b[zb] for each output matrix z of the row-major batch
    shape, za / zb from the per-axis matrix strides (0 on broadcast axes):
    the broadcasting product of VulkanExecution.cs:499-541 and
    TensorOps.MatMul.  float64 accumulation."""
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    count = int(np.prod(batch_shape)) if len(batch_shape) else 1
    out = np.empty((count, m, n), np.float64)
    for z in range(count):
        t, za, zb = z, 0, 0
        for j in range(len(batch_shape) - 1, -1, -1):
            coord = t % batch_shape[j]
            t //= batch_shape[j]
            za += coord * a_strides[j]
            zb += coord * b_strides[j]
        out[z] = a[za * m * k:(za + 1) * m * k].reshape(m, k) @ b[zb * k * n:(zb + 1) * k * n].reshape(k, n)
    return out.astype(np.float32)
