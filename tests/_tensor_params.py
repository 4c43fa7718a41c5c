"""Parameter blocks for the generic device ops, built the way the reference's
callers build them, so the CPU pins and the GPU parity tests exercise the
layouts the reference actually dispatches.

Each builder returns ``(op, params, work_items, out_shape)``; ``params`` is a
32-slot uint32 list with P(0) == work items.
"""
from __future__ import annotations

import numpy as np


def bits(v: float) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def block(*values) -> list:
    """DeviceOps.Parameters (DeviceExecution.cs:107-112)."""
    p = [0] * 32
    for j, v in enumerate(values):
        p[j] = int(v) & 0xFFFFFFFF
    return p


def _strides(shape):
    s, acc = [0] * len(shape), 1
    for d in range(len(shape) - 1, -1, -1):
        s[d] = acc
        acc *= shape[d]
    return s


def unary(op, shape, scale=1.0):
    """DeviceOps.Unary (DeviceExecution.cs:119-120)."""
    n = int(np.prod(shape))
    return op, block(n, bits(scale)), n, tuple(shape)


def binary(op, a_shape, b_shape):
    """DeviceOps.Binary (DeviceExecution.cs:128-139): 4-d broadcast strides,
    0 on axes of size 1."""
    shape = np.broadcast_shapes(tuple(a_shape), tuple(b_shape))
    assert len(shape) <= 4
    n = int(np.prod(shape))
    p = block(n)
    ad = [1] * (4 - len(a_shape)) + list(a_shape)
    bd = [1] * (4 - len(b_shape)) + list(b_shape)
    yd = [1] * (4 - len(shape)) + list(shape)
    ast, bst = _strides(ad), _strides(bd)
    for d in range(4):
        p[1 + d] = yd[d]
        p[5 + d] = 0 if ad[d] == 1 else ast[d]
        p[9 + d] = 0 if bd[d] == 1 else bst[d]
    return op, p, n, tuple(shape)


def softmax(shape, axis):
    """DeviceOps.Softmax (DeviceExecution.cs:144-149)."""
    inner, outer = int(np.prod(shape[axis + 1:])), int(np.prod(shape[:axis]))
    return 25, block(inner * outer, shape[axis], inner), inner * outer, tuple(shape)


def transpose(shape, perm):
    """DeviceOps.Transpose (DeviceExecution.cs:157-164)."""
    out = [shape[q] for q in perm]
    n = int(np.prod(shape))
    p = block(n)
    lead, st = 4 - len(shape), _strides(shape)
    for d in range(4):
        p[1 + d] = 1 if d < lead else out[d - lead]
        p[5 + d] = 0 if d < lead else st[perm[d - lead]]
    return 23, p, n, tuple(out)


def resize(shape, h, w):
    """Compute.cs:720: nearest resize to (h, w)."""
    n = shape[0] * shape[1] * h * w
    return 20, block(n, shape[2], shape[3], h, w), n, (shape[0], shape[1], h, w)


def pool_out(size, k, s, p0, p1, ceil):
    """Compute.PoolOutputSize (Compute.cs:699-707)."""
    num = size + p0 + p1 - k + (s - 1 if ceil else 0)
    o = num // s + 1
    return min(o, (size + p0 + s - 1) // s) if ceil else o


def pool(shape, kernel, stride, pads, average, count_include_pad=False, ceil=False):
    """Compute.cs:677-693: max (21) or average (22) pool."""
    h, w = shape[2:]
    oh = pool_out(h, kernel[0], stride[0], pads[0], pads[2], ceil)
    ow = pool_out(w, kernel[1], stride[1], pads[1], pads[3], ceil)
    n = shape[0] * shape[1] * oh * ow
    p = block(n, h, w, oh, ow, kernel[0], kernel[1], stride[0], stride[1], pads[0], pads[1],
              1 if count_include_pad else 0, pads[2], pads[3], 1 if ceil else 0)
    return 22 if average else 21, p, n, (shape[0], shape[1], oh, ow)


def slice_(shape, axis, start, length):
    """VulkanExecution.cs:486-492: DeviceSlice's shader route (op 24)."""
    inner = int(np.prod(shape[axis + 1:]))
    out = list(shape)
    out[axis] = length
    n = int(np.prod(out))
    return 24, block(n, shape[axis], length, inner, start), n, tuple(out)


def concat_part(part_shape, out_shape, axis, start):
    """VulkanExecution.cs:440-452: one input's concat write (op 26)."""
    inner = int(np.prod(out_shape[axis + 1:]))
    n = int(np.prod(part_shape))
    return 26, block(n, part_shape[axis], out_shape[axis], inner, start), n, tuple(out_shape)


def decode_head(batch, h, w, bins, nc, stride, xyxy, out_spatial=0, anchor_offset=0):
    """DeviceOps.DecodeHead (DeviceExecution.cs:172-177), plus the output
    spatial / anchor offset slots the multi-level decode sets."""
    n = batch * h * w
    p = block(n, h * w, w, bins, nc, bits(stride), 1 if xyxy else 0, out_spatial, anchor_offset)
    total = out_spatial or h * w
    return 30, p, n, (batch, nc + 4, total)


def decode_pose(shape, count, dims, stride, yolo26):
    """DeviceOps.DecodePose (DeviceExecution.cs:185-190)."""
    n = int(np.prod(shape))
    spatial = shape[2] * shape[3]
    return 31, block(n, spatial, shape[3], dims, bits(stride), 1 if yolo26 else 0), n, \
        (shape[0], count * dims, spatial)


def depthwise(x_shape, k, stride, pads, dilation, silu):
    """VulkanExecution.cs:338-344: generic depthwise route (op 32)."""
    b, c, ih, iw = x_shape
    oh = (ih + pads[0] + pads[2] - dilation[0] * (k[0] - 1) - 1) // stride[0] + 1
    ow = (iw + pads[1] + pads[3] - dilation[1] * (k[1] - 1) - 1) // stride[1] + 1
    n = b * c * oh * ow
    p = block(n, c, ih, iw, c, oh, ow, k[0], k[1], stride[0], stride[1], pads[0], pads[1], dilation[0],
              dilation[1], c, 1 if silu else 0)
    return 32, p, n, (b, c, oh, ow)


def conv_transpose(x_shape, w_shape, strides, pads, dilation, out_pad, groups):
    """Compute.cs:124-138 (op 33): weights [ic][oc/groups][kh][kw]."""
    batch, ic, ih, iw = x_shape
    ocg, kh, kw = w_shape[1:]
    oc = ocg * groups
    oh = (ih - 1) * strides[0] - pads[0] - pads[2] + dilation[0] * (kh - 1) + out_pad[0] + 1
    ow = (iw - 1) * strides[1] - pads[1] - pads[3] + dilation[1] * (kw - 1) + out_pad[1] + 1
    n = batch * oc * oh * ow
    p = block(n, ic, ih, iw, oc, oh, ow, kh, kw, strides[0], strides[1], pads[0], pads[1], dilation[0],
              dilation[1], groups)
    return 33, p, n, (batch, oc, oh, ow)


def dfl(shape, bins):
    """OnnxHead.cs:88 (op 34): input [B][4*bins][A], output [B][4][A]."""
    out = (shape[0], shape[1] // bins, shape[2])
    n = int(np.prod(out))
    return 34, block(n, shape[2], bins), n, out


def depth_to_space(product_shape, oc):
    """VulkanTransposeConv.cs:28 (op 35): [B][4*oc][h][w] -> [B][oc][2h][2w]."""
    out = (product_shape[0], oc, product_shape[2] * 2, product_shape[3] * 2)
    n = int(np.prod(out))
    return 35, block(n, out[2], out[3], oc), n, out


def row_max(shape):
    """OnnxDeviceOperations.cs:38-39 (op 36): max over the last axis."""
    rows, size = int(np.prod(shape[:-1])), shape[-1]
    return 36, block(rows, size), rows, tuple(shape[:-1])


def gather(in_shape, idx_shape, axis):
    """OnnxDeviceOperations.cs:49-72 (op 37): GatherElements."""
    n = int(np.prod(idx_shape))
    p = block(n)
    lead, st = 4 - len(in_shape), _strides(in_shape)
    for d in range(4):
        p[1 + d] = 1 if d < lead else idx_shape[d - lead]
        p[5 + d] = 0 if d < lead else st[d - lead]
    p[9], p[10] = axis + lead, in_shape[axis]
    return 37, p, n, tuple(idx_shape)
