"""Cases of the generic device ops: inputs, a parameter block built as the
reference's callers build it, and the result a library routine gives for the
same operation (torch.nn.functional on the CPU, numpy).  The CPU tests pin the
oracle's restatement of tensor.comp against ``expect``; the GPU tests compare
the HIP ``sy_compute`` entry with the oracle on the same inputs.

``tol`` is the relative tolerance (to the largest magnitude of the expected
output) for ops that evaluate exp / pow or add taps in a different order; 0
means bit-exact (data movement, comparisons, one rounding of +,-,*,/).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from _tensor_params import (binary, block, concat_part, conv_transpose, decode_head, decode_pose, depth_to_space,
                            depthwise, dfl, gather, pool, resize, row_max, slice_, softmax, transpose, unary)


def assert_close(got, exp, tol):
    got, exp = np.asarray(got, np.float32).reshape(-1), np.asarray(exp, np.float32).reshape(-1)
    assert got.shape == exp.shape
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    if tol == 0:
        assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32)), \
            float(np.abs(got[~nan] - exp[~nan]).max())
    else:
        scale = max(float(np.abs(exp[~nan]).max()), 1e-30)
        err = float(np.abs(got[~nan].astype(np.float64) - exp[~nan]).max()) / scale
        assert err <= tol, err


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32))


def _case(name, built, a, b=None, d=None, expect=None, tol=0.0, out_len=None, prefill=None):
    op, params, items, out_shape = built
    n_out = int(np.prod(out_shape)) if out_len is None else out_len
    return dict(name=name, op=op, params=params, items=items, out_shape=out_shape, out_len=n_out,
                a=None if a is None else np.ascontiguousarray(a, np.float32).reshape(-1),
                b=None if b is None else np.ascontiguousarray(b, np.float32).reshape(-1),
                d=None if d is None else np.ascontiguousarray(d, np.float32).reshape(-1),
                expect=None if expect is None else np.asarray(expect, np.float32).reshape(-1), tol=tol,
                prefill=prefill)


def cases():
    rng = np.random.default_rng(1234)
    r = lambda *s: rng.standard_normal(s).astype(np.float32)
    out = []

    # Unary 1-9 (DeviceOps.Unary).
    x = r(2, 3, 17, 19) * 4
    xt = _t(x)
    out += [
        _case("silu", unary(1, x.shape), x, expect=F.silu(xt), tol=2e-6),
        _case("sigmoid", unary(2, x.shape), x, expect=torch.sigmoid(xt), tol=2e-6),
        _case("relu", unary(3, x.shape), x, expect=F.relu(xt)),
        _case("scale", unary(4, x.shape, 0.37), x, expect=xt * np.float32(0.37)),
        _case("exp", unary(5, x.shape), x, expect=torch.exp(xt), tol=2e-6),
        _case("sqrt", unary(6, x.shape), np.abs(x), expect=torch.sqrt(_t(np.abs(x))), tol=2.5e-7),
        _case("neg", unary(7, x.shape), x, expect=-xt),
        _case("abs", unary(8, x.shape), x, expect=torch.abs(xt)),
        _case("leaky", unary(9, x.shape, 0.1), x, expect=F.leaky_relu(xt, 0.1)),
    ]
    # Broadcast binary 10-16 (DeviceOps.Binary) over several broadcast patterns.
    pats = [((2, 3, 5, 7), (2, 3, 5, 7)), ((2, 3, 5, 7), (3, 1, 1)), ((1, 8, 1), (4, 1, 6)),
            ((7,), (3, 5, 7)), ((2, 1, 4, 1), (1, 3, 1, 5))]
    ops = {10: np.add, 11: np.subtract, 12: np.multiply, 13: np.divide, 15: np.maximum, 16: np.minimum}
    for k, (sa, sb) in enumerate(pats):
        a, b = r(*sa), r(*sb)
        for op, fn in ops.items():
            bb = b if op != 13 else np.where(np.abs(b) < 0.1, 0.5, b).astype(np.float32)
            out.append(_case(f"bin{op}_{k}", binary(op, sa, sb), a, bb, expect=fn(a, bb)))
        pa = np.abs(a) + 0.1
        out.append(_case(f"pow_{k}", binary(14, sa, sb), pa, b, expect=torch.pow(_t(pa), _t(b)), tol=4e-6))
    # NaN propagates through relu, max, min and the max pool (IEEE 754-2019
    # maximum / minimum, as torch and numpy do).
    xn = r(2, 3, 9, 7)
    xn.reshape(-1)[::13] = np.nan
    yn = r(2, 3, 9, 7)
    yn.reshape(-1)[5::11] = np.nan
    out += [
        _case("relu_nan", unary(3, xn.shape), xn, expect=F.relu(_t(xn))),
        _case("bin15_nan", binary(15, xn.shape, yn.shape), xn, yn, expect=np.maximum(xn, yn)),
        _case("bin16_nan", binary(16, xn.shape, yn.shape), xn, yn, expect=np.minimum(xn, yn)),
        _case("maxpool_nan", pool(xn.shape, (3, 3), (1, 1), (1, 1, 1, 1), False), xn,
              expect=F.max_pool2d(_t(xn), 3, 1, 1)),
    ]
    # Nearest resize 20 (Compute.cs:720) at integer ratios and a downsample.
    x = r(2, 3, 6, 5)
    for h, w in [(12, 10), (18, 15), (3, 5)]:
        out.append(_case(f"resize_{h}x{w}", resize(x.shape, h, w), x,
                         expect=F.interpolate(_t(x), size=(h, w), mode="nearest")))
    # Pools 21/22 (Compute.cs:677-693).
    x = r(2, 4, 13, 11)
    for k, s, p, ceil in [((5, 5), (1, 1), (2, 2, 2, 2), False), ((3, 3), (2, 2), (1, 1, 1, 1), False),
                          ((2, 2), (2, 2), (0, 0, 0, 0), True), ((3, 2), (2, 1), (1, 0, 1, 0), False)]:
        out.append(_case(f"maxpool_{k[0]}{k[1]}s{s[0]}c{int(ceil)}", pool(x.shape, k, s, p, False, ceil=ceil), x,
                         expect=F.max_pool2d(_t(x), k, s, (p[0], p[1]), ceil_mode=ceil)))
        for cip in (False, True):
            out.append(_case(f"avgpool_{k[0]}{k[1]}s{s[0]}c{int(ceil)}i{int(cip)}",
                             pool(x.shape, k, s, p, True, cip, ceil), x,
                             expect=F.avg_pool2d(_t(x), k, s, (p[0], p[1]), ceil_mode=ceil,
                                                 count_include_pad=cip,
                                                 divisor_override=k[0] * k[1] if cip else None), tol=1e-6))
    # Transpose 23 (DeviceOps.Transpose).
    for shape, perm in [((2, 3, 4, 5), (0, 2, 3, 1)), ((6, 7), (1, 0)), ((3, 4, 5), (2, 0, 1)),
                        ((2, 3, 4, 5), (3, 1, 0, 2))]:
        x = r(*shape)
        out.append(_case(f"transpose_{''.join(map(str, perm))}", transpose(shape, perm), x,
                         expect=np.transpose(x, perm)))
    # Slice 24 (DeviceSlice's shader route).
    x = r(2, 9, 5, 3)
    for axis, start, length in [(1, 2, 4), (2, 1, 3), (3, 2, 1), (0, 1, 1)]:
        idx = [slice(None)] * 4
        idx[axis] = slice(start, start + length)
        out.append(_case(f"slice_ax{axis}", slice_(x.shape, axis, start, length), x, expect=x[tuple(idx)]))
    # Softmax 25 (DeviceOps.Softmax).
    x = r(3, 5, 7, 4) * 3
    for axis in range(4):
        out.append(_case(f"softmax_ax{axis}", softmax(x.shape, axis), x, expect=torch.softmax(_t(x), axis),
                         tol=2e-6))
    # Concat 26: one dispatch writes input 1 of [x0, x1, x2] at its axis offset;
    # the output starts as the concatenation with that part zeroed.
    parts = [r(2, 3, 4, 5), r(2, 2, 4, 5), r(2, 4, 4, 5)]
    full = np.concatenate(parts, 1)
    pre = full.copy()
    pre[:, 3:5] = 0
    out.append(_case("concat_mid", concat_part(parts[1].shape, full.shape, 1, 3), parts[1], expect=full,
                     prefill=pre))
    # Head decode 30 (DeviceOps.DecodeHead), DFL and single-bin, both layouts,
    # and one level written at an anchor offset of a 3-level output.
    for bins, xyxy in [(16, False), (16, True), (1, True), (1, False)]:
        boxes, scores = r(2, 4 * bins, 5, 6) * 2, r(2, 7, 5, 6)
        if bins == 1:
            boxes = np.abs(boxes)
        out.append(_case(f"decode_b{bins}_x{int(xyxy)}", decode_head(2, 5, 6, bins, 7, 16.0, xyxy), boxes, scores,
                         expect=None, tol=4e-6))
    boxes, scores = r(2, 64, 4, 3) * 2, r(2, 5, 4, 3)
    out.append(_case("decode_level_offset", decode_head(2, 4, 3, 16, 5, 32.0, False, out_spatial=40,
                                                        anchor_offset=25), boxes, scores, tol=4e-6))
    # Pose decode 31 (DeviceOps.DecodePose), YOLOv8 and YOLO26 rules.
    for y26 in (False, True):
        kp = r(2, 17 * 3, 4, 5)
        out.append(_case(f"pose_y26{int(y26)}", decode_pose(kp.shape, 17, 3, 8.0, y26), kp, tol=2e-6))
    # Depthwise conv 32 (generic route) with bias, SiLU, stride, dilation, asym pads.
    for k, s, p, dil, silu, bias in [((3, 3), (1, 1), (1, 1, 1, 1), (1, 1), True, True),
                                     ((5, 5), (2, 2), (2, 2, 2, 2), (1, 1), False, True),
                                     ((3, 3), (1, 2), (2, 0, 1, 1), (2, 1), False, False),
                                     ((7, 7), (1, 1), (3, 3, 3, 3), (1, 1), True, False)]:
        x, w = r(2, 6, 11, 9), r(6, 1, *k)
        bb = r(6) if bias else None
        built = depthwise(x.shape, k, s, p, dil, silu)
        xp = F.pad(_t(x), (p[1], p[3], p[0], p[2]))
        y = F.conv2d(xp, _t(w), None if bb is None else _t(bb), stride=s, dilation=dil, groups=6)
        if silu:
            y = F.silu(y)
        out.append(_case(f"dw_k{k[0]}s{s[0]}{s[1]}d{dil[0]}", built, x, w, bb, expect=y, tol=2e-6))
    # Transposed conv 33 (Compute.ConvTranspose) incl. groups, dilation, pads, output padding.
    for ic, ocg, k, st, pd, dil, op_, g in [(8, 6, (2, 2), (2, 2), (0, 0, 0, 0), (1, 1), (0, 0), 1),
                                            (6, 4, (3, 3), (2, 2), (1, 1, 1, 1), (1, 1), (1, 1), 2),
                                            (4, 3, (3, 2), (1, 2), (0, 1, 0, 1), (2, 1), (0, 1), 1),
                                            (6, 2, (4, 4), (3, 3), (1, 2, 1, 2), (1, 1), (2, 0), 3)]:
        x, w, bb = r(2, ic, 5, 4), r(ic, ocg, *k), r(ocg * g)
        built = conv_transpose(x.shape, w.shape, st, pd, dil, op_, g)
        y = F.conv_transpose2d(_t(x), _t(w), _t(bb), stride=st, padding=(pd[0], pd[1]), output_padding=op_,
                               groups=g, dilation=dil)
        out.append(_case(f"convT_k{k[0]}{k[1]}s{st[0]}{st[1]}g{g}", built, x, w, bb, expect=y, tol=4e-6))
    # DFL 34 (OnnxHead.cs:88): input [B][4*16][A].
    x = r(2, 64, 37) * 3
    sm = torch.softmax(_t(x).view(2, 4, 16, 37), 2)
    exp34 = (sm * torch.arange(16, dtype=torch.float32).view(1, 1, 16, 1)).sum(2)
    out.append(_case("dfl16", dfl(x.shape, 16), x, expect=exp34, tol=4e-6))
    # Depth to space 35 (VulkanTransposeConv.cs:28) = pixel shuffle by 2.
    x = r(2, 4 * 5, 3, 4)
    out.append(_case("d2s", depth_to_space(x.shape, 5), x, expect=F.pixel_shuffle(_t(x), 2)))
    # Row max 36 with MathF.Max rules: NaN wins, +0 over -0.
    x = r(5, 6, 9)
    x[0, 0, 3] = np.nan
    x[1, 2, :] = -1.0
    x[1, 2, 4] = -0.0
    x[1, 2, 6] = 0.0
    x[2, 3, :] = -0.0
    rm = x.max(-1)
    rm[0, 0] = np.nan
    rm[1, 2] = 0.0
    rm[2, 3] = -0.0
    out.append(_case("rowmax", row_max(x.shape), x, expect=rm))
    # GatherElements 37 with negative indices.
    x = r(3, 5, 4)
    for axis in range(3):
        idx_shape = list(x.shape)
        idx_shape[axis] = 6
        idx = rng.integers(-x.shape[axis], x.shape[axis], size=idx_shape)
        pos = np.where(idx < 0, idx + x.shape[axis], idx)
        out.append(_case(f"gather_ax{axis}", gather(x.shape, tuple(idx_shape), axis), x, idx.astype(np.float32),
                         expect=torch.gather(_t(x), axis, torch.from_numpy(pos))))
    out += layout_cases(rng)
    return out


def layout_cases(rng):
    """Sizes that reach every launch path of the generic ops: float4 streams
    (aligned, lengths a multiple of 4) beside their scalar forms (odd lengths,
    element offsets), 64 x 64 LDS-tiled transposes with partial edge tiles,
    row gathers, and wave-per-row softmax and row maximum with rows longer
    than the registers hold."""
    r = lambda *s: rng.standard_normal(s).astype(np.float32)
    out = []
    x = r(3, 5, 37, 41) * 3
    out.append(_case("silu_vec", unary(1, x.shape), x, expect=F.silu(_t(x)), tol=2e-6))
    xo = r(1001)
    op, p, n, shape = unary(7, (1000,))
    p[28], p[30] = 1, 3  # misaligned input and output: scalar path
    out.append(_case("neg_offsets", (op, p, n, shape), xo, expect=np.concatenate([[0, 0, 0], -xo[1:]]),
                     out_len=1003))
    # Binary: same shapes (one run), a channel broadcast (stride-0 rows of 4k),
    # a row broadcast and a scalar.
    for k, (sa, sb) in enumerate([((2, 64, 40, 40), (2, 64, 40, 40)), ((2, 64, 40, 40), (1, 64, 1, 1)),
                                  ((8, 96, 128), (96, 1)), ((6, 4, 5, 16), (1,))]):
        a, b = r(*sa), r(*sb)
        out.append(_case(f"bin10_big{k}", binary(10, sa, sb), a, b, expect=a + b))
        out.append(_case(f"bin12_big{k}", binary(12, sa, sb), a, b, expect=a * b))
    # Transposes: NCHW -> NHWC and back at tile sizes with and without edges,
    # a transpose whose inner axis stays contiguous, and a 4-d permutation
    # with no contiguous axis left (after collapsing).
    for shape, perm in [((2, 64, 40, 40), (0, 2, 3, 1)), ((2, 40, 40, 64), (0, 3, 1, 2)),
                        ((1, 3, 67, 129), (0, 2, 3, 1)), ((3, 70, 5, 66), (0, 3, 2, 1)),
                        ((4, 6, 10, 12), (1, 0, 2, 3)), ((5, 7, 9, 11), (2, 3, 0, 1)),
                        ((129, 65), (1, 0))]:
        x = r(*shape)
        out.append(_case(f"transpose_{'x'.join(map(str, shape))}_{''.join(map(str, perm))}", transpose(shape, perm),
                         x, expect=np.transpose(x, perm)))
    # A strided view with no unit-stride axis: the per-element gather.
    x = r(80)
    p = block(20, 1, 1, 4, 5, 0, 0, 20, 2)
    out.append(_case("transpose_strided_view", (23, p, 20, (4, 5)), x, expect=x.reshape(4, 20)[:, 0:10:2]))
    # Slices and concat writes of float4-aligned runs, and of odd ones.
    x = r(2, 96, 20, 20)
    out.append(_case("slice_vec", slice_(x.shape, 1, 32, 48), x, expect=x[:, 32:80]))
    x = r(2, 7, 9, 3)
    out.append(_case("slice_odd", slice_(x.shape, 2, 3, 5), x, expect=x[:, :, 3:8]))
    parts = [r(2, 32, 16, 16), r(2, 64, 16, 16)]
    full = np.concatenate(parts, 1)
    pre = full.copy()
    pre[:, 32:] = 0
    out.append(_case("concat_vec", concat_part(parts[1].shape, full.shape, 1, 32), parts[1], expect=full,
                     prefill=pre))
    # Softmax over long contiguous rows (registers, then re-reads) and a
    # strided axis; row maximum over long rows.
    for shape in [(6, 400), (5, 1000), (3, 63)]:
        x = r(*shape) * 4
        out.append(_case(f"softmax_rows{shape[1]}", softmax(shape, 1), x, expect=torch.softmax(_t(x), 1), tol=2e-6))
    x = r(2, 80, 300) * 4
    out.append(_case("softmax_cols", softmax(x.shape, 1), x, expect=torch.softmax(_t(x), 1), tol=2e-6))
    x = r(7, 300)
    x[3, 200] = np.nan
    x[5] = -1.0
    x[5, 250] = -0.0
    x[5, 17] = 0.0
    rm = x.max(-1)
    rm[3] = np.nan
    rm[5] = 0.0
    out.append(_case("rowmax_long", row_max(x.shape), x, expect=rm))
    return out


def matmul_cases():
    """(name, m, n, k, batch_shape, a_batch_shape, b_batch_shape): numpy
    broadcasting over the batch axes, as TensorOps.MatMul."""
    return [
        ("single_mfma", 96, 80, 64, (), (), ()),
        ("single_tile_k7", 33, 45, 7, (), (), ()),
        ("odd_mfma", 67, 129, 36, (), (), ()),
        ("batched", 40, 24, 32, (3, 2), (3, 2), (3, 2)),
        ("broadcast_b", 50, 60, 20, (4,), (4,), (1,)),
        ("broadcast_a", 17, 31, 12, (2, 3), (1, 3), (2, 3)),
        ("broadcast_both_tile", 9, 11, 13, (2, 3), (2, 1), (1, 3)),
        ("attention_like", 64, 64, 32, (1, 4), (1, 4), (1, 4)),
    ]


def batch_strides(out_batch, operand_batch):
    """Matrix strides per output batch axis (0 where the operand broadcasts)."""
    ob = (1,) * (len(out_batch) - len(operand_batch)) + tuple(operand_batch)
    strides, acc = [0] * len(ob), 1
    for j in range(len(ob) - 1, -1, -1):
        strides[j] = 0 if ob[j] == 1 else acc
        acc *= ob[j]
    return strides
