"""Thin Python handle over the C ABI: a HIP context with frames, device tensors
and the op calls, shaped like the reference's IDeviceBackend
(src/SimdYolo/DeviceExecution.cs:4-76).  Used by tests and bench.py; the work
itself is all in libsimdyolo_hip.so.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N
from ._native import Tensor, check, fptr


class HipContext:
    def __init__(self, device: int = 0):
        self._lib = N.lib()
        h = ctypes.c_void_p()
        check(self._lib.sy_create(device, ctypes.byref(h)))
        self.handle = h
        self.frame_id = None

    # ----------------------------------------------------------- lifecycle
    def close(self):
        if self.handle:
            self._lib.sy_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def name(self) -> str:
        return self._lib.sy_name(self.handle).decode()

    # ----------------------------------------------------------- frames
    def begin_frame(self) -> int:
        fid = ctypes.c_int64()
        check(self._lib.sy_frame_begin(self.handle, ctypes.byref(fid)))
        self.frame_id = fid.value
        return fid.value

    def end_frame(self):
        check(self._lib.sy_frame_end(self.handle))

    def flush(self):
        check(self._lib.sy_flush(self.handle))

    def alloc(self, n, c, h, w) -> Tensor:
        t = Tensor()
        check(self._lib.sy_frame_alloc(self.handle, n, c, h, w, ctypes.byref(t)))
        return t

    def upload(self, host_nchw: np.ndarray, dst: Tensor | None = None) -> Tensor:
        a = np.ascontiguousarray(host_nchw, dtype=np.float32)
        if dst is None:
            dst = self.alloc(*a.shape)
        assert tuple(a.shape) == dst.shape, (a.shape, dst.shape)
        check(self._lib.sy_upload_nchw(self.handle, fptr(a), ctypes.byref(dst)))
        return dst

    def download(self, t: Tensor) -> np.ndarray:
        out = np.empty(t.shape, np.float32)
        check(self._lib.sy_download_nchw(self.handle, ctypes.byref(t), fptr(out)))
        return out

    # ----------------------------------------------------------- raw memory
    def malloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        check(self._lib.sy_malloc(self.handle, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, ptr: int):
        check(self._lib.sy_free(self.handle, ptr))

    def h2d(self, dst: int, src: np.ndarray):
        src = np.ascontiguousarray(src)
        check(self._lib.sy_memcpy(self.handle, dst, src.ctypes.data, src.nbytes, 0))

    def d2h(self, src: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(self._lib.sy_memcpy(self.handle, out.ctypes.data, src, out.nbytes, 1))
        return out

    # ----------------------------------------------------------- ops
    def conv_create(self, w, bias=None, stride=(1, 1), pads=(0, 0, 0, 0), dilation=(1, 1), groups=1,
                    silu=False) -> int:
        w = np.ascontiguousarray(w, dtype=np.float32)
        oc, icg, kh, kw = w.shape
        b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
        h = ctypes.c_uint64()
        check(self._lib.sy_conv_create(self.handle, fptr(w), fptr(b) if b is not None else None, oc, icg * groups,
                                       kh, kw, stride[0], stride[1], pads[0], pads[1], pads[2], pads[3],
                                       dilation[0], dilation[1], groups, int(silu), ctypes.byref(h)))
        return h.value

    def conv_transpose2x2_create(self, w, bias=None) -> int:
        """nn.ConvTranspose2d(ic, oc, 2, 2) with PyTorch's [ic][oc][2][2] weight."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        ic, oc = w.shape[:2]
        b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
        h = ctypes.c_uint64()
        check(self._lib.sy_conv_transpose2x2_create(self.handle, fptr(w), fptr(b) if b is not None else None, ic, oc,
                                                     ctypes.byref(h)))
        return h.value

    def conv_set_algo(self, conv: int, algo: int):
        check(self._lib.sy_conv_set_algo(self.handle, conv, algo))

    def conv_algo(self, conv: int) -> int:
        a = ctypes.c_int()
        check(self._lib.sy_conv_get_algo(self.handle, conv, ctypes.byref(a)))
        return a.value

    def conv_out_size(self, conv: int, h: int, w: int):
        oh, ow = ctypes.c_int(), ctypes.c_int()
        check(self._lib.sy_conv_out_size(self.handle, conv, h, w, ctypes.byref(oh), ctypes.byref(ow)))
        return oh.value, ow.value

    def conv(self, conv: int, x: Tensor, y: Tensor, residual: Tensor | None = None):
        check(self._lib.sy_conv_run(self.handle, conv, ctypes.byref(x), ctypes.byref(y),
                                    ctypes.byref(residual) if residual is not None else None))

    def conv_upsampled(self, conv: int, xu: Tensor, x: Tensor, y: Tensor, residual: Tensor | None = None):
        """1x1 conv over concat(upsample2x(xu), rest); x is the concat view."""
        check(self._lib.sy_conv_run_upsampled(self.handle, conv, ctypes.byref(xu), ctypes.byref(x), ctypes.byref(y),
                                              ctypes.byref(residual) if residual is not None else None))

    def add(self, a: Tensor, b: Tensor, y: Tensor):
        check(self._lib.sy_add(self.handle, ctypes.byref(a), ctypes.byref(b), ctypes.byref(y)))

    def resize_nearest(self, x: Tensor, y: Tensor):
        check(self._lib.sy_resize_nearest(self.handle, ctypes.byref(x), ctypes.byref(y)))

    def maxpool(self, x: Tensor, y: Tensor, kernel, stride, pads, ceil_mode=False):
        check(self._lib.sy_maxpool(self.handle, ctypes.byref(x), ctypes.byref(y), kernel[0], kernel[1], stride[0],
                                   stride[1], pads[0], pads[1], pads[2], pads[3], int(ceil_mode)))

    def sppf_pool(self, x: Tensor, y5: Tensor, y9: Tensor, y13: Tensor):
        check(self._lib.sy_sppf_pool(self.handle, ctypes.byref(x), ctypes.byref(y5), ctypes.byref(y9),
                                     ctypes.byref(y13)))

    def copy(self, x: Tensor, y: Tensor):
        check(self._lib.sy_copy(self.handle, ctypes.byref(x), ctypes.byref(y)))

    def detect_decode(self, levels, strides, bins, nc, xyxy, out_ptr: int, total: int):
        arr = (Tensor * len(levels))(*levels)
        s = np.ascontiguousarray(strides, dtype=np.float32)
        check(self._lib.sy_detect_decode(self.handle, arr, fptr(s), len(levels), bins, nc, int(xyxy), out_ptr,
                                         total))

    def e2e_topk(self, head_ptr: int, batch, channels, anchors, nc, maximum, onnx_rules, out_ptr: int):
        check(self._lib.sy_e2e_topk(self.handle, head_ptr, batch, channels, anchors, nc, maximum, int(onnx_rules),
                                    out_ptr))

    def attention(self, qkv: Tensor, heads: int, key_dim: int, head_dim: int, scale: float, o: Tensor, v: Tensor):
        check(self._lib.sy_attention(self.handle, ctypes.byref(qkv), heads, key_dim, head_dim, float(scale),
                                     ctypes.byref(o), ctypes.byref(v)))

    def compute(self, op: int, inputs, params, work_items: int, out_ptr: int, out_len: int):
        """One tensor.comp op. `inputs` holds up to three (device_ptr, length_in_floats) pairs or None for
        the A, B and D bindings; `params` up to 32 uint32 slots (floats passed as their bit pattern)."""
        ptrs = (ctypes.c_void_p * 3)()
        lens = (ctypes.c_size_t * 3)()
        for i, t in enumerate(list(inputs)[:3]):
            if t is not None:
                ptrs[i], lens[i] = t[0], t[1]
        p = (ctypes.c_uint32 * 32)()
        for i, v in enumerate(list(params)[:32]):
            p[i] = int(v) & 0xFFFFFFFF
        check(self._lib.sy_compute(self.handle, op, ptrs, lens, p, int(work_items), out_ptr, int(out_len)))

    def matmul(self, a_ptr: int, b_ptr: int, c_ptr: int, m: int, n: int, k: int, batch_shape=(), a_strides=(),
               b_strides=(), a_len: int = 0, b_len: int = 0, c_len: int = 0):
        r = len(batch_shape)
        bs = (ctypes.c_int32 * max(r, 1))(*batch_shape)
        as_ = (ctypes.c_int64 * max(r, 1))(*a_strides)
        bst = (ctypes.c_int64 * max(r, 1))(*b_strides)
        check(self._lib.sy_matmul(self.handle, a_ptr, b_ptr, c_ptr, m, n, k, r, bs, as_, bst, a_len, b_len, c_len))

    # ----------------------------------------------------------- graphs / timing
    def graph_begin(self):
        check(self._lib.sy_graph_begin(self.handle))

    def graph_end(self) -> int:
        g = ctypes.c_uint64()
        check(self._lib.sy_graph_end(self.handle, ctypes.byref(g)))
        return g.value

    def graph_launch(self, g: int):
        check(self._lib.sy_graph_launch(self.handle, g))

    def tune_save(self, path: str):
        """Write the autotuner's decisions of this context (a text table)."""
        check(self._lib.sy_tune_save(self.handle, path.encode()))

    def tune_load(self, path: str):
        """Merge a tuning table written by the same library build."""
        check(self._lib.sy_tune_load(self.handle, path.encode()))

    def timer_start(self):
        check(self._lib.sy_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        check(self._lib.sy_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    def profile_enable(self, on: bool):
        check(self._lib.sy_profile_enable(self.handle, int(on)))

    def profile_read(self) -> dict:
        """{kernel: (launches, total_ms, algorithmic_flops, algorithmic_bytes)}"""
        cap = 256
        names = ctypes.create_string_buffer(cap * 64)
        counts = (ctypes.c_int * cap)()
        ms = (ctypes.c_float * cap)()
        fl = (ctypes.c_double * cap)()
        by = (ctypes.c_double * cap)()
        n = ctypes.c_int()
        check(self._lib.sy_profile_read(self.handle, names, len(names), counts, ms, fl, by, cap, ctypes.byref(n)))
        raw = names.raw.split(b"\0")
        return {raw[i].decode(): (counts[i], ms[i], fl[i], by[i]) for i in range(n.value)}

    def mask_decode(self, protos: Tensor, coeff_ptr: int, ld_coeff: int, boxes, transform, out_ptr: int,
                    capacity: int):
        """boxes: list of (x, y, w, h) in source pixels.  Returns [(left, top, width, height, offset)]."""
        k = len(boxes)
        dets = (N.DetectionT * max(1, k))(*[N.DetectionT(0, 1.0, *map(float, b), 0) for b in boxes])
        info = (N.MaskInfo * max(1, k))()
        check(self._lib.sy_mask_decode(self.handle, ctypes.byref(protos), coeff_ptr, ld_coeff, k, dets,
                                       ctypes.byref(transform), out_ptr, capacity, info))
        return [(i.left, i.top, i.width, i.height, i.offset) for i in info[:k]]
