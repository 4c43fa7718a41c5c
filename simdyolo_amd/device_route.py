"""The op-by-op device route: a Python mirror of ``integration/csharp/HipBackend.cs``
driven the way the reference's ``PtModel.Run`` drives an ``IDeviceBackend``.

A SimdYolo host that selects the HIP device and walks a loaded ``.pt`` model one
module at a time (``src/SimdYolo/PtModel.cs:184-220``, module semantics
``:267-504``) reaches the library through this sequence of calls, every one of
them an entry of the C ABI:

* ``DeviceConv`` (``Compute.cs:194``): an op-23 transpose NCHW -> NHWC, the
  library's convolution, an op-23 transpose back (the library's kernels run
  channels-last; the reference's device tensors are dense NCHW);
* ``Compute`` (``DeviceExecution.cs:41``) for the module glue: op 10 for the
  bottleneck shortcut (``PtModel.cs:303``), op 21 for SPPF's pools
  (``:417-424``), op 20 for ``Upsample`` (``Compute.cs:715-721``);
* ``DeviceConcat`` as one op-26 write per input (``VulkanExecution.cs:433-478``);
* ``DeviceSlice`` for C2f's chunk: a borrowed view when the slice is one
  contiguous run (batch 1), else op 24 (``VulkanExecution.cs:486-492``);
* the joined head decode, op 30 per level into ``[B, nc + 4, A]``
  (``VulkanExecution.cs:295-324``).

Replay (``VulkanReplay.cs:31-129``, on hipGraphs): the first frame of an input
shape runs eagerly (convolutions tune, scratch grows) and, if it used the
input as its only host upload and read nothing back before its outputs, marks
the shape replayable; the next frame of that shape is captured into a graph
(inputs uploaded before the capture begins) and launched once; later frames of
the shape copy the input into the captured upload buffer, launch the graph and
download the outputs.  If anything in a captured frame needs the host (an
upload, a download, an allocation the library refuses under capture), the
capture is ended there, the recorded work is launched once and the frame goes
on op by op.

``HipDeviceBackend`` mirrors ``HipBackend.cs`` method for method;
``YoloV8Walk`` mirrors the parts of ``PtModel.Forward`` the YOLOv8 detect
models use; ``DeviceRouteDetector.predict_raw`` mirrors
``YoloDetector.RunInference`` (``YoloDetector.cs:262-313``).
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _native as N
from ._native import Tensor, check, fptr
from .device import HipContext

SY_ESTATE = N.SY_ESTATE


class DeviceTensor:
    """A dense row-major device tensor of one frame (``DeviceStorage`` + shape)."""
    __slots__ = ("ptr", "length", "shape", "frame")

    def __init__(self, ptr: int, length: int, shape, frame: int):
        self.ptr, self.length, self.shape, self.frame = int(ptr), int(length), tuple(int(d) for d in shape), frame

    @property
    def rank(self) -> int:
        return len(self.shape)


def _count(shape) -> int:
    return int(np.prod(shape)) if len(shape) else 1


def _strides(shape):
    s, acc = [0] * len(shape), 1
    for d in range(len(shape) - 1, -1, -1):
        s[d] = acc
        acc *= shape[d]
    return s


def parameters(*values) -> list:
    """DeviceOps.Parameters (DeviceExecution.cs:107-112): 32 slots, the rest zero."""
    p = [0] * 32
    for j, v in enumerate(values):
        p[j] = int(v) & 0xFFFFFFFF
    return p


def bits(v: float) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


class HipDeviceBackend:
    """HipBackend.cs over the C ABI (IDeviceBackend + the fast paths)."""

    def __init__(self, device: int = 0, replay: bool = True):
        self.ctx = HipContext(device)
        self._lib = N.lib()
        self.frame_active = False
        self.frame_id = 0
        self._constants: dict[int, tuple[np.ndarray, int]] = {}   # id(host array) -> (array, device ptr)
        self._frame_inputs: dict[int, tuple[np.ndarray, DeviceTensor]] = {}
        self._convs: dict[tuple, int] = {}
        # replay state (VulkanReplay.cs:5-30)
        self.replay_enabled = replay
        self.replayed_frames = 0
        self._candidate = False
        self._capture_input = None
        self._capture_upload: DeviceTensor | None = None
        self._host_uploads = 0
        self._capturing = False
        self._replayable_shape = None
        self._plan = None  # (shape, input DeviceTensor, graph id, [(ptr, length, shape, alias)])

    def close(self):
        if self.ctx is not None:
            for _, p in self._constants.values():
                self.ctx.free(p)
            self._constants.clear()
            self.ctx.close()
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ------------------------------------------------------------ library calls
    def _call(self, fn, *args):
        """Runs one library call.  Under capture, a call the library refuses
        there (SY_ESTATE: it needs the host or an allocation) ends the capture,
        launches what was recorded, and runs eagerly."""
        rc = fn(*args)
        if rc == SY_ESTATE and self._capturing:
            self._abort_capture()
            rc = fn(*args)
        check(rc)

    # ------------------------------------------------------------ frames
    def begin_frame(self):
        if self.frame_active:
            raise RuntimeError("An inference is already recording.")
        fid = ctypes.c_int64()
        check(self._lib.sy_frame_begin(self.ctx.handle, ctypes.byref(fid)))
        self.frame_id = fid.value
        self.frame_active = True
        self._frame_inputs.clear()

    def end_frame(self):
        try:
            if self._capturing:
                self._abort_capture()
            if self.frame_active:
                check(self._lib.sy_frame_end(self.ctx.handle))
        finally:
            self.frame_active = False
            self._frame_inputs.clear()
            self._candidate = False
            self._capture_input = None

    def _alloc(self, shape) -> DeviceTensor:
        n = max(1, _count(shape))
        t = Tensor()
        self._call(self._lib.sy_frame_alloc, self.ctx.handle, 1, 1, 1, n, ctypes.byref(t))
        return DeviceTensor(t.data, _count(shape), shape, self.frame_id)

    def upload(self, x, constant: bool = False) -> DeviceTensor:
        """HipBackend.Upload: device tensors of this frame pass through;
        constants are uploaded once per host array; other host tensors once
        per frame."""
        if isinstance(x, DeviceTensor):
            if x.frame != self.frame_id:
                raise RuntimeError("Device tensor belongs to another inference.")
            return x
        key = id(x)
        if key in self._frame_inputs:
            return self._frame_inputs[key][1]
        data = np.ascontiguousarray(x, dtype=np.float32)
        if constant:
            if key not in self._constants:
                p = ctypes.c_void_p()
                self._call(self._lib.sy_malloc, self.ctx.handle, max(data.nbytes, 4), ctypes.byref(p))
                self._call(self._lib.sy_memcpy, self.ctx.handle, p.value, data.ctypes.data, data.nbytes, 0)
                self._constants[key] = (x, p.value)
            t = DeviceTensor(self._constants[key][1], data.size, data.shape, self.frame_id)
        else:
            self._observe_upload(x)
            t = self._alloc(data.shape)
            self._call(self._lib.sy_memcpy, self.ctx.handle, t.ptr, data.ctypes.data, data.nbytes, 0)
        self._frame_inputs[key] = (x, t)
        return t

    def download(self, t: DeviceTensor) -> np.ndarray:
        """IDeviceBackend.Download (a host read: no longer a replay candidate)."""
        if t.frame != self.frame_id or not self.frame_active:
            raise RuntimeError("Device output belongs to another inference.")
        self._candidate = False
        out = np.empty(t.shape, np.float32)
        self._call(self._lib.sy_memcpy, self.ctx.handle, out.ctypes.data, t.ptr, out.nbytes, 1)
        return out

    # ------------------------------------------------------------ generic ops
    def compute(self, op: int, inputs, shape, params, work_items: int) -> DeviceTensor:
        out = self._alloc(shape)
        ptrs = (ctypes.c_void_p * 3)()
        lens = (ctypes.c_size_t * 3)()
        for i, x in enumerate(inputs[:3]):
            s = self.upload(x)
            ptrs[i], lens[i] = s.ptr, max(1, s.length)
        p = (ctypes.c_uint32 * 32)(*[v if j < 27 else 0 for j, v in enumerate(params)])
        self._call(self._lib.sy_compute, self.ctx.handle, op, ptrs, lens, p, int(work_items), out.ptr,
                   max(1, out.length))
        return out

    def device_concat(self, tensors, axis: int, shape) -> DeviceTensor:
        out = self._alloc(shape)
        inner = _count(shape[axis + 1:])
        start = 0
        ptrs = (ctypes.c_void_p * 3)()
        lens = (ctypes.c_size_t * 3)()
        for x in tensors:
            length = _count(x.shape)
            if length == 0:
                continue
            s = self.upload(x)
            p = (ctypes.c_uint32 * 32)(*parameters(length, x.shape[axis], shape[axis], inner, start))
            ptrs[0], lens[0] = s.ptr, s.length
            self._call(self._lib.sy_compute, self.ctx.handle, 26, ptrs, lens, p, length, out.ptr, out.length)
            start += x.shape[axis]
        return out

    def device_slice(self, x, shape, axis: int, start: int) -> DeviceTensor:
        s = self.upload(x)
        inner, outer = _count(s.shape[axis + 1:]), _count(s.shape[:axis])
        if outer == 1:  # one contiguous run: a borrowed view
            return DeviceTensor(s.ptr + 4 * start * inner, _count(shape), shape, self.frame_id)
        return self.compute(24, [s], shape, parameters(_count(shape), s.shape[axis], shape[axis], inner, start),
                            _count(shape))

    # ------------------------------------------------------------ convolution
    def _convolution(self, w, bias, stride, pads, dilation, groups, silu) -> int:
        key = (id(w), id(bias) if bias is not None else 0, tuple(stride), tuple(pads), tuple(dilation), groups,
               bool(silu))
        conv = self._convs.get(key)
        if conv is not None:
            return conv
        oc, icg, kh, kw = w.shape
        h = ctypes.c_uint64()
        wd = np.ascontiguousarray(w, np.float32)
        bd = np.ascontiguousarray(bias, np.float32) if bias is not None else None
        self._call(self._lib.sy_conv_create, self.ctx.handle, fptr(wd), fptr(bd) if bd is not None else None, oc,
                   icg * groups, kh, kw, stride[0], stride[1], pads[0], pads[1], pads[2], pads[3], dilation[0],
                   dilation[1], groups, int(silu), ctypes.byref(h))
        self._convs[key] = h.value
        self._keep = getattr(self, "_keep", [])
        self._keep += [w, bias]
        return h.value

    def device_conv(self, x, w, bias, shape, stride, pads, dilation, groups, silu) -> DeviceTensor:
        conv = self._convolution(w, bias, stride, pads, dilation, groups, silu)
        xs = x.shape
        n, ic, h, wd = xs
        oc, oh, ow = shape[1], shape[2], shape[3]
        nhwc = transpose(self, x, (0, 2, 3, 1), (n, h, wd, ic))
        y = self._alloc((n, oh, ow, oc))
        xv = Tensor(nhwc.ptr, n, ic, h, wd, ic, N.LAYOUT_NHWC)
        yv = Tensor(y.ptr, n, oc, oh, ow, oc, N.LAYOUT_NHWC)
        self._call(self._lib.sy_conv_run, self.ctx.handle, conv, ctypes.byref(xv), ctypes.byref(yv), None)
        return transpose(self, y, (0, 3, 1, 2), shape)

    # ------------------------------------------------------------ fast paths
    def decode_head_levels(self, levels, shape, bins: int, xyxy: bool) -> DeviceTensor:
        """Op 30 per level into the joined output, each at its anchor offset."""
        out = self._alloc(shape)
        total, start = shape[2], 0
        ptrs = (ctypes.c_void_p * 3)()
        lens = (ctypes.c_size_t * 3)()
        for boxes, scores, stride in levels:
            n, _, h, w = boxes.shape
            nc = scores.shape[1]
            b, s = self.upload(boxes), self.upload(scores)
            p = (ctypes.c_uint32 * 32)(*parameters(n * h * w, h * w, w, bins, nc, bits(stride), int(xyxy), total,
                                                   start))
            ptrs[0], lens[0], ptrs[1], lens[1] = b.ptr, b.length, s.ptr, s.length
            self._call(self._lib.sy_compute, self.ctx.handle, 30, ptrs, lens, p, n * h * w, out.ptr, out.length)
            start += h * w
        return out

    # ------------------------------------------------------------ replay
    def begin_replay_capture(self, x: np.ndarray):
        """BeginReplayCapture: the frame is a replay candidate while its only
        host upload is `x` and nothing is read back.  The input is uploaded
        first, so every frame of a shape allocates in the same order; a shape
        whose previous frame qualified is captured from here on."""
        self._candidate = self.replay_enabled and isinstance(x, np.ndarray) and x.size > 0
        if not self._candidate:
            return
        self._capture_input = x
        self._host_uploads = 0
        self._capture_upload = self.upload(x)
        if self._plan is None and self._replayable_shape == tuple(x.shape):
            check(self._lib.sy_graph_begin(self.ctx.handle))
            self._capturing = True

    def _observe_upload(self, x):
        if self._candidate and x is not self._capture_input:
            self._candidate = False
        self._host_uploads += 1

    def _abort_capture(self):
        """Ends a capture early: the recorded work runs once; the frame goes on eagerly."""
        self._capturing = False
        self._candidate = False
        self._replayable_shape = None
        g = ctypes.c_uint64()
        check(self._lib.sy_graph_end(self.ctx.handle, ctypes.byref(g)))
        check(self._lib.sy_graph_launch(self.ctx.handle, g.value))
        check(self._lib.sy_graph_destroy(self.ctx.handle, g.value))

    def materialize_outputs(self, outputs):
        """MaterializeOutputs / DownloadFrameOutputs: finishes a capture (the
        graph runs once for this frame), then downloads each output into a
        fresh host array.  A candidate frame's shape becomes replayable."""
        if self._capturing:
            self._capturing = False
            g = ctypes.c_uint64()
            check(self._lib.sy_graph_end(self.ctx.handle, ctypes.byref(g)))
            check(self._lib.sy_graph_launch(self.ctx.handle, g.value))
            aliases, descr = {}, []
            for i, t in enumerate(outputs):
                alias = aliases.setdefault(id(t), i)
                descr.append((t.ptr, t.length, t.shape, alias))
            self._plan = (tuple(self._capture_input.shape), self._capture_upload, g.value, descr)
        elif self._candidate and self._plan is None and all(t.length > 0 for t in outputs):
            self._replayable_shape = tuple(self._capture_input.shape)
        check(self._lib.sy_flush(self.ctx.handle))
        host = []
        for t in outputs:
            out = np.empty(t.shape, np.float32)
            check(self._lib.sy_memcpy(self.ctx.handle, out.ctypes.data, t.ptr, out.nbytes, 1))
            host.append(out)
        return host

    def try_replay(self, x: np.ndarray):
        """TryReplay: the captured frame of x's shape, or None."""
        if self._plan is None or self.frame_active or not isinstance(x, np.ndarray) or tuple(x.shape) != self._plan[0]:
            return None
        shape, inp, graph, descr = self._plan
        data = np.ascontiguousarray(x, np.float32)
        check(self._lib.sy_memcpy(self.ctx.handle, inp.ptr, data.ctypes.data, data.nbytes, 0))
        rc = self._lib.sy_graph_launch(self.ctx.handle, graph)
        if rc == SY_ESTATE:  # the context's scratch moved since the capture: capture again
            self._lib.sy_graph_destroy(self.ctx.handle, graph)
            self._plan = None
            return None
        check(rc)
        outs = []
        for i, (ptr, length, oshape, alias) in enumerate(descr):
            if alias != i:
                outs.append(outs[alias])
                continue
            out = np.empty(oshape, np.float32)
            check(self._lib.sy_memcpy(self.ctx.handle, out.ctypes.data, ptr, out.nbytes, 1))
            outs.append(out)
        self.replayed_frames += 1
        return outs


# ---------------------------------------------------------------- DeviceOps

def transpose(owner: HipDeviceBackend, x: DeviceTensor, perm, shape) -> DeviceTensor:
    """DeviceOps.Transpose (DeviceExecution.cs:157-164)."""
    p = parameters(_count(x.shape))
    lead, st = 4 - len(x.shape), _strides(x.shape)
    for i in range(4):
        p[1 + i] = 1 if i < lead else shape[i - lead]
        p[5 + i] = 0 if i < lead else st[perm[i - lead]]
    return owner.compute(23, [x], shape, p, _count(x.shape))


def binary(owner: HipDeviceBackend, a: DeviceTensor, b: DeviceTensor, op: int) -> DeviceTensor:
    """DeviceOps.Binary (DeviceExecution.cs:128-139)."""
    shape = np.broadcast_shapes(a.shape, b.shape)
    p = parameters(_count(shape))
    ad = [1] * (4 - len(a.shape)) + list(a.shape)
    bd = [1] * (4 - len(b.shape)) + list(b.shape)
    yd = [1] * (4 - len(shape)) + list(shape)
    ast, bst = _strides(ad), _strides(bd)
    for d in range(4):
        p[1 + d] = yd[d]
        p[5 + d] = 0 if ad[d] == 1 else ast[d]
        p[9 + d] = 0 if bd[d] == 1 else bst[d]
    return owner.compute(op, [a, b], shape, p, _count(shape))


def max_pool(owner: HipDeviceBackend, x: DeviceTensor, k: int, s: int, pad: int) -> DeviceTensor:
    """TensorOps.Pool's device route (Compute.cs:677-693), square window, no ceil."""
    n, c, h, w = x.shape
    oh, ow = (h + 2 * pad - k) // s + 1, (w + 2 * pad - k) // s + 1
    shape = (n, c, oh, ow)
    p = parameters(_count(shape), h, w, oh, ow, k, k, s, s, pad, pad, 0, pad, pad, 0)
    return owner.compute(21, [x], shape, p, _count(shape))


def resize_nearest(owner: HipDeviceBackend, x: DeviceTensor, oh: int, ow: int) -> DeviceTensor:
    """TensorOps.ResizeNearest's device route (Compute.cs:715-721)."""
    n, c, h, w = x.shape
    shape = (n, c, oh, ow)
    return owner.compute(20, [x], shape, parameters(_count(shape), h, w, oh, ow), _count(shape))


# ---------------------------------------------------------------- the PtModel walk (YOLOv8 detect)

def _fold(w, gamma, beta, mean, var, eps):
    """PtModel.Prepare's BN fold through the library's host routine (sy_fold_bn)."""
    oc = w.shape[0]
    wo, bo = np.empty_like(w), np.empty(oc, np.float32)
    zero = np.zeros(oc, np.float32)
    N.lib().sy_fold_bn(fptr(w), oc, int(w.size // oc), fptr(zero), fptr(gamma), fptr(beta), fptr(mean), fptr(var),
                       ctypes.c_float(eps), fptr(wo), fptr(bo))
    return wo, bo


class _Params:
    """Consumes parameter tensors in state_dict order (sy_model_layout entries)."""

    def __init__(self, entries: np.ndarray, flat: np.ndarray, eps: float):
        self.entries, self.flat, self.eps, self.i, self.off = entries, flat, eps, 0, 0

    def take(self, kind: int, dims) -> np.ndarray:
        e = self.entries[self.i]
        if int(e[0]) != kind or tuple(int(d) for d in e[1:1 + len(dims)]) != tuple(dims):
            raise ValueError(f"parameter {self.i}: expected kind {kind} {dims}, layout has {e.tolist()}")
        n = int(np.prod(e[1:5]))
        v = self.flat[self.off:self.off + n].reshape(dims)
        self.i += 1
        self.off += n
        return np.ascontiguousarray(v, np.float32)

    def conv(self, ic, oc, k, s):
        """ultralytics Conv: conv weight + BatchNorm, folded; SiLU."""
        w = self.take(0, (oc, ic, k, k))
        g, b, m, v = (self.take(kind, (oc, 1, 1, 1)).reshape(oc) for kind in (1, 2, 3, 4))
        wf, bf = _fold(w, g, b, m, v, self.eps)
        return dict(w=wf, b=bf, k=k, s=s, silu=True)

    def conv2d(self, ic, oc, bias_kind):
        """nn.Conv2d 1x1 with its own bias (Detect's last conv of a branch)."""
        w = self.take(0, (oc, ic, 1, 1))
        b = self.take(bias_kind, (oc, 1, 1, 1)).reshape(oc)
        return dict(w=w, b=b, k=1, s=1, silu=False)


class YoloV8Walk:
    """PtModel.Forward over the modules of ultralytics yolov8.yaml (detect):
    Conv, C2f (+ Bottleneck), SPPF, Upsample, Concat, Detect, in the order
    PtModel.Run visits them."""

    def __init__(self, cfg: N.ModelConfig, params: np.ndarray):
        from . import synth
        if cfg.arch != N.ARCH_YOLOV8 or cfg.nm != 0:
            raise ValueError("the op-by-op walk covers the YOLOv8 detect models")
        entries = synth.layout(cfg)
        P = _Params(entries, np.asarray(params, np.float32), cfg.bn_eps)
        ch = lambda c: int(math.ceil(min(c, cfg.max_channels) * cfg.width / 8) * 8)
        rep = lambda n: max(round(n * cfg.depth), 1) if n > 1 else n
        self.nc, self.bins = cfg.nc, cfg.reg_max
        L = []  # (type, from, module)

        def c2f(c1, c2, n, shortcut):
            c = int(c2 * 0.5)
            m = dict(cv1=P.conv(c1, 2 * c, 1, 1), cv2=P.conv((2 + n) * c, c2, 1, 1), c=c,
                     m=[dict(cv1=P.conv(c, c, 3, 1), cv2=P.conv(c, c, 3, 1), add=shortcut) for _ in range(n)])
            return m

        c0, c1, c2, c3, c4 = ch(64), ch(128), ch(256), ch(512), ch(1024)
        L.append(("conv", -1, P.conv(3, c0, 3, 2)))
        L.append(("conv", -1, P.conv(c0, c1, 3, 2)))
        L.append(("c2f", -1, c2f(c1, c1, rep(3), True)))
        L.append(("conv", -1, P.conv(c1, c2, 3, 2)))
        L.append(("c2f", -1, c2f(c2, c2, rep(6), True)))
        L.append(("conv", -1, P.conv(c2, c3, 3, 2)))
        L.append(("c2f", -1, c2f(c3, c3, rep(6), True)))
        L.append(("conv", -1, P.conv(c3, c4, 3, 2)))
        L.append(("c2f", -1, c2f(c4, c4, rep(3), True)))
        L.append(("sppf", -1, dict(cv1=P.conv(c4, c4 // 2, 1, 1), cv2=P.conv(c4 // 2 * 4, c4, 1, 1))))
        L.append(("up", -1, None))
        L.append(("cat", (-1, 6), None))
        L.append(("c2f", -1, c2f(c4 + c3, c3, rep(3), False)))
        L.append(("up", -1, None))
        L.append(("cat", (-1, 4), None))
        L.append(("c2f", -1, c2f(c3 + c2, c2, rep(3), False)))
        L.append(("conv", -1, P.conv(c2, c2, 3, 2)))
        L.append(("cat", (-1, 12), None))
        L.append(("c2f", -1, c2f(c2 + c3, c3, rep(3), False)))
        L.append(("conv", -1, P.conv(c3, c3, 3, 2)))
        L.append(("cat", (-1, 9), None))
        L.append(("c2f", -1, c2f(c3 + c4, c4, rep(3), False)))
        chs = (c2, c3, c4)
        cb = max(16, chs[0] // 4, 4 * cfg.reg_max)
        cc = max(chs[0], min(cfg.nc, 100))
        boxes = [[P.conv(chs[i], cb, 3, 1), P.conv(cb, cb, 3, 1), P.conv2d(cb, 4 * cfg.reg_max, 5)] for i in range(3)]
        classes = [[P.conv(chs[i], cc, 3, 1), P.conv(cc, cc, 3, 1), P.conv2d(cc, cfg.nc, 6)] for i in range(3)]
        L.append(("detect", (15, 18, 21), dict(boxes=boxes, classes=classes, strides=(8.0, 16.0, 32.0))))
        if P.i != len(entries):
            raise ValueError("parameter layout not fully consumed")
        self.layers = L

    # PtModel.Conv -> TensorOps.Conv -> IDeviceBackend.DeviceConv
    @staticmethod
    def _conv(be, m, x):
        n, _, h, w = x.shape
        k, s, p = m["k"], m["s"], m["k"] // 2
        oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
        shape = (n, m["w"].shape[0], oh, ow)
        return be.device_conv(x, m["w"], m["b"], shape, (s, s), (p, p, p, p), (1, 1), 1, m["silu"])

    def _c2f(self, be, m, x):
        y = self._conv(be, m["cv1"], x)
        n, c2, h, w = y.shape
        half = (n, c2 // 2, h, w)
        ys = [be.device_slice(y, half, 1, 0), be.device_slice(y, half, 1, c2 // 2)]  # Chunk
        for b in m["m"]:
            t = self._conv(be, b["cv2"], self._conv(be, b["cv1"], ys[-1]))
            ys.append(binary(be, ys[-1], t, 10) if b["add"] else t)  # x + f(x)
        cat = be.device_concat(ys, 1, (n, sum(t.shape[1] for t in ys), h, w))
        return self._conv(be, m["cv2"], cat)

    def _sppf(self, be, m, x):
        sp = [self._conv(be, m["cv1"], x)]
        for _ in range(3):
            sp.append(max_pool(be, sp[-1], 5, 1, 2))
        n, c, h, w = sp[0].shape
        return self._conv(be, m["cv2"], be.device_concat(sp, 1, (n, 4 * c, h, w)))

    def _detect(self, be, m, xs):
        levels = []
        for i, x in enumerate(xs):
            b, c = x, x
            for conv in m["boxes"][i]:
                b = self._conv(be, conv, b)
            for conv in m["classes"][i]:
                c = self._conv(be, conv, c)
            levels.append((b, c, m["strides"][i]))
        n = xs[0].shape[0]
        total = sum(x.shape[2] * x.shape[3] for x in xs)
        return be.decode_head_levels(levels, (n, self.nc + 4, total), self.bins, False)

    def run(self, be: HipDeviceBackend, x: np.ndarray) -> DeviceTensor:
        values = []
        cur = x
        for kind, src, m in self.layers:
            arg = cur if src == -1 else None
            if kind == "conv":
                cur = self._conv(be, m, arg)
            elif kind == "c2f":
                cur = self._c2f(be, m, arg)
            elif kind == "sppf":
                cur = self._sppf(be, m, arg)
            elif kind == "up":
                cur = resize_nearest(be, arg, arg.shape[2] * 2, arg.shape[3] * 2)
            elif kind == "cat":
                parts = [cur if j == -1 else values[j] for j in src]
                n, _, h, w = parts[0].shape
                cur = be.device_concat(parts, 1, (n, sum(t.shape[1] for t in parts), h, w))
            else:
                cur = self._detect(be, m, [values[j] for j in src])
            values.append(cur)
        return cur


class DeviceRouteDetector:
    """YoloDetector.PredictRaw over the op-by-op route (YoloDetector.cs:262-313)."""

    def __init__(self, cfg: N.ModelConfig, params: np.ndarray, device: int = 0, replay: bool = True):
        self.walk = YoloV8Walk(cfg, params)
        self.backend = HipDeviceBackend(device, replay)

    def close(self):
        self.backend.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def predict_raw(self, x: np.ndarray) -> np.ndarray:
        be = self.backend
        cached = be.try_replay(x)
        if cached is not None:
            return cached[0]
        be.begin_frame()
        try:
            be.begin_replay_capture(x)
            out = self.walk.run(be, x)
            return be.materialize_outputs([out])[0]
        finally:
            be.end_frame()
