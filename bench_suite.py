"""Measurements beside the headline bench line: the per-layer microbench
(3x3 s1/s2, 1x1, maxpool5 at YOLOv8n/s shapes, batch 1 and 32), whole-model
throughput for the other model configurations (YOLO11n, YOLOv8m batch 64,
Segment models) and the post-processing kernels (end-to-end top-k, mask
decode, NMS candidates, device letterbox).  All inputs are synthetic and
seeded; every figure is HIP-event time on the library stream.

    python bench_suite.py --section layers|models|post|bandwidth|route
    rocprofv3 --kernel-trace --output-format csv -d DIR -o bw -- python bench_suite.py --section bandwidth > LOG
    python bench_suite.py --trace DIR/bw_kernel_trace.csv LOG
    rocprofv3 --kernel-trace --output-format csv -d DIR -o kt -- python bench.py --eager ... > BENCH_LOG
    python bench_suite.py --forward-trace DIR/kt_kernel_trace.csv STEPS BENCH_LOG
    python bench_suite.py --pmc-traffic FETCH_CSV WRITE_CSV BENCH_LOG   (two --pmc passes, with --copy-probe-mib)
    python bench_suite.py --pmc-mfma MFMA_CSV BENCH_LOG

Per kernel it prints the algorithmic work of one launch (flops, bytes: the
minimum data a launch must move, not counting re-reads) and the fraction of
the MI355X roof that bounds it (FP32 MFMA 157.3 TFLOP/s, HBM 8 TB/s).
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from bench import PEAK_FP32_MFMA_TFLOPS, PEAK_HBM_GBS, RIDGE  # noqa: E402


def out(msg=""):
    print(msg, flush=True)


def time_ms(ctx, fn, iters=20, warm=3):
    for _ in range(warm):
        fn()
    ctx.flush()
    ctx.timer_start()
    for _ in range(iters):
        fn()
    return ctx.timer_stop() / iters


def kernels(ctx, fn, reps=3):
    """{profile name: (launches, avg us, flops/launch, bytes/launch)} of fn's launches."""
    ctx.profile_enable(True)
    for _ in range(reps):
        fn()
    ctx.flush()
    prof = ctx.profile_read()
    ctx.profile_enable(False)
    return {k: (c // reps, 1e3 * ms / c, fl / c, by / c) for k, (c, ms, fl, by) in prof.items()}


def roof(flops, nbytes, us):
    if us <= 0:
        return "-"
    if flops > 0 and flops / max(nbytes, 1.0) > RIDGE:
        a = flops / (us * 1e-6) / 1e12
        return f"{a:7.1f} TFLOP/s {100 * a / PEAK_FP32_MFMA_TFLOPS:5.1f}% mfma"
    a = nbytes / (us * 1e-6) / 1e9
    return f"{a:7.0f} GB/s    {100 * a / PEAK_HBM_GBS:5.1f}% hbm "


def kernel_lines(prof, indent="    "):
    for k, (n, us, fl, by) in sorted(prof.items(), key=lambda kv: -kv[1][0] * kv[1][1]):
        out(f"{indent}{k:<26} x{n:<3} {us:9.1f} us  {fl / 1e9:8.3f} GF {by / 1e6:9.2f} MB  {roof(fl, by, us)}")


# ------------------------------------------------------------------ layers

def section_layers():
    from simdyolo_amd import synth
    from simdyolo_amd.device import HipContext
    hip = HipContext(0)
    out(f"# device: {hip.name}")
    out("# conv cases: autotuned algorithm (first call times the candidates); total = HIP-event average")
    out("#   over 20 calls; 'direct' = 2*9*ic*oc*OH*OW*B flops / total time (the Winograd GEMM executes less).")
    cases = []
    for b in (1, 32):
        for c in (32, 64, 128, 256):
            for s in (160, 80, 40, 20):
                cases.append((f"3x3 s1 {c}->{c} @{s}", b, c, s, s, c, 3, 1))
        cases.append(("3x3 s2 3->16 @640 (stem, NCHW)", b, 3, 640, 640, 16, 3, 2))
        cases.append(("3x3 s2 64->128 @80", b, 64, 80, 80, 128, 3, 2))
        cases.append(("1x1 128->256 @40", b, 128, 40, 40, 256, 1, 1))
    for name, b, ic, h, w, oc, k, s in cases:
        hip.begin_frame()
        try:
            wt = synth.kaiming((oc, ic, k, k), ic + oc)
            bias = synth.activations((oc,), oc) * np.float32(0.1)
            p = k // 2
            conv = hip.conv_create(wt, bias, (s, s), (p, p, p, p), silu=True)
            if ic == 3:
                from simdyolo_amd import Tensor
                ptr = hip.malloc(b * 3 * h * w * 4)
                x = Tensor(ptr, b, 3, h, w, 3, 1)
            else:
                x = hip.alloc(b, ic, h, w)
                ptr = None
            oh, ow = hip.conv_out_size(conv, h, w)
            y = hip.alloc(b, oc, oh, ow)
            hip.conv(conv, x, y)  # tunes
            ms = time_ms(hip, lambda: hip.conv(conv, x, y))
            prof = kernels(hip, lambda: hip.conv(conv, x, y))
            direct = 2.0 * ic * oc * k * k * oh * ow * b
            out(f"B={b:<2} {name:<32} {1e3 * ms:9.1f} us total  {direct / (ms * 1e-3) / 1e12:7.1f} TFLOP/s direct")
            kernel_lines(prof)
            if ptr:
                hip.free(ptr)
        finally:
            hip.end_frame()
    for b in (1, 32):
        hip.begin_frame()
        try:
            x = hip.alloc(b, 256, 20, 20)
            y = hip.alloc(b, 256, 20, 20)
            ms = time_ms(hip, lambda: hip.maxpool(x, y, (5, 5), (1, 1), (2, 2, 2, 2)))
            nbytes = 2 * 4.0 * b * 256 * 400
            out(f"B={b:<2} {'maxpool5 s1 p2 @20x20x256':<32} {1e3 * ms:9.1f} us total  "
                f"{roof(0, nbytes, 1e3 * ms)}")
            buf = hip.alloc(b, 4 * 256, 20, 20)
            sl = [buf.slice(i * 256, 256) for i in range(4)]
            ms = time_ms(hip, lambda: hip.sppf_pool(*sl))
            nbytes = 4 * 4.0 * b * 256 * 400
            out(f"B={b:<2} {'SPPF 3x maxpool5 @20x20x256':<32} {1e3 * ms:9.1f} us total  "
                f"{roof(0, nbytes, 1e3 * ms)}")
        finally:
            hip.end_frame()
    hip.close()


# ------------------------------------------------------------------ models

def model_line(hip, name, cfg, batch, size, steps):
    from simdyolo_amd import synth
    from simdyolo_amd.detector import YoloDetector
    det = YoloDetector(cfg, synth.params(cfg), ctx=hip)
    try:
        inp, _ = det.buffers(batch, size, size)
        hip.h2d(inp, synth.images(batch, size, size))
        for _ in range(3):
            det.run(batch, size, size)
        ms = time_ms(hip, lambda: det.run(batch, size, size), iters=steps, warm=2)
        out(f"{name:<28} B={batch:<3} {ms:9.3f} ms/step  {batch / (ms * 1e-3):10.1f} images/s  (hipGraph replay)")
        arena, unshared, scratch = det.plan_memory(batch, size, size)
        wbytes, _ = det.memory()
        out(f"    memory: activation arena {arena / 2**20:.2f} MiB (liveness-shared; {unshared / 2**20:.2f} MiB "
            f"unshared), scratch {scratch / 2**20:.2f} MiB, weights {wbytes / 2**20:.2f} MiB")
        det.set_graph(False)
        prof = kernels(hip, lambda: det.run(batch, size, size), reps=2)
        det.set_graph(True)
        tot = sum(n * us for n, us, _, _ in prof.values())
        out(f"    eager kernel sum {tot / 1e3:.3f} ms; kernels by share:")
        for k, (n, us, fl, by) in sorted(prof.items(), key=lambda kv: -kv[1][0] * kv[1][1])[:10]:
            out(f"    {k:<26} x{n:<3} {100 * n * us / tot:5.1f}%  avg {us:8.1f} us  {roof(fl, by, us)}")
    finally:
        det.close()


def section_models():
    from simdyolo_amd import synth
    from simdyolo_amd.device import HipContext
    hip = HipContext(0)
    out(f"# device: {hip.name}")
    out("# whole forward (stem .. joined head decode), seeded random-init weights, uniform u8 pixels / 255")
    model_line(hip, "YOLOv8n 640", synth.config("n"), 1, 640, 100)
    model_line(hip, "YOLOv8n 640", synth.config("n"), 32, 640, 20)
    model_line(hip, "YOLO11n 640", synth.config("n", arch="yolo11"), 1, 640, 100)
    model_line(hip, "YOLO11n 640", synth.config("n", arch="yolo11"), 32, 640, 20)
    model_line(hip, "YOLOv8n-seg 640 (nm 32)", synth.config("n", nm=32, npr=256), 1, 640, 100)
    model_line(hip, "YOLO11n-seg 640 (nm 32)", synth.config("n", arch="yolo11", nm=32, npr=256), 1, 640, 100)
    model_line(hip, "YOLO26n-seg 640 (e2e, nm 32)", synth.config("n", arch="yolo26", nm=32, npr=256), 1, 640, 100)
    model_line(hip, "YOLO26n-seg 640 (e2e, nm 32)", synth.config("n", arch="yolo26", nm=32, npr=256), 32, 640, 20)
    model_line(hip, "YOLOv8m 640", synth.config("m"), 64, 640, 5)
    hip.close()


# ------------------------------------------------------------------ op-by-op device route

def section_route():
    """YOLOv8n 640 through the op-by-op route that integration/csharp/HipBackend.cs
    drives (each conv bracketed by op-23 transposes, module glue as generic
    ops), beside the whole-model entry points: host input in, host head out
    per call (PCIe included) for both, and the resident graph replay of
    sy_model_run.  Also the op-23 NCHW -> NHWC transpose on its own."""
    import time
    from simdyolo_amd import synth
    from simdyolo_amd.detector import YoloDetector
    from simdyolo_amd.device import HipContext
    from simdyolo_amd.device_route import DeviceRouteDetector, transpose
    cfg = synth.config("n")
    params = synth.params(cfg)
    out("# YOLOv8n 640, seeded random-init weights; host NCHW input -> host [B, 84, 8400] head per call")

    def wall(fn, iters):
        fn()
        t = time.perf_counter()
        for _ in range(iters):
            fn()
        return (time.perf_counter() - t) / iters * 1e3

    for batch, iters in ((1, 40), (32, 5)):
        x = synth.images(batch, 640, 640)
        with DeviceRouteDetector(cfg, params, replay=False) as det:
            det.predict_raw(x)
            ms = wall(lambda: det.predict_raw(x), iters)
            out(f"route, op by op (no replay)      B={batch:<3} {ms:9.3f} ms/call {batch / (ms * 1e-3):9.1f} images/s")
            be = det.backend
            be.ctx.profile_enable(True)
            det.predict_raw(x)
            prof = be.ctx.profile_read()
            be.ctx.profile_enable(False)
            tot = sum(ms_ for _, ms_, _, _ in prof.values())
            out(f"    eager kernel sum {tot:.3f} ms; by kernel:")
            for k, (n, ms_, fl, by) in sorted(prof.items(), key=lambda kv: -kv[1][1])[:8]:
                us = 1e3 * ms_ / n
                out(f"    {k:<30} x{n:<4} {100 * ms_ / tot:5.1f}%  avg {us:8.1f} us  {roof(fl / n, by / n, us)}")
        with DeviceRouteDetector(cfg, params) as det:
            for _ in range(2):
                det.predict_raw(x)
            ms = wall(lambda: det.predict_raw(x), iters)
            assert det.backend.replayed_frames >= iters
            out(f"route, graph replay (TryReplay)  B={batch:<3} {ms:9.3f} ms/call {batch / (ms * 1e-3):9.1f} images/s")
        hip = HipContext(0)
        with YoloDetector(cfg, params, ctx=hip) as det:
            for _ in range(2):
                det.predict_raw(x)
            ms = wall(lambda: det.predict_raw(x), iters)
            out(f"sy_model_predict_raw             B={batch:<3} {ms:9.3f} ms/call {batch / (ms * 1e-3):9.1f} images/s")
            inp, _ = det.buffers(batch, 640, 640)
            hip.h2d(inp, x)
            for _ in range(3):
                det.run(batch, 640, 640)
            ms = time_ms(hip, lambda: det.run(batch, 640, 640), iters=20, warm=2)
            out(f"sy_model_run (resident, graph)   B={batch:<3} {ms:9.3f} ms/step {batch / (ms * 1e-3):9.1f} images/s")
        hip.close()
    # op 23 on its own: [1, 64, 160, 160] NCHW -> NHWC and back.
    from simdyolo_amd.device_route import HipDeviceBackend
    with HipDeviceBackend(0, replay=False) as be:
        be.begin_frame()
        try:
            x = synth.activations((1, 64, 160, 160), 3)
            d = be.upload(x)
            nbytes = 2 * 4 * x.size
            for name, src, perm, shape in (("NCHW->NHWC", d, (0, 2, 3, 1), (1, 160, 160, 64)),
                                           ("NHWC->NCHW", None, (0, 3, 1, 2), (1, 64, 160, 160))):
                src = src or transpose(be, d, (0, 2, 3, 1), (1, 160, 160, 64))
                be.ctx.flush()
                ms = time_ms(be.ctx, lambda: transpose(be, src, perm, shape), iters=50, warm=5)
                prof = kernels(be.ctx, lambda: transpose(be, src, perm, shape), reps=5)
                (k, (n, us, fl, by)), = prof.items()
                out(f"op 23 {name} [1, 64, 160, 160]: {k} {us:.1f} us/launch (events), "
                    f"{by / 1e6:.2f} MB -> {roof(fl, by, us)}; back to back {ms * 1e3:.1f} us")
        finally:
            be.end_frame()


# ------------------------------------------------------------------ post

def section_post():
    from simdyolo_amd import _native as N
    from simdyolo_amd import synth
    from simdyolo_amd.device import HipContext
    hip = HipContext(0)
    lib = N.lib()
    out(f"# device: {hip.name}")
    rng = np.random.Generator(np.random.PCG64(11))
    # End-to-end two-stage top-k (k = 300 of 8400 anchors, 80 classes).
    for batch, extra in ((1, 32), (32, 0), (32, 32)):
        ch, anchors, nc, k = 84 + extra, 8400, 80, 300
        head = rng.standard_normal((batch, ch, anchors)).astype(np.float32)
        src = hip.malloc(head.nbytes)
        dst = hip.malloc(batch * k * (6 + extra) * 4)
        try:
            hip.h2d(src, head)
            fn = lambda: hip.e2e_topk(src, batch, ch, anchors, nc, k, False, dst)  # noqa: E731
            ms = time_ms(hip, fn)
            prof = kernels(hip, fn)
            out(f"e2e top-k B={batch:<2} [{ch}, {anchors}] k={k}: {1e3 * ms:8.1f} us total")
            kernel_lines(prof)
        finally:
            hip.free(src)
            hip.free(dst)
    # NMS candidate stage (compaction + sort of the anchors over threshold).
    for batch in (1, 32):
        head = rng.standard_normal((batch, 84, 8400)).astype(np.float32)
        head[:, 4:] = (head[:, 4:] * 0.3 - 2.0)  # a few hundred anchors above 0.25 per image
        src = hip.malloc(head.nbytes)
        cand = hip.malloc(batch * 30000 * ctypes.sizeof(N.DetectionT))
        cnt = hip.malloc(4 * batch)
        opt = N.DecodeOptions(0.25, 0.45, 300, 30000, 80, 0, 0)
        try:
            hip.h2d(src, head)
            fn = lambda: N.check(lib.sy_nms_candidates(hip.handle, src, batch, 84, 8400,  # noqa: E731
                                                       ctypes.byref(opt), cand, cnt))
            ms = time_ms(hip, fn)
            prof = kernels(hip, fn)
            out(f"NMS candidates B={batch:<2} [84, 8400]: {1e3 * ms:8.1f} us total")
            kernel_lines(prof)
        finally:
            hip.free(src)
            hip.free(cand)
            hip.free(cnt)
    # Instance masks: 300 instances, 32 x 160 x 160 prototypes, 640x480 source.
    hip.begin_frame()
    try:
        W, H, nm, kk = 640, 480, 32, 300
        proto = hip.upload(synth.activations((1, nm, 160, 160), 6))
        coeffs = synth.activations((kk, nm), 7) * np.float32(0.3)
        xy = rng.uniform(0, 1, (kk, 2)) * np.array([W - 80, H - 80])
        wh = rng.uniform(8, 80, (kk, 2))
        boxes = [(float(a), float(b), float(c), float(d)) for (a, b), (c, d) in zip(xy, wh)]
        t = N.LetterboxT(W, H, 640, 640, 1.0, 1.0, 0, 80)
        cap = int(sum((int(np.ceil(b[0] + b[2])) - int(b[0])) * (int(np.ceil(b[1] + b[3])) - int(b[1]))
                      for b in boxes))
        cbuf = hip.malloc(coeffs.nbytes)
        mbuf = hip.malloc(cap * 4)
        dets = (N.DetectionT * kk)(*[N.DetectionT(0, 1.0, *b, 0) for b in boxes])
        info = (N.MaskInfo * kk)()
        try:
            hip.h2d(cbuf, coeffs)
            fn = lambda: N.check(lib.sy_mask_decode(hip.handle, ctypes.byref(proto), cbuf, nm, kk, dets,  # noqa: E731
                                                    ctypes.byref(t), mbuf, cap, info))
            ms = time_ms(hip, fn, iters=10)
            prof = kernels(hip, fn)
            out(f"mask decode k={kk} protos [{nm},160,160] source {W}x{H}: {1e3 * ms:8.1f} us per call "
                f"(synchronous C call: host instance records, one upload, GEMM, crop)")
            kernel_lines(prof)
        finally:
            hip.free(cbuf)
            hip.free(mbuf)
    finally:
        hip.end_frame()
    # Device letterbox: 1920x1080 RGB24 -> 640x640 NCHW floats.
    for (w, h) in ((1920, 1080), (640, 640)):
        img = rng.integers(0, 256, size=(h, w * 3), dtype=np.uint8)
        src = hip.malloc(img.nbytes)
        dst = hip.malloc(3 * 640 * 640 * 4)
        lt = N.LetterboxT()
        try:
            hip.h2d(src, img)
            fn = lambda: N.check(lib.sy_letterbox_device(hip.handle, src, w, h, 640, 640, 0, 0, dst,  # noqa: E731
                                                         ctypes.byref(lt)))
            ms = time_ms(hip, fn)
            prof = kernels(hip, fn)
            out(f"letterbox {w}x{h} -> 640x640: {1e3 * ms:8.1f} us total")
            kernel_lines(prof)
        finally:
            hip.free(src)
            hip.free(dst)
    hip.close()

# ----------------------------------------------------------------- bandwidth

BW_REPS = 20


def _marker(hip, buf, i):
    """A plain 4-channel copy whose grid (i + 1 workgroups of 256 threads)
    tags the start of case i in a kernel trace."""
    from simdyolo_amd import Tensor
    t_in = Tensor(buf, 1, 4, 256 * (i + 1), 1, 4, 0)
    t_out = Tensor(buf + 4 * 4 * 256 * 64, 1, 4, 256 * (i + 1), 1, 4, 0)
    hip.copy(t_in, t_out)


def section_bandwidth():
    """HBM-bound kernels at batch 32 (and top-k / NMS at batch 1) next to plain
    device copies of similar sizes, each case preceded by a marker launch so
    that `--trace` can attribute a rocprofv3 kernel trace of this run to the
    cases.  Prints the case list (labels and each kernel's algorithmic bytes
    per launch) as one JSON line."""
    import json
    from simdyolo_amd import Tensor, _native as N
    from simdyolo_amd import synth
    from simdyolo_amd.device import HipContext
    hip = HipContext(0)
    lib = N.lib()
    out(f"# device: {hip.name}")
    rng = np.random.Generator(np.random.PCG64(13))
    mark = hip.malloc(4 * 4 * 256 * 128)
    cases = []

    def run(label, fn):
        i = len(cases)
        fn()  # warm (and packs weights)
        hip.flush()
        prof = kernels(hip, fn, reps=2)
        _marker(hip, mark, i)
        for _ in range(BW_REPS):
            fn()
        hip.flush()
        cases.append({"label": label, "kernels": {k: [v[0], v[3]] for k, v in prof.items()},
                      "per_call": sum(v[0] for v in prof.values())})
        out(f"{label}: " + ", ".join(f"{k} {v[1]:.1f} us (events)" for k, v in prof.items()))

    hip.begin_frame()
    try:
        # Plain copies: the reachable rate for a launch moving this many bytes
        # (6 to 210 MiB: the sizes of the depthwise, pool and transpose cases).
        for mb in (3, 6, 13, 16, 26, 52, 105):
            px = mb * 1024 * 1024 // (4 * 256)
            a, b = hip.alloc(1, 256, 1, px), hip.alloc(1, 256, 1, px)
            run(f"copy {2 * mb} MiB (read {mb} + write {mb})", lambda a=a, b=b: hip.copy(a, b))
        # Depthwise 3x3 at the YOLO11n batch-32 shapes: each of the four
        # kernels pinned (algorithm fixed, so SIMDYOLO_HIP_TILE picks it).
        from simdyolo_amd import CONV_DEPTHWISE
        for c, hw in ((64, 80), (128, 40), (256, 20), (80, 80), (80, 40), (80, 20)):
            x = hip.upload(synth.activations((32, c, hw, hw), c + hw))
            y = hip.alloc(32, c, hw, hw)
            conv = hip.conv_create(synth.kaiming((c, 1, 3, 3), 3), synth.activations((c,), 4), (1, 1),
                                   (1, 1, 1, 1), groups=c, silu=True)
            hip.conv_set_algo(conv, CONV_DEPTHWISE)
            for tile, kern in enumerate(("register", "tile", "column4", "column8")):
                os.environ["SIMDYOLO_HIP_TILE"] = str(tile)
                run(f"depthwise 3x3 {c}@{hw} B=32 ({kern})", lambda conv=conv, x=x, y=y: hip.conv(conv, x, y))
                os.environ.pop("SIMDYOLO_HIP_TILE", None)
        # Max pool 5x5 and the SPPF chain at 20x20 (YOLOv8n: 128 channels; microbench: 256).
        for c in (128, 256):
            x = hip.upload(synth.activations((32, c, 20, 20), c))
            buf = hip.alloc(32, 3 * c, 20, 20)
            ys = [buf.slice(i * c, c) for i in range(3)]
            run(f"maxpool5 20x20x{c} B=32", lambda x=x, ys=ys: hip.maxpool(x, ys[0], (5, 5), (1, 1), (2, 2, 2, 2)))
            run(f"SPPF 20x20x{c} B=32", lambda x=x, ys=ys: hip.sppf_pool(x, *ys))
        # Winograd input transform at the largest YOLOv8n batch-32 layer.
        x = hip.upload(synth.activations((32, 64, 80, 80), 5))
        y = hip.alloc(32, 64, 80, 80)
        from simdyolo_amd import CONV_WINOGRAD, CONV_WINOGRAD2
        conv = hip.conv_create(synth.kaiming((64, 64, 3, 3), 6), None, (1, 1), (1, 1, 1, 1), silu=True)
        hip.conv_set_algo(conv, CONV_WINOGRAD2)
        run("Winograd 3x3 64@80 B=32 (input transform + planes)", lambda: hip.conv(conv, x, y))
        # The fused forms (transform inside the planes kernel) on the same layer.
        hip.conv_set_algo(conv, CONV_WINOGRAD)
        for form, name in ((0, "four-wave"), (1, "warp-specialized"), (2, "two groups")):
            os.environ["SIMDYOLO_HIP_TILE"] = str(form)
            run(f"Winograd 3x3 64@80 B=32 (fused, {name})", lambda: hip.conv(conv, x, y))
        os.environ.pop("SIMDYOLO_HIP_TILE", None)
        # Generic device ops (sy_compute) at the op-by-op route's shapes: the
        # op-23 NCHW <-> NHWC transposes around every conv, a shortcut add.
        from simdyolo_amd.device_route import parameters
        for shape in ((1, 64, 160, 160), (32, 64, 80, 80)):
            n, c, h, w = shape
            cnt = n * c * h * w
            a, b = hip.malloc(4 * cnt), hip.malloc(4 * cnt)
            hip.h2d(a, synth.activations(shape, 9))
            tp = parameters(cnt, n, h, w, c, c * h * w, w, 1, h * w)          # NCHW -> NHWC
            tb = parameters(cnt, n, c, h, w, h * w * c, 1, w * c, c)          # NHWC -> NCHW
            run(f"op 23 NCHW->NHWC {list(shape)}", lambda a=a, b=b, tp=tp, cnt=cnt: hip.compute(23, [(a, cnt)], tp, cnt, b, cnt))
            run(f"op 23 NHWC->NCHW {list(shape)}", lambda a=a, b=b, tb=tb, cnt=cnt: hip.compute(23, [(b, cnt)], tb, cnt, a, cnt))
            ad = parameters(cnt, n, c, h, w, c * h * w, h * w, w, 1, c * h * w, h * w, w, 1)
            run(f"op 10 add {list(shape)}", lambda a=a, b=b, ad=ad, cnt=cnt: hip.compute(10, [(a, cnt), (b, cnt)], ad, cnt, a, cnt))
            hip.free(a)
            hip.free(b)
    finally:
        hip.end_frame()
    # End-to-end top-k and the NMS candidate stage on [B, 84, 8400] heads.
    for batch in (32, 1):
        head = rng.standard_normal((batch, 84, 8400)).astype(np.float32)
        head[:, 4:] = head[:, 4:] * 0.3 - 2.0
        src = hip.malloc(head.nbytes)
        dst = hip.malloc(batch * 300 * 6 * 4)
        cand = hip.malloc(batch * 30000 * ctypes.sizeof(N.DetectionT))
        cnt = hip.malloc(4 * batch)
        opt = N.DecodeOptions(0.25, 0.45, 300, 30000, 80, 0, 0)
        try:
            hip.h2d(src, head)
            run(f"e2e top-k B={batch} [84, 8400] k=300",
                lambda: hip.e2e_topk(src, batch, 84, 8400, 80, 300, False, dst))
            run(f"NMS candidates B={batch} [84, 8400]",
                lambda: N.check(lib.sy_nms_candidates(hip.handle, src, batch, 84, 8400, ctypes.byref(opt), cand,
                                                      cnt)))
        finally:
            for ptr in (src, dst, cand, cnt):
                hip.free(ptr)
    hip.free(mark)
    hip.close()
    print(json.dumps({"bandwidth_cases": cases, "reps": BW_REPS}), flush=True)


def summarize_trace(trace_csv, log):
    """Per case and kernel: the median kernel-trace duration (End - Start) of the
    timed launches after the case's marker, the library's algorithmic bytes
    per launch, and the rate against MI355X's 8 TB/s."""
    import csv
    import json
    import statistics
    from bench import symbol
    meta = None
    with open(log) as f:
        for line in f:
            if line.startswith("{") and "bandwidth_cases" in line:
                meta = json.loads(line)
    cases, reps = meta["bandwidth_cases"], meta["reps"]
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    name = lambda r: r["Kernel_Name"].split("(")[0].replace("void ", "")  # noqa: E731
    marks = {}
    for i, r in enumerate(rows):
        if "binary4_kernel" in name(r) and int(r["Workgroup_Size_X"]) == 256:
            g = int(r["Grid_Size_X"]) // 256
            if 1 <= g <= len(cases) and g - 1 not in marks:
                marks[g - 1] = i
    out(f"# {'case / kernel':<58} {'launches':>8} {'median us':>10} {'algo MB':>9} {'GB/s':>8} {'of 8 TB/s':>10}")
    for ci, case in enumerate(cases):
        lo = marks[ci] + 1
        seg = rows[lo:lo + reps * case["per_call"]]  # this case's timed launches
        out(case["label"])
        per = {}
        for r in seg:
            per.setdefault(name(r), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        lib_names = list(case["kernels"])
        for k, d in per.items():
            nbytes = None
            if len(per) == 1 and len(lib_names) == 1:
                nbytes = case["kernels"][lib_names[0]][1]
            else:
                for lib_name, (_, b) in case["kernels"].items():
                    sym = symbol(lib_name)
                    if sym and (sym == k or ("*" in sym and k.startswith(sym.split("<")[0]))):
                        nbytes = b
            med = statistics.median(d)
            line = f"    {k:<56} {len(d) // reps:8d} {med:10.2f}"
            if nbytes:
                gbs = nbytes / (med * 1e-6) / 1e9
                line += f" {nbytes / 1e6:9.2f} {gbs:8.0f} {100 * gbs / PEAK_HBM_GBS:9.1f}%"
            out(line)


def summarize_forward_trace(trace_csv, steps, bench_log):
    """Per kernel symbol of an eager `bench.py` run under the kernel tracer:
    launches per forward, time per forward, average End-Start duration and
    share, over the last `steps` forwards (a forward ends with the head
    decode; the earlier ones include the autotuner's timing launches).  The
    bench line's own per-launch HIP-event averages are listed beside them."""
    import collections
    import csv
    import json
    from bench import symbol
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    name = lambda r: r["Kernel_Name"].split("(")[0].replace("void ", "")  # noqa: E731
    ends = [i for i, r in enumerate(rows) if name(r) == "sy::decode_kernel"]
    if len(ends) <= steps:
        raise SystemExit(f"the trace holds {len(ends)} forwards, fewer than {steps} + 1")
    seg = rows[ends[-steps - 1] + 1:ends[-1] + 1]
    agg = collections.defaultdict(list)
    for r in seg:
        agg[name(r)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    bench = {}
    with open(bench_log) as f:
        for line in f:
            if line.startswith("{") and '"kernels"' in line:
                for k in json.loads(line)["kernels"]:
                    sym = symbol(k["kernel"])
                    if sym:
                        bench[sym] = (k["avg_launch_us"], k["kernel"])
    total = sum(sum(v) for v in agg.values()) / steps
    out(f"# {steps} steady-state forwards of eager launches; total kernel time per forward {total / 1e3:.3f} ms")
    out(f"# {'symbol':<52} {'calls/step':>10} {'ms/step':>8} {'avg us':>8} {'share %':>8} {'bench avg us':>13}"
        f"  bench name")
    for k, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        b = bench.get(k)
        out(f"{k:<54} {len(v) / steps:10.2f} {sum(v) / steps / 1e3:8.3f} {sum(v) / len(v):8.2f} "
            f"{100 * sum(v) / steps / total:8.2f} {b[0] if b else float('nan'):13.2f}  {b[1] if b else '-'}")


def _pmc_forwards(csv_path):
    """{counter: {symbol: [values per dispatch]}} over the forwards of an eager
    bench.py run after its first one (which may time autotuning candidates),
    plus the dispatches after the last forward (the copy probe)."""
    import collections
    import csv
    rows = sorted(csv.DictReader(open(csv_path)), key=lambda r: int(r["Dispatch_Id"]))
    name = lambda r: r["Kernel_Name"].split("(")[0].replace("void ", "")  # noqa: E731
    ids = sorted({int(r["Dispatch_Id"]) for r in rows})
    kname = {int(r["Dispatch_Id"]): name(r) for r in rows}
    ends = [d for d in ids if kname[d] == "sy::decode_kernel"]
    if len(ends) < 2:
        raise SystemExit(f"{csv_path}: fewer than two forwards")
    first, last = ends[0], ends[-1]
    fwd = collections.defaultdict(lambda: collections.defaultdict(list))
    tail = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in rows:
        d = int(r["Dispatch_Id"])
        dst = fwd if first < d <= last else tail if d > last else None
        if dst is not None:
            dst[r["Counter_Name"]][name(r)].append(float(r["Counter_Value"]))
    return fwd, tail, len(ends) - 1


def _bench_kernels(bench_log):
    """{symbol: (profile name, algorithmic flops per launch, bytes per launch)}
    from the bench line's eager per-kernel table."""
    import json
    from bench import symbol
    out_ = {}
    with open(bench_log) as f:
        for line in f:
            if line.startswith("{") and '"kernels"' in line:
                for k in json.loads(line)["kernels"]:
                    sym = symbol(k["kernel"])
                    if sym and "*" not in sym:
                        out_[sym] = (k["kernel"], k["flops_per_launch"], k["bytes_per_launch"])
    return out_


def _label(sym):
    """Bench profile name of a fixed-kernel symbol, else the symbol without spaces."""
    from bench import SYMBOLS
    names = [k for k, v in SYMBOLS.items() if v == sym]
    return names[0] if names else sym.replace(", ", ",")


def summarize_pmc_traffic(fetch_csv, write_csv, bench_log):
    """HBM bytes per launch from FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by what the counter reads for the copy probe (the
    largest plain copy after the forwards: it reads and writes the same
    known byte count)."""
    fwd_f, tail_f, nf = _pmc_forwards(fetch_csv)
    fwd_w, tail_w, _ = _pmc_forwards(write_csv)
    copy = "sy::binary4_kernel<false>"
    fc, wc = max(tail_f["FETCH_SIZE"].get(copy, [0.0])), max(tail_w["WRITE_SIZE"].get(copy, [0.0]))
    if not fc or not wc:
        raise SystemExit("no copy-probe dispatch after the forwards (run bench.py with --copy-probe-mib)")
    # The probe copies a whole number of MiB; its write count is (almost) exact.
    kib = round(wc / 1024.0) * 1024.0
    fs, ws = fc / kib, wc / kib
    algo = _bench_kernels(bench_log)
    out(f"# calibration: a plain copy of {kib / 1024:.0f} MiB ({kib:.0f} KiB read + {kib:.0f} KiB written) reads")
    out(f"#   FETCH_SIZE {fc:.0f} KiB (scale {fs:.4f}) and WRITE_SIZE {wc:.0f} KiB (scale {ws:.4f});")
    out("#   hbm_bytes = 1024 * (FETCH_SIZE / fetch_scale + WRITE_SIZE / write_scale), averaged over the")
    out(f"#   dispatches of {nf} forward passes after the first (all batch 32).")
    out("# algo_bytes = the library's algorithmic bytes per launch for the same kernel (bench eager pass);")
    out("#   a kernel launched on layers of different shapes reports its average over them.")
    out("# ratio = hbm_bytes / algo_bytes (above 1: re-reads or partial-line writes).")
    out("#")
    out(f"# {'kernel (bench name or symbol)':<38} {'dispatches':>10} {'FETCH KiB':>12} {'WRITE KiB':>12} "
        f"{'algo_bytes':>14} {'ratio':>6} {'hbm_bytes':>14}")
    fd, wd = fwd_f["FETCH_SIZE"], fwd_w["WRITE_SIZE"]
    rows = []
    for sym, vals in fd.items():
        f = sum(vals) / len(vals)
        w = sum(wd.get(sym, [0.0])) / max(1, len(wd.get(sym, [])))
        hbm = 1024.0 * (f / fs + w / ws)
        rows.append((hbm * len(vals), sym, len(vals), f, w, hbm))
    for _, sym, n, f, w, hbm in sorted(rows, reverse=True):
        if sym == copy:
            continue
        a = algo.get(sym)
        label = a[0] if a else _label(sym)
        ab = f"{a[2]:14.0f} {hbm / a[2]:6.2f}" if a and a[2] else f"{'-':>14} {'-':>6}"
        out(f"{label:<40} {n:10d} {f:12.1f} {w:12.1f} {ab} {hbm:14.0f}")


def summarize_pmc_mfma(mfma_csv, bench_log):
    """MFMA work, matrix-pipe busy fraction and achieved rate per kernel from
    SQ_INSTS_VALU_MFMA_MOPS_F32, SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE."""
    fwd, _, nf = _pmc_forwards(mfma_csv)
    algo = _bench_kernels(bench_log)
    mops, busy, act = fwd["SQ_INSTS_VALU_MFMA_MOPS_F32"], fwd["SQ_VALU_MFMA_BUSY_CYCLES"], fwd["GRBM_GUI_ACTIVE"]
    sqb = fwd.get("SQ_BUSY_CYCLES", {})
    out(f"# {nf} forward passes after the first; per launch averages.")
    out("# executed_GF = SQ_INSTS_VALU_MFMA_MOPS_F32 * 512 FLOP (MFMA work including tile padding);")
    out("# algo_GF = the library's algorithmic FLOPs per launch (unpadded), from the bench's eager pass;")
    out("# active_us = GRBM_GUI_ACTIVE / 8 XCDs / 2.4 GHz (the counter sums the 8 XCDs; under counter collection);")
    out("# mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 * 256 CUs * 4 SIMDs): the fraction of")
    out("#   SIMD-cycles the matrix pipe was busy while the kernel ran (one v_mfma_f32_32x32x2f32 = 64 busy cycles);")
    out("# achieved = algo_GF / active_us, frac = achieved / 157.3 TFLOP/s (MI355X dense FP32 matrix).")
    out("# sq_busy = SQ_BUSY_CYCLES / GRBM_GUI_ACTIVE, each summed over its hardware instances as the counter")
    out("#   reports it: the sequencers' busy share while the kernel ran, in units of GRBM instances.")
    out("#")
    out(f"# {'kernel (bench name or symbol)':<38} {'launches':>8} {'executed_GF':>11} {'algo_GF':>8} {'pad':>5} "
        f"{'active_us':>9} {'mfma_busy':>9} {'sq_busy':>7} {'TFLOP/s':>8} {'frac':>6}")
    rows = []
    for sym, v in mops.items():
        if sum(v) == 0:
            continue
        n = len(v)
        ex = 512.0 * sum(v) / n / 1e9
        a_us = sum(act[sym]) / n / 8 / 2.4e3
        busy_f = (sum(busy[sym]) / n) / (sum(act[sym]) / n / 8 * 256 * 4)
        sq_f = sum(sqb.get(sym, [0.0])) / max(sum(act[sym]), 1.0)
        rows.append((ex * n, sym, n, ex, a_us, busy_f, sq_f))
    for _, sym, n, ex, a_us, busy_f, sq_f in sorted(rows, reverse=True):
        a = algo.get(sym)
        if a and a[1]:
            ag = a[1] / 1e9
            tf = ag / a_us * 1e3  # GFLOP per microsecond -> TFLOP/s
            out(f"{a[0]:<40} {n:8d} {ex:11.3f} {ag:8.3f} {ex / ag:5.2f} {a_us:9.2f} {busy_f:9.3f} {sq_f:7.2f} "
                f"{tf:8.1f} {tf / PEAK_FP32_MFMA_TFLOPS:6.3f}")
        else:
            out(f"{_label(sym):<40} {n:8d} {ex:11.3f} {'-':>8} {'-':>5} {a_us:9.2f} {busy_f:9.3f} {sq_f:7.2f} "
                f"{'-':>8} {'-':>6}")


def section_gemm1x1():
    """Every implicit-GEMM tile (0-23) and weight-stationary row width (32-35)
    forced on YOLOv8n's batch-32 1x1 convolutions: how far the best candidate
    sits from the MFMA and HBM rooflines, and how close the next ones are."""
    import os
    from simdyolo_amd import synth, CONV_IGEMM
    from simdyolo_amd.device import HipContext
    hip = HipContext(0)
    out(f"# device: {hip.name}")
    out("# 1x1 conv, batch 32, bias + SiLU; each candidate forced with SIMDYOLO_HIP_TILE, HIP-event average of")
    out("#   20 back-to-back calls after 3 warm ones; FLOPs 2*M*IC*OC, bytes 4*M*(IC+OC) (M = 32*H*W);")
    out("#   peaks 157.3 TFLOP/s and 8 TB/s; the six fastest candidates follow the best.")
    B = 32
    for ic, hw, oc in ((64, 80, 64), (96, 80, 64), (192, 80, 64), (64, 80, 128), (80, 80, 80), (128, 40, 128),
                       (192, 40, 128), (384, 20, 256)):
        x = synth.activations((B, ic, hw, hw), 1)
        wt = synth.kaiming((oc, ic, 1, 1), 2)
        b = synth.activations((oc,), 3) * np.float32(0.1)
        hip.begin_frame()
        try:
            conv = hip.conv_create(wt, b, (1, 1), (0, 0, 0, 0), silu=True)
            hip.conv_set_algo(conv, CONV_IGEMM)
            xv = hip.alloc(B, ic, hw, hw)
            hip.upload(x, xv)
            yv = hip.alloc(B, oc, hw, hw)
            res = []
            for t in list(range(24)) + [32, 33, 34, 35]:
                os.environ["SIMDYOLO_HIP_TILE"] = str(t)
                try:
                    for _ in range(3):
                        hip.conv(conv, xv, yv)
                    hip.flush()
                    hip.timer_start()
                    for _ in range(20):
                        hip.conv(conv, xv, yv)
                    res.append((hip.timer_stop() / 20 * 1e3, t))
                except Exception:
                    pass  # a candidate that does not take this shape
            os.environ.pop("SIMDYOLO_HIP_TILE", None)
        finally:
            hip.end_frame()
        res.sort()
        m = B * hw * hw
        fl, by = 2.0 * m * ic * oc, 4.0 * m * (ic + oc)
        us, t = res[0]
        out(f"1x1 {ic:>3}->{oc:<3} @{hw:<3} best t{t:<2} {us:7.1f} us  {fl / us / 1e6:6.1f} TFLOP/s "
            f"({100 * fl / us / 1e6 / 157.3:3.0f}% mfma)  {by / us / 1e3:6.0f} GB/s ({100 * by / us / 1e3 / 8000:3.0f}% hbm)"
            f" | " + ", ".join(f"t{tt} {u:.1f}" for u, tt in res[1:7]))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--section", choices=["layers", "models", "post", "bandwidth", "route", "gemm1x1"])
    ap.add_argument("--trace", nargs=2, metavar=("KERNEL_TRACE_CSV", "BANDWIDTH_LOG"),
                    help="summarise a rocprofv3 kernel trace of a --section bandwidth run")
    ap.add_argument("--forward-trace", nargs=3, metavar=("KERNEL_TRACE_CSV", "STEPS", "BENCH_LOG"),
                    help="summarise a rocprofv3 kernel trace of an eager bench.py run")
    ap.add_argument("--pmc-traffic", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "BENCH_LOG"),
                    help="HBM bytes per kernel from FETCH_SIZE / WRITE_SIZE passes over an eager bench.py run")
    ap.add_argument("--pmc-mfma", nargs=2, metavar=("MFMA_CSV", "BENCH_LOG"),
                    help="MFMA counters per kernel from a PMC pass over an eager bench.py run")
    args = ap.parse_args()
    if args.pmc_traffic:
        summarize_pmc_traffic(*args.pmc_traffic)
        return
    if args.pmc_mfma:
        summarize_pmc_mfma(*args.pmc_mfma)
        return
    if args.trace:
        summarize_trace(*args.trace)
        return
    if args.forward_trace:
        csv_path, steps, log = args.forward_trace
        summarize_forward_trace(csv_path, int(steps), log)
        return
    {"layers": section_layers, "models": section_models, "post": section_post,
     "bandwidth": section_bandwidth, "route": section_route, "gemm1x1": section_gemm1x1}[args.section]()


if __name__ == "__main__":
    main()
