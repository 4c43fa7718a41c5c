"""YOLOv8n 640x640 FP32 forward throughput on one MI355X.

One step = one whole-network forward (PredictRaw: stem -> backbone -> neck ->
Detect -> joined DFL decode into [B, 84, 8400]) over one batch of synthetic
images already resident in HBM, replayed as one hipGraph.  Prints one JSON
line.  Also reports, for the dominant kernel, its roofline fraction from
per-launch HIP events on the library's stream (an eager pass with per-kernel
event timing), and a CPU baseline: a C restatement of the reference's FP32
CPU path (oracle/cpu_fast.c) timed on this host's cores on a bounded sample.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 32] [--size 640]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense FP32 matrix
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
RIDGE = PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # FLOP/B
METRIC = "images/s YOLOv8n 640\u00b2 FP32 bs1/bs32; % FP32-MFMA peak & % HBM peak per kernel"
# HBM bytes per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes,
# scaled by the plain-copy calibration (see the file's header).
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_yolov8n_640_b32.txt")

# Library profile names -> the kernel symbols rocprofv3 reports.
SYMBOLS = {"wino_input": "sy::wino_in_kernel<4>", "wino_input_blk": "sy::wino_in_blk_kernel",
           "wino_output": "sy::wino_out_kernel", "wino_gemm_out": "sy::wino_go_kernel<4>",
           "wino_gemm_out_w8": "sy::wino_go_kernel<8>",
           "wino_fused": "sy::wino_fx_kernel<9, 1>", "wino_fused_ws": "sy::wino_fw_kernel", "wino_fused_g2": "sy::wino_fx_kernel<9, 2>", "direct_conv": "sy::direct_kernel",
           "stem_conv": "sy::stem_kernel<16>",
           "conv3x3_c16_oc16_s1": "sy::conv_c16_kernel<16, 1, 8>",
           "conv3x3_c16_oc32_s1": "sy::conv_c16_kernel<32, 1, 8>",
           "conv3x3_c16_oc16_s2": "sy::conv_c16_kernel<16, 2, 4>",
           "conv3x3_c16_oc32_s2": "sy::conv_c16_kernel<32, 2, 4>",
           "depthwise_conv": "sy::depthwise_kernel", "depthwise_reg_s1": "sy::dw3_kernel<1>",
           "depthwise_reg_s2": "sy::dw3_kernel<2>", "depthwise_tile20": "sy::dw3_tile_kernel<20>",
           "depthwise_tile32": "sy::dw3_tile_kernel<32>", "depthwise_col4": "sy::dw3_col_kernel<4>",
           "depthwise_col8": "sy::dw3_col_kernel<8>", "sppf_pool": "sy::sppf_plane_kernel<3>",
           "sppf_rows20": "sy::sppf_rows20_kernel<3>",
           "detect_decode": "sy::decode_kernel", "copy": "sy::binary4_kernel<false>",
           "resize_nearest": "sy::resize2x4_kernel",
           "topk_class_pass": "sy::topk_class_pass_kernel", "topk_select": "sy::topk_select_kernel<*>", "topk_extras": "sy::topk_extras_kernel",
           "nms_cand_scan": "sy::cand_scan_kernel",
           "nms_cand_sort": "sy::cand_sort_kernel"}


def symbol(name):
    """rocprofv3 symbol of a library profile name: igemm_m<mode>_<bm>x<bn>_<wm><wn>_k<bk>[_p<pf>] or
    wino_gemm_<bm>x<bn>_<wm><wn>_k<bk>[_p<pf>] (pf: K tiles loaded ahead, 1 when absent),
    pw_gemm_n<32*NW> / wino_pw_n<32*NW> (the K-chunk template argument depends on the layer,
    written *), or a fixed kernel."""
    m = re.fullmatch(r"(igemm_m(\d)|wino_gemm)_(\d+)x(\d+)_(\d)(\d)_k(\d+)(?:_p(\d))?", name)
    if m:
        kind, mode = (0, m.group(2)) if m.group(2) is not None else (1, "2")
        pf = m.group(8) or "1"
        return (f"sy::igemm_kernel<{kind}, {mode}, {m.group(3)}, {m.group(4)}, {m.group(5)}, {m.group(6)}, "
                f"{m.group(7)}, {pf}>")
    m = re.fullmatch(r"(pw_gemm|wino_pw)_n(\d+)", name)
    if m:
        return f"sy::pw_kernel<{int(m.group(2)) // 32}, *>"
    return SYMBOLS.get(name)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_table(prof, steps):
    rows = []
    total = sum(v[1] for v in prof.values())
    for name, (count, ms, flops, nbytes) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        # Roofline bound from arithmetic intensity against the ridge point.
        if flops > 0 and flops / max(nbytes, 1) > RIDGE:
            bound, achieved, peak, unit = "mfma", flops / (ms * 1e-3) / 1e12, PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
        else:
            bound, achieved, peak, unit = "hbm", nbytes / (ms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
        rows.append({"kernel": name, "launches_per_step": count / steps, "ms_per_step": ms / steps,
                     "share": ms / total if total else 0.0, "bound": bound, "achieved": achieved, "unit": unit,
                     "frac": achieved / peak, "avg_launch_us": 1e3 * ms / count,
                     "flops_per_launch": flops / count, "bytes_per_launch": nbytes / count})
    return rows


def load_traffic():
    """{profile name: HBM bytes per launch} from the committed PMC summary."""
    out = {}
    if not os.path.exists(TRAFFIC_FILE):
        return out
    with open(TRAFFIC_FILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 2 and not line.startswith("#") and symbol(parts[0]):
                try:
                    out[parts[0]] = float(parts[-1])
                except ValueError:
                    pass
    return out


def copy_probe(ctx, mib, reps=3):
    """A plain dense copy of `mib` MiB, the known-size kernel that calibrates
    the FETCH_SIZE / WRITE_SIZE counters."""
    from simdyolo_amd import Tensor
    nbytes = mib << 20
    src, dst = ctx.malloc(nbytes), ctx.malloc(nbytes)
    h = mib * 4  # 256 channels x 256 pixels per row: 256 KiB per row
    x = Tensor(src, 1, 256, h, 256, 256, 0)
    y = Tensor(dst, 1, 256, h, 256, 256, 0)
    for _ in range(reps):
        ctx.copy(x, y)
    ctx.flush()
    ctx.free(src)
    ctx.free(dst)
    log(f"copy probe: {reps} copies of {mib} MiB")


def step_times(ctx, step, n):
    """Per-step event times (each step bracketed and waited for): median and
    95th percentile in ms."""
    t = []
    for _ in range(n):
        ctx.timer_start()
        step()
        t.append(ctx.timer_stop())
    return {"median_ms": float(np.median(t)), "p95_ms": float(np.percentile(t, 95))}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(params, size, batch, budget_s):
    """The reference's FP32 CPU algorithms (oracle/cpu_fast.c: Winograd
    F(4,3)/F(2,3) routing, packed AVX2/FMA GEMM, OpenMP over this host's
    cores) timed on a bounded sample: batch 1 frames for about half the
    budget, then batch-`batch` forwards for the rest (at least two)."""
    import oracle
    from simdyolo_amd import synth
    fast = oracle.FastYolov8(params)
    cores = fast.threads()
    try:
        x1 = synth.images(1, size, size, seed=synth.SEED + 7)
        fast.forward(x1)  # plans the weights
        t1 = []
        t_end = time.perf_counter() + budget_s / 2
        while time.perf_counter() < t_end or len(t1) < 10:
            t0 = time.perf_counter()
            fast.forward(x1)
            t1.append(time.perf_counter() - t0)
        xb = synth.images(batch, size, size, seed=synth.SEED + 8)
        fast.forward(xb)
        tb = []
        t_end = time.perf_counter() + budget_s / 2
        while time.perf_counter() < t_end or len(tb) < 2:
            t0 = time.perf_counter()
            fast.forward(xb)
            tb.append(time.perf_counter() - t0)
    finally:
        fast.close()
    med1, medb = float(np.median(t1)), float(np.median(tb))
    return {"value": batch / medb, "unit": "images/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "batch1": {"images_per_s": 1.0 / med1, "median_ms": med1 * 1e3,
                       "p95_ms": float(np.percentile(t1, 95)) * 1e3, "frames": len(t1)},
            "sample": f"YOLOv8n {size}x{size}: {len(tb)} forwards of batch {batch} (median "
                      f"{medb * 1e3:.0f} ms, {batch / medb:.1f} images/s) and {len(t1)} batch-1 frames (median "
                      f"{med1 * 1e3:.1f} ms); oracle/cpu_fast.c, a C restatement of the reference's FP32 CPU "
                      f"path (Winograd F(4,3)/F(2,3) per Compute.cs:185-188, packed AVX2/FMA GEMM, FastExp SiLU, "
                      f"AVX-512 off), OpenMP over {cores} threads of {cpu_model()}; not the reference's .NET "
                      f"binary"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--size", type=int, default=640)
    ap.add_argument("--scale", default="n")
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-bs1", action="store_true")
    ap.add_argument("--windows", type=int, default=3, help="timed windows of --steps steps each (median)")
    ap.add_argument("--no-pcie", action="store_true", help="skip the host-buffer PredictRaw rate")
    ap.add_argument("--eager", action="store_true",
                    help="launch the forward kernel by kernel instead of replaying its hipGraph")
    ap.add_argument("--tune-table", default=None,
                    help="autotuner decision table: loaded when the file exists, written after the run "
                         "(reproduces one run's kernel choices in profiler runs)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run a plain copy of this many MiB (PMC calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library runs the whole forward on a single MI355X "
              "(the path shards by batch with no collective; multi-GPU runs are not part of it). "
              "Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from simdyolo_amd import synth
    from simdyolo_amd.detector import YoloDetector

    cfg = synth.config(args.scale)
    params = synth.params(cfg)
    B, S = args.batch, args.size
    det = YoloDetector(cfg, params)
    ctx = det.ctx
    if args.eager:
        det.set_graph(False)
    log(f"device: {ctx.name}")
    if args.tune_table and os.path.exists(args.tune_table):
        ctx.tune_load(args.tune_table)
        log(f"tuning table {args.tune_table} loaded")
    x = synth.images(B, S, S)
    if not args.no_pcie:
        # The host-buffer path creates its copy streams on its first call, and
        # HIP maps a process's streams onto four hardware queues in creation
        # order: created after the resident graph's branch stream, the download
        # stream would share the forward stream's queue (8.8 against 6.8 ms per
        # B=32 call).  One batch-1 call first keeps them apart, as a host that
        # uses both paths would do.
        det.predict_raw(np.ascontiguousarray(x[:1]))
    inp, out = det.buffers(B, S, S)
    ctx.h2d(inp, x)
    ctx.flush()

    # Warmup (captures the graph on the first run).
    for _ in range(args.warmup):
        det.run(B, S, S)
    ctx.flush()
    log(f"warmup {args.warmup} done")

    # Timed windows (the reference's method: several windows, median of
    # them): each window is K steps between two events on the library stream.
    windows = []
    t0 = time.perf_counter()
    for _ in range(args.windows):
        ctx.flush()
        ctx.timer_start()
        for _ in range(args.steps):
            det.run(B, S, S)
        windows.append(ctx.timer_stop() / args.steps)
    ctx.flush()
    wall = time.perf_counter() - t0
    ms_per_step = float(np.median(windows))
    value = B / (ms_per_step * 1e-3)
    log(f"timed {args.windows} x {args.steps} steps: {', '.join(f'{w:.3f}' for w in windows)} ms/step (events), "
        f"wall {wall * 1e3 / (args.steps * args.windows):.3f} ms/step")
    per_step = step_times(ctx, lambda: det.run(B, S, S), args.steps)

    level = det.branch_level(B, S, S)
    head = ctx.d2h(out, det.output_shape(B, S, S))
    finite = bool(np.isfinite(head).all())

    # Batch-1 latency (graph replay), the reference's published configuration.
    bs1 = None
    if not args.no_bs1:
        i1, _ = det.buffers(1, S, S)
        ctx.h2d(i1, x[:1])
        for _ in range(10):
            det.run(1, S, S)
        ctx.flush()
        n1 = 100
        w1 = []
        for _ in range(args.windows):
            ctx.timer_start()
            for _ in range(n1):
                det.run(1, S, S)
            w1.append(ctx.timer_stop() / n1)
        ms1 = float(np.median(w1))
        st1 = step_times(ctx, lambda: det.run(1, S, S), n1)
        bs1 = {"ms_per_image": ms1, "images_per_s": 1e3 / ms1, "windows_ms": w1, "steps_per_window": n1,
               "per_step_median_ms": st1["median_ms"], "per_step_p95_ms": st1["p95_ms"],
               "branch_level": det.branch_level(1, S, S)}
        log(f"batch 1: {ms1:.3f} ms/image (median of {args.windows} windows), per-step p95 {st1['p95_ms']:.3f} ms")

    # PCIe-inclusive rate: PredictRaw with host buffers (upload of the NCHW
    # batch from pageable memory, forward, download of the head), which is
    # what the reference's device timings include.  Reported beside `value`.
    pcie = None
    if not args.no_pcie:
        pcie = {}
        for nb in (B, 1):
            xb = np.ascontiguousarray(x[:nb])
            # Warm calls: the chunk plans' first uses tune, plan and capture.
            for _ in range(3 if nb > 1 else 5):
                det.predict_raw(xb)
            reps = 10 if nb > 1 else 50
            t = []
            for _ in range(reps):
                t1 = time.perf_counter()
                det.predict_raw(xb)
                t.append(time.perf_counter() - t1)
            med = float(np.median(t))
            pcie[f"batch{nb}"] = {"ms_per_call": med * 1e3, "images_per_s": nb / med, "calls": reps,
                                  "p95_ms": float(np.percentile(t, 95)) * 1e3}
            log(f"PredictRaw from host memory, batch {nb}: {med * 1e3:.3f} ms/call ({nb / med:.0f} images/s)")

    # Per-kernel event timing (eager launches on the library stream).
    det.set_graph(False)
    ctx.profile_enable(True)
    for _ in range(args.profile_steps):
        det.run(B, S, S)
    ctx.flush()
    prof = ctx.profile_read()
    ctx.profile_enable(False)
    det.set_graph(not args.eager)
    rows = kernel_table(prof, args.profile_steps)
    eager_ms = sum(r["ms_per_step"] for r in rows)
    dom = rows[0]
    traffic = load_traffic().get(dom["kernel"])
    roofline = {"bound": dom["bound"], "achieved": dom["achieved"],
                "peak": PEAK_FP32_MFMA_TFLOPS if dom["bound"] == "mfma" else PEAK_HBM_GBS,
                "unit": dom["unit"], "frac": dom["frac"], "traffic": traffic, "kernel": dom["kernel"],
                "symbol": symbol(dom["kernel"]), "avg_launch_us": dom["avg_launch_us"],
                "algorithmic_per_launch": dom["flops_per_launch"] if dom["bound"] == "mfma"
                else dom["bytes_per_launch"],
                "algorithmic_bytes_per_launch": dom["bytes_per_launch"]}
    if dom["kernel"].startswith("wino_fused"):
        roofline["counts"] = ("FLOPs of the 36 transformed-plane GEMMs, 2*36*tiles*IC*OC (a quarter of the direct "
                              "convolution's); the input and output transforms the kernel also runs are FP32 VALU "
                              "work on the same SIMDs and are not counted")
    for r in rows[:12]:
        log(f"  {r['kernel']:<22} {r['ms_per_step']:8.3f} ms/step {100 * r['share']:5.1f}%  "
            f"{r['achieved']:8.1f} {r['unit']:<8} ({100 * r['frac']:5.1f}% of {r['bound']} peak)")
    if args.tune_table and not os.path.exists(args.tune_table):
        ctx.tune_save(args.tune_table)
        log(f"tuning table written to {args.tune_table}")
    if args.copy_probe_mib > 0:
        copy_probe(ctx, args.copy_probe_mib)
    det.close()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(params, S, B, args.cpu_budget)
        log(f"cpu baseline: {cpu['value']:.2f} images/s at batch {B}, {cpu['batch1']['images_per_s']:.2f} at "
            f"batch 1, {cpu['cores']} threads ({cpu['cpu']})")

    line = {
        "metric": METRIC,
        "value": value, "unit": "images/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_per_step, "windows": args.windows, "windows_ms_per_step": windows,
        "per_step_median_ms": per_step["median_ms"], "per_step_p95_ms": per_step["p95_ms"],
        "timing": f"median of {args.windows} windows of {args.steps} graph replays, HIP events on the library "
                  f"stream; inputs resident in HBM",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (seeded random-init YOLOv8 weights, uniform u8 pixels / 255)",
        "config": {"workload": f"YOLOv8{args.scale} detect forward {S}x{S}, batch {B}, "
                               f"{'eager launches' if args.eager else 'hipGraph replay'}",
                   "batch": B, "size": S, "scale": args.scale, "parallelism": "single GPU",
                   "branch_level": level},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "batch1": bs1,
        "pcie_inclusive": pcie,
        "eager_profile_ms_per_step": eager_ms,
        "kernels": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()} for r in rows[:16]],
        "head_finite": finite,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
