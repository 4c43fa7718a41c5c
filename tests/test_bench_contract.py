"""bench.py's contract pieces that run without a GPU: the one-GPU refusal,
the roofline arithmetic of its kernel table, and the link from the roofline
kernel to the committed rocprofv3 summaries under profiles/."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr or "single MI355X" in r.stderr
    assert r.stdout.strip() == ""


def test_kernel_table_roofline_arithmetic():
    # name: (launches, total ms, total flops, total bytes) over 2 steps.
    prof = {"gemm": (4, 2.0, 4 * 1.0e9, 4 * 1.0e7),      # AI 100 > ridge: MFMA-bound
            "copy": (2, 1.0, 0.0, 2 * 4.0e8)}             # no flops: HBM-bound
    rows = {r["kernel"]: r for r in bench.kernel_table(prof, steps=2)}
    g, c = rows["gemm"], rows["copy"]
    assert g["bound"] == "mfma" and c["bound"] == "hbm"
    assert g["launches_per_step"] == 2 and g["ms_per_step"] == 1.0 and g["avg_launch_us"] == 500.0
    assert g["achieved"] == pytest.approx(4e9 / 2e-3 / 1e12)          # TFLOP/s
    assert g["frac"] == pytest.approx(g["achieved"] / bench.PEAK_FP32_MFMA_TFLOPS)
    assert c["achieved"] == pytest.approx(8e8 / 1e-3 / 1e9)           # GB/s
    assert c["frac"] == pytest.approx(c["achieved"] / bench.PEAK_HBM_GBS)
    assert g["share"] == pytest.approx(2.0 / 3.0)
    assert bench.RIDGE == pytest.approx(157.3e12 / 8e12)


def test_profile_names_map_to_kernel_symbols():
    assert bench.symbol("igemm_m2_64x64_22_k16") == "sy::igemm_kernel<0, 2, 64, 64, 2, 2, 16, 1>"
    assert bench.symbol("igemm_m1_64x64_22_k32_p2") == "sy::igemm_kernel<0, 1, 64, 64, 2, 2, 32, 2>"
    assert bench.symbol("wino_gemm_128x32_41_k16") == "sy::igemm_kernel<1, 2, 128, 32, 4, 1, 16, 1>"
    assert bench.symbol("pw_gemm_n96") == "sy::pw_kernel<3, *>"
    assert bench.symbol("wino_gemm_out") == "sy::wino_go_kernel<4>"
    assert bench.symbol("wino_gemm_out_w8") == "sy::wino_go_kernel<8>"
    assert bench.symbol("not_a_kernel") is None


def test_committed_profiles_cover_the_roofline_kernel():
    """The dominant kernel's HBM traffic comes from the committed PMC summary,
    and the kernel-trace summary names its symbol."""
    traffic = bench.load_traffic()
    assert traffic.get("wino_gemm_out", 0) > 0
    with open(os.path.join(ROOT, "profiles", "kernel_trace_yolov8n_640_b32.txt")) as f:
        trace = f.read()
    assert bench.symbol("wino_gemm_out") in trace
    assert "rocprofv3 --kernel-trace --stats" in trace
