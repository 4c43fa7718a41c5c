"""The host-thread copy pool behind the pinned staging (host_copy.h): built
with g++ on the host (it has no device code) and run over sizes that split
unevenly between the threads, including those whose floor share per thread
is a page multiple with a remainder (those once left their last bytes
uncopied)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "simdyolo_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_copy_pool_covers_every_byte(tmp_path):
    exe = str(tmp_path / "host_copy_check")
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", CSRC, os.path.join(HERE, "host_copy_check.cpp"), "-o", exe,
                    "-lpthread"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
