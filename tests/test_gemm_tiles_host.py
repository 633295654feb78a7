"""CPU check of the large-tile GEMM's tile order and buffer windows.

Compiles ``tests/host/gemm_tiles_check.cpp`` against ``csrc/gemm_tiles.h`` (the
same ``__host__ __device__`` functions the kernel uses) with g++ and runs it: the
tile order must be a bijection, and every wavefront's buffer window must make valid
rows readable and rows past M / N unreadable (zero), with its base inside the
allocation.
"""

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_gemm_tile_windows(tmp_path):
    exe = tmp_path / "gemm_tiles_check"
    subprocess.run(["g++", "-O1", "-std=c++17", f"-I{ROOT / 'ayaka-py_amd' / 'csrc'}",
                    str(ROOT / "tests" / "host" / "gemm_tiles_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
