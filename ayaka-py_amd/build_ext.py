"""Build ``libayaka_fp8.so`` (the gfx950 HIP kernels behind the C ABI in
``include/ayaka_fp8.h``) in-tree, next to the Python package that loads it.

Usage: ``python ayaka-py_amd/build_ext.py`` (or ``build()`` from Python). Each
``csrc/*.hip`` file is compiled to an object with ``hipcc --offload-arch=gfx950``
in parallel, then linked into one shared library. hipcc cross-compiles, so this
runs on a host without a GPU.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
OUT_DIR = ROOT / "ayaka" / "kernel" / "hip"
LIB_NAME = "libayaka_fp8.so"
BUILD_DIR = ROOT / "_build"

ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU ops, which
# have produced silently wrong results on this hardware pool.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and pathlib.Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


# Per-file flags. gemm_block.hip keeps its MFMA accumulators in VGPRs: it rescales them
# with VALU multiplies every 128-K block, which the AGPR form would turn into AGPR
# read / multiply / write triples.
FILE_FLAGS: dict[str, list[str]] = {
    "gemm_block.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(hipcc: str, src: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    return obj


def _check_resolves(lib: pathlib.Path) -> None:
    """Load the linked library with every symbol bound now. A kernel template whose host
    side fails to instantiate leaves its launch stub undefined without a compile error;
    the library then links but cannot be loaded."""
    import ctypes

    try:
        ctypes.CDLL(str(lib), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    except OSError as err:
        raise RuntimeError(f"{lib.name} does not load: {err}") from err


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libayaka_fp8.so``."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda s: _compile(hipcc, s), sources))
    target = OUT_DIR / LIB_NAME
    tmp = target.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    _check_resolves(tmp)
    os.replace(tmp, target)
    if verbose:
        print(f"built {target}")
    return target


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
