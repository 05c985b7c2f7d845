"""Compile the gfx950 HIP kernels into ``systems_for_llms_amd/lib/libsfl.so``.

Each ``csrc/*.hip`` file is compiled to an object under ``_build/`` in parallel
with ``hipcc --offload-arch=gfx950``, then linked into one shared library that
exports the C ABI declared in ``include/sfl.h``. Run as
``python -m systems_for_llms_amd.build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
REPO = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = REPO / "_build"
LIB_DIR = PACKAGE / "lib"
LIB_PATH = LIB_DIR / "libsfl.so"
ARCH = "gfx950"

# Packed fp32 arithmetic is disabled for every kernel: the compiler must not
# form v_pk_{add,mul,fma}_f32 from scalar or float2 code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-file additions. Kernel-argument preloading (gfx940+) for the decode-step
# kernels: the command processor loads the first 14 argument dwords into SGPRs
# before the waves start, and those kernels put the pointers and sizes their
# first loads need there. The code object keeps a prologue that fetches them
# itself for firmware without preloading.
_PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=14"]
FILE_FLAGS = {
    "decode_linear.hip": _PRELOAD,
    "decode_attention.hip": _PRELOAD,
    "decode_step.hip": _PRELOAD,
}


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the HIP kernels need ROCm's hipcc to build")


def _compile(source: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = jobs or min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
