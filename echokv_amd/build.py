"""Build ``echokv_amd/libechokv.so`` (gfx950) from ``echokv_amd/csrc/*.hip`` with hipcc,
and the native host side ``echokv_amd/libechokv_host.so`` from ``echokv_amd/host/*.cpp``
with g++.

    python -m echokv_amd.build            # or __graft_entry__.build()

Each translation unit compiles to an object in ``echokv_amd/_build/`` (in
parallel), then one shared library links them. hipcc cross-compiles, so
this runs without a GPU.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libechokv.so"
ARCH = os.environ.get("ECHOKV_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # IEEE fp32 division / denormals for bit-exact storage numerics.
    "-fno-gpu-flush-denormals-to-zero",
    # No packed fp32 arithmetic in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({' '.join(cmd)}):\n{err}")
    return err


HOST_SRCS = (PKG / "host" / "plan.cpp", PKG / "host" / "step.cpp")
HOST_OUT = PKG / "libechokv_host.so"


def build_host() -> str:
    """The native host planner (CPU code, g++): ``libechokv_host.so``."""
    tmp = HOST_OUT.with_suffix(".so.tmp")
    log = _run([os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
                f"-I{PKG.parent / 'include'}", *map(str, HOST_SRCS), "-o", str(tmp)])
    os.replace(tmp, HOST_OUT)
    return log


def build_library(verbose: bool = False) -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    cmds = [[hipcc(), *FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), 8)) as ex:
        logs = list(ex.map(_run, cmds))
    tmp = OUT.with_suffix(".so.tmp")
    logs.append(_run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]))
    os.replace(tmp, OUT)
    logs.append(build_host())
    if verbose:
        for l in logs:
            if l.strip():
                print(l)
    return OUT


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
