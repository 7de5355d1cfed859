"""Build ``fastmd_amd/lib/libfastmd_hip.so`` from the HIP sources of this directory for gfx950.

Every ``*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` into an object (in
parallel), then linked into one shared library whose C ABI is ``include/fastmd_hip.h``.
Run as ``python -m fastmd_amd.csrc.build`` or through ``__graft_entry__.build()``; it always
recompiles (it is the build check). No torch import is needed to build.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PACKAGE = os.path.dirname(HERE)
ROOT = os.path.dirname(PACKAGE)
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(PACKAGE, "lib")
LIB_NAME = "libfastmd_hip.so"
ARCH = os.environ.get("FASTMD_OFFLOAD_ARCH", "gfx950")

# Files whose float arithmetic must round every operation (bit-exact neighbour list, ASE NHC).
NO_CONTRACT = {"nl.hip", "nhc.hip"}

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-lambda-capture",
    # Packed FP32 instructions are kept out of the device code (see the build notes).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{HERE}",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the MI355X kernels need the ROCm toolchain")
    return path


def _filter(text: str) -> str:
    # hipcc's host pass does not know the device target feature above: harmless, drop the noise.
    return "\n".join(line for line in text.splitlines() if "is not a recognized feature for this target" not in line)


def sources() -> list[str]:
    return sorted(f for f in os.listdir(HERE) if f.endswith(".hip"))


def build(verbose: bool = False, jobs: int | None = None) -> str:
    hipcc = _hipcc()
    obj_dir = os.path.join(PACKAGE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)

    def compile_one(name: str) -> str:
        src = os.path.join(HERE, name)
        obj = os.path.join(obj_dir, name.replace(".hip", ".o"))
        flags = list(COMMON_FLAGS)
        if name in NO_CONTRACT:
            flags.append("-ffp-contract=off")
        cmd = [hipcc, *flags, "-c", src, "-o", obj]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        out = _filter(proc.stdout + proc.stderr).strip()
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {name}:\n{out}")
        if verbose and out:
            print(out, file=sys.stderr)
        return obj

    names = sources()
    jobs = jobs or min(len(names), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(compile_one, names))
    target = os.path.join(LIB_DIR, LIB_NAME)
    tmp = target + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{_filter(proc.stdout + proc.stderr)}")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(verbose=True))
