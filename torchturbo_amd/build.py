"""Build the HIP kernel library ``libtorchturbo_moe.so`` for gfx950.

Every ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` to an
object, then linked into one shared library next to this file
(``torchturbo_amd/_lib/``). Runs on a machine without a GPU (hipcc
cross-compiles). Usage: ``python -m torchturbo_amd.build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libtorchturbo_moe.so"
ARCH = os.environ.get("TT_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Scalar float code stays unfused so products and sums round where the
    # reference rounds them.
    "-ffp-contract=off",
    # Keep the compiler from forming packed-fp32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-source flags. gmm.hip: no cross-lane merging of atomics (the merge
# waits for the atomic's return right away, stalling the GEMM pipeline on its
# in-flight loads; the queue atomics there are issued by one lane anyway).
SOURCE_FLAGS = {
    "gmm.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP kernels)")


def library_path() -> Path:
    return OUT_DIR / LIB_NAME


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every kernel source and link the shared library; return its path."""
    cc = hipcc()
    build_dir = OUT_DIR / "obj"
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = build_dir / (src.stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-I", str(PKG.parent / "include"),
               "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
        return obj

    workers = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, srcs))
    lib = library_path()
    tmp = lib.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
