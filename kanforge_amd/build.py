"""Build recipe of libkfhip.so (the HIP kernels + C ABI) for gfx950.

Run ``python -m kanforge_amd.build`` (or call ``build()``); the library is
written next to this file so it ships with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB = HERE / "libkfhip.so"
ARCH = os.environ.get("KF_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops stay off: plain scalar float code only
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libkfhip.so)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-6000:]}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into libkfhip.so (always recompiles): one object per source,
    compiled in parallel, then linked."""
    objdir = Path(tempfile.mkdtemp(prefix="kfhip-build-"))
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    try:
        srcs = sources()
        objs = [objdir / (src.stem + ".o") for src in srcs]
        cc = hipcc()
        jobs = [[cc, *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", "-o", str(obj), str(src)] for src, obj in zip(srcs, objs)]
        with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
            for fut in [pool.submit(_run, job, verbose) for job in jobs]:
                fut.result()
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
        os.replace(tmp, LIB)
    finally:
        tmp.unlink(missing_ok=True)
        shutil.rmtree(objdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
