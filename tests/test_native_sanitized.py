"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer, without a GPU.

libkfhip's sources are compiled with the host side instrumented (device code at -O0, never run)
and linked with tests/native/abi_host_check.cpp, which queries every workspace size over the
benchmarked and tested layer shapes and drives the argument validation of every entry point.
Nothing launches a kernel, so this runs on a machine without a GPU; any heap or stack overflow,
use after free, signed overflow or bad shift in the host code (descriptor validation, route and
tile planning, workspace arithmetic) stops the program with the sanitizer's report.
"""

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "kanforge_amd" / "csrc"
HIPCC = Path("/opt/rocm/bin/hipcc")
CLANG = Path("/opt/rocm/lib/llvm/bin/clang++")
ROCM_LIB = Path("/opt/rocm/lib")
# host-side instrumentation only (each sanitizer flag behind -Xarch_host)
HOST_SAN = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer"]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise AssertionError(f"{' '.join(map(str, cmd[:3]))} ... failed:\n{res.stderr[-4000:]}")


@pytest.mark.skipif(not (HIPCC.exists() and CLANG.exists()), reason="the ROCm toolchain is not installed")
def test_c_abi_host_code_under_asan_and_ubsan(tmp_path):
    def compile_source(src: Path) -> Path:
        obj = tmp_path / (src.stem + ".o")
        _run([str(HIPCC), "--offload-arch=gfx950", "-O0", "-g", "-std=c++17", "-fPIC", *HOST_SAN, "-Xclang",
              "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result", f"-I{ROOT / 'include'}", "-c",
              "-o", str(obj), str(src)])
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        objs = list(pool.map(compile_source, sorted(CSRC.glob("*.hip"))))
    driver = tmp_path / "abi_host_check.o"
    san = "-fsanitize=address,undefined"
    _run([str(CLANG), "-O1", "-g", "-std=c++17", san, "-fno-sanitize-recover=undefined", f"-I{ROOT / 'include'}",
          "-c", "-o", str(driver), str(ROOT / "tests" / "native" / "abi_host_check.cpp")])
    exe = tmp_path / "abi_host_check"
    _run([str(CLANG), san, str(driver), *map(str, objs), f"-L{ROCM_LIB}", "-lamdhip64", f"-Wl,-rpath,{ROCM_LIB}",
          "-o", str(exe)])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-6000:]
    assert "Sanitizer" not in out, out[-6000:]
    assert "abi host checks:" in res.stdout and "failed" not in res.stdout, res.stdout
