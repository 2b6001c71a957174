"""Host-side models of the decode kernels' index math, built with the CPU
compiler under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU):
the persistent kernel's range split and the piece bookkeeping shared with
its reduce kernel (tests/host_model/range_split_check.cpp, which includes
the kernels' own lite-vllm_amd/csrc/lv_split.h), the oracle's C sampler
(oracle/sampler_ref.c) driven over edge-case rows, and the library's host
code (workspace sizes against a model of what the kernels address, argument
checks of every entry point, tests/host_model/capi_host_check.cpp)."""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "lite-vllm_amd" / "csrc"
HERE = Path(__file__).resolve().parent / "host_model"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _cxx():
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    return cxx


def test_range_split_and_piece_bookkeeping(tmp_path):
    exe = tmp_path / "range_split_check"
    subprocess.run([_cxx(), "-std=c++17", "-O1", "-g", *SAN, f"-I{CSRC}",
                    str(HERE / "range_split_check.cpp"), "-o", str(exe)], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "all checks passed" in proc.stdout


def test_oracle_sampler_under_sanitizers(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    exe = tmp_path / "sampler_ref_check"
    subprocess.run([gcc, "-std=c11", "-O1", "-g", "-ffp-contract=off", *SAN,
                    str(HERE / "sampler_ref_check.c"), str(ROOT / "oracle" / "sampler_ref.c"),
                    "-o", str(exe), "-lm"], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "all passed" in proc.stdout


def test_library_host_code_under_sanitizers(tmp_path):
    """The library's sources compiled host-only (relocatable device code,
    none of it built, so nothing can launch) with ASan/UBSan on the host
    side, linked into a driver that checks every workspace-size function
    against a model of what the kernels address and every entry point's
    refusal of bad arguments."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("no hipcc")
    host_san = [x for f in SAN for x in ("-Xarch_host", f)]
    flags = ["--offload-host-only", "-fgpu-rdc", "-O1", "-g", "-fPIC", "-std=c++17",
             f"-I{ROOT / 'include'}", f"-I{CSRC}", *host_san]

    def compile_one(src: Path) -> Path:
        obj = tmp_path / (src.stem + ".o")
        subprocess.run([hipcc, *flags, "-c", str(src), "-o", str(obj)], check=True,
                       capture_output=True)
        return obj
    srcs = sorted(CSRC.glob("*.hip")) + [HERE / "capi_host_check.cpp"]
    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(compile_one, srcs))
    exe = tmp_path / "capi_host_check"
    subprocess.run([hipcc, "-fgpu-rdc", "--offload-arch=gfx950", *host_san, *map(str, objs),
                    "-o", str(exe)], check=True, capture_output=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "all passed" in proc.stdout
