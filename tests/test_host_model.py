"""Host-side models of the decode kernels' index math, built with the CPU
compiler under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU):
the persistent kernel's range split and the piece bookkeeping shared with
its reduce kernel (tests/host_model/range_split_check.cpp, which includes
the kernels' own lite-vllm_amd/csrc/lv_split.h), and the oracle's C sampler
(oracle/sampler_ref.c) driven over edge-case rows."""

from __future__ import annotations

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
