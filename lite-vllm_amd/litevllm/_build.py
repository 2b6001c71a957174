"""Build liblitevllm_hip.so from lite-vllm_amd/csrc with hipcc for gfx950.

Usage: ``python -m litevllm._build`` (from lite-vllm_amd/) or
``litevllm._build.build()``.  Every source is recompiled on each call; the
objects go to lite-vllm_amd/_build/ and the shared library next to this file
(git-ignored, but shipped with the source tree to the GPU host).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent              # lite-vllm_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"  # repo-level C ABI headers
OBJ_DIR = ROOT / "_build"
LIB_NAME = "liblitevllm_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = os.environ.get("LITEVLLM_HIP_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fno-gpu-rdc",
    # Keep the compiler from forming packed fp32 ops (v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# Per-source extra flags.  The sampler's arithmetic is defined operation by
# operation (no contraction, IEEE division) so the CPU restatement can match
# it bit for bit.
EXTRA_FLAGS = {
    "sampler.hip": ["-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt"],
    # products and sums rounded separately, as the reference's separate ops do
    "fused_layers.hip": ["-ffp-contract=off"],
    "linear.hip": ["-ffp-contract=off"],
}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the HIP extension cannot be built")
    return exe


def _compile(src: Path, hipcc: str) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {src.name} (exit {proc.returncode}):\n{' '.join(cmd)}\n"
            f"{proc.stdout}\n{proc.stderr}"
        )
    return obj


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = True) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = max(1, min(len(srcs), os.cpu_count() or 1, 8))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fno-gpu-rdc",
           *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[litevllm] built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
