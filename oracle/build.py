"""Compile the oracle's C restatement (sampler_ref.c) with gcc.

Output: oracle/_build/liboracle.so (git-ignored; it travels with the tree
to the GPU host).  The reference (lite-vllm 0.1.0) is pure Python, so there
is no reference C/C++ source to compile into oracle/_ref.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "sampler_ref.c"
OUT_DIR = HERE / "_build"
LIB_PATH = OUT_DIR / "liboracle.so"

# No fast-math, no contraction: one IEEE fp32 operation per source operation.
CFLAGS = ["-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
          "-Wall", "-Wextra"]


def build() -> Path:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler for the oracle")
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{proc.stderr}")
    tmp.replace(LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
