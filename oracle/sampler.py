"""CPU restatement of the fused sampler (test oracle).

greedy: first index of the fp32 maximum, as _argmax_kernel / torch.argmax
(reference litevllm/layers/sampler.py:60-84, 111-124).  temperature rows:
the fixed-order inverse-CDF definition, implemented in sampler_ref.c and
loaded here through ctypes (built by oracle/build.py).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .build import LIB_PATH, build

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.oracle_exp2_det.restype = ctypes.c_float
        lib.oracle_exp2_det.argtypes = [ctypes.c_float]
        lib.oracle_sample.restype = None
        lib.oracle_sample.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _lib = lib
    return _lib


def greedy(logits: np.ndarray) -> np.ndarray:
    """First index of the row maximum (fp32), int64 [B]."""
    x = np.asarray(logits, dtype=np.float32)
    return np.argmax(x, axis=-1).astype(np.int64)


def exp2_det(t: np.ndarray) -> np.ndarray:
    lib = _load()
    t = np.asarray(t, dtype=np.float32).ravel()
    return np.array([lib.oracle_exp2_det(float(v)) for v in t], dtype=np.float32)


def sample(logits: np.ndarray, temperature: np.ndarray, uniform: np.ndarray) -> np.ndarray:
    """Rows with temperature 0 -> greedy, others -> inverse-CDF draw at uniform."""
    lib = _load()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = x.shape
    t = np.ascontiguousarray(temperature, dtype=np.float32)
    u = np.ascontiguousarray(uniform, dtype=np.float32)
    out = np.empty(B, dtype=np.int64)
    lib.oracle_sample(x.ctypes.data, B, V, t.ctypes.data, u.ctypes.data, out.ctypes.data)
    return out
