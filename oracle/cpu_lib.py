"""ctypes wrapper of oracle/libgdn2_cpu.so (C restatement of the gdn2 recurrence).

TEST INFRASTRUCTURE ONLY: imported by tests/ and by bench.py's cpu_baseline leg.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libgdn2_cpu.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        fp = ctypes.POINTER(ctypes.c_float)
        lib.gdn2_cpu_recurrent_fwd_f32.restype = ctypes.c_int
        lib.gdn2_cpu_recurrent_fwd_f32.argtypes = [fp] * 9 + [ctypes.c_int] * 5 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_int]
        lib.gdn2_cpu_max_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def recurrent_fwd_f32(q, k, v, g, b, w, h0=None, scale=None, l2norm=True, nthreads=0):
    """float32 recurrence over [B,T,H,*] arrays; returns (o, final_state)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    arrs = [np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, g, b, w)]
    h0a = None if h0 is None else np.ascontiguousarray(h0, dtype=np.float32)
    o = np.empty((B, T, H, V), dtype=np.float32)
    ht = np.empty((B, H, K, V), dtype=np.float32)
    if scale is None:
        scale = K ** -0.5
    rc = load().gdn2_cpu_recurrent_fwd_f32(*[_p(a) for a in arrs], _p(h0a), _p(o), _p(ht),
                                           B, T, H, K, V, float(scale), int(l2norm), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"gdn2_cpu_recurrent_fwd_f32 failed ({rc})")
    return o, ht
