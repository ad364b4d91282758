"""The CPU performance baseline bench.py reports (``cpu_baseline``): ctypes view of
``libaxis_cpu_step.so`` (oracle/cpu_step.c), a blocked-SGEMM OpenMP port of the 3-block CNN step.

Not the checker -- oracle.py is, and tests/test_cpu_baseline.py holds this port to the oracle --
and never part of the product: only bench.py's cpu_baseline leg and tests/ import it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from oracle import oracle

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libaxis_cpu_step.so")
_lib = None

F32P = ctypes.POINTER(ctypes.c_float)
PARAM_ORDER = ("conv0.weight", "conv0.bias", "conv1.weight", "conv1.bias", "conv2.weight", "conv2.bias",
               "linear.weight", "linear.bias")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            oracle.build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.axcpu_cnn_step.restype = ctypes.c_float
    return _lib


def threads() -> int:
    return int(lib().axcpu_threads())


def kernel_width() -> int:
    """Columns of the GEMM register tile picked for this host (32: AVX-512, 16: AVX2)."""
    return int(lib().axcpu_kernel_width())


def _f(a):
    return a.ctypes.data_as(F32P)


def sgemm(form: str, a, b, m: int, k: int, n: int) -> np.ndarray:
    """nn: a[m][k] b[k][n]; nt: a = g[m][n], b[k][n] -> [m][k]; tn: a[m][k], b = g[m][n] -> [k][n]."""
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    out = np.empty({"nn": m * n, "nt": m * k, "tn": k * n}[form], np.float32)
    I = ctypes.c_int64
    getattr(lib(), f"axcpu_sgemm_{form}")(I(m), I(k), I(n), _f(a), _f(b), _f(out))
    return out


def cnn_step(x, y, params: dict, batch: int, size: int, classes: int, channels, t: int = 1, lr: float = 1e-3,
             moments=None):
    """One fwd + bwd + Adam(lr) step from `params` (not modified); returns (loss, grads, new params).
    `moments` (m, v dicts) carry Adam state across calls and are updated in place."""
    p = {k: np.array(params[k], np.float32, copy=True) for k in PARAM_ORDER}
    if moments is None:
        moments = ({k: np.zeros_like(p[k]) for k in PARAM_ORDER}, {k: np.zeros_like(p[k]) for k in PARAM_ORDER})
    g = {k: np.empty_like(p[k]) for k in PARAM_ORDER}
    arr = lambda d: (F32P * 8)(*[_f(d[k]) for k in PARAM_ORDER])
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    ch = (ctypes.c_int * 4)(*channels)
    loss = lib().axcpu_cnn_step(batch, size, classes, ch, _f(x), _f(y), arr(p), arr(moments[0]), arr(moments[1]),
                                arr(g), t, ctypes.c_float(lr))
    return float(loss), g, p
