"""The CPU performance baseline bench.py reports (oracle/cpu_step.c, blocked-SGEMM OpenMP port of
the config-4 step) against float64 products and against the oracle's whole step.  Both GEMM
kernels (AVX-512 8x32 and AVX2 6x16 register tiles) are covered: the AVX2 one in a subprocess
with AXCPU_KERNEL=avx2."""
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import cpu_baseline as cb

SHAPES = [("nn", (300, 257, 70)), ("nt", (129, 77, 513)), ("tn", (70000, 33, 45)), ("tn", (100, 300, 40)),
          ("nn", (5, 3, 2)), ("nt", (1000, 1152, 64))]


def _check_sgemm():
    rng = np.random.default_rng(0)
    for form, (m, k, n) in SHAPES:
        # nn: a[m][k] b[k][n]; nt: a = g[m][n], b[k][n]; tn: a[m][k], b = g[m][n]
        sa, sb = {"nn": ((m, k), (k, n)), "nt": ((m, n), (k, n)), "tn": ((m, k), (m, n))}[form]
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32)
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        want = a64 @ b64 if form == "nn" else (a64 @ b64.T if form == "nt" else a64.T @ b64)
        got = cb.sgemm(form, a, b, m, k, n).reshape(want.shape)
        err = np.abs(got - want).max() / np.abs(want).max()
        assert err < 1e-5, (form, m, k, n, err)


def _check_step():
    from oracle import oracle
    batch, size, classes, ch = 4, 16, 10, (3, 8, 16, 32)
    x, y, params = oracle.cnn_inputs(batch, size, classes, ch)
    loss_ref, g_ref = oracle.cnn_forward_backward(x, y, params, batch, size, classes, ch)
    p_ref = oracle.AdamOracle(1e-3).step(params, g_ref)
    loss, g, p = cb.cnn_step(x, y, params, batch, size, classes, ch)
    assert abs(loss - loss_ref) < 1e-5 * max(1.0, abs(loss_ref))
    for name in g:
        assert np.abs(g[name] - g_ref[name]).max() < 1e-4 * np.abs(g_ref[name]).max(), name
        assert np.abs(p[name] - p_ref[name]).max() < 1e-5 * max(np.abs(p_ref[name]).max(), 1e-3), name


def test_sgemm_forms_match_float64():
    _check_sgemm()


def test_cnn_step_matches_the_oracle():
    _check_step()


def test_avx2_kernel_path():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r); from tests import test_cpu_baseline as t; "
            "from oracle import cpu_baseline as cb; assert cb.kernel_width() == 16; "
            "t._check_sgemm(); t._check_step()" % root)
    env = dict(os.environ, AXCPU_KERNEL="avx2", OMP_NUM_THREADS="4")
    subprocess.run([sys.executable, "-c", code], check=True, env=env, cwd=root)
