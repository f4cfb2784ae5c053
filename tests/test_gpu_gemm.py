"""Prefill GEMM on the GPU: m5_gemm / m5_gemm_auto (src/m5/m5_gemm.c:249-272,
src/m5/m5_gemm_fused.c:231-241) vs the oracle's or_gemm (pinned as "equals
stacked GEMVs").  Bar: max|dY| <= 1e-5 * max|Y_ref| over the whole output.
"""
import numpy as np
import pytest

from helpers import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _case(code, T, n_out, n_in, seed):
    from dracohip import lib
    rng = np.random.default_rng(seed)
    W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
    X = rng.standard_normal((T, n_in)).astype(np.float32)
    X[0, :7] = 0.0           # zeros, a large value and a tiny one in one super-block
    if n_in > 300:
        X[-1, 300] = 80.0
        X[-1, 301] = 1e-30
    return W, X


@pytest.mark.parametrize("code", [5, 4, 0, 3])
@pytest.mark.parametrize("T,n_out,n_in", [(1, 16, 256), (7, 40, 512), (37, 96, 2048), (256, 2048, 2048),
                                          (64, 8192, 2048), (100, 2048, 8192), (9, 48, 768),
                                          # the ragged last prefill chunk on the K-split products, 3 super-blocks
                                          # per row with n_out off the 16-row tile, n_in at the 16384 cap
                                          (191, 512, 2048), (191, 2048, 8192), (33, 1000, 768), (255, 130, 4096),
                                          (32, 16, 16384)])
def test_gemm_vs_oracle(hip, oracle, code, T, n_out, n_in):
    from dracohip import lib
    W, X = _case(code, T, n_out, n_in, T + n_out + code)
    Y = np.zeros((T, n_out), np.float32)
    wbuf = np.zeros(8, np.float32)
    assert hip.m5_gemm(code, lib.pf(X), lib.pu8(W), T, n_out, n_in, lib.pf(Y), lib.pf(wbuf)) == 0, lib.last_error()
    ref = np.zeros_like(Y)
    assert oracle.lib.or_gemm(code, lib.pf(X), lib.pu8(W), T, n_out, n_in, lib.pf(ref)) == 0
    assert rel_err(Y, ref) <= TOL
    Y2 = np.zeros_like(Y)
    assert hip.m5_gemm_auto(code, lib.pf(X), lib.pu8(W), T, n_out, n_in, lib.pf(Y2)) == 0
    assert np.array_equal(Y, Y2)


def test_gemm_equals_stacked_gemv(hip):
    from dracohip import lib
    W, X = _case(5, 24, 512, 2048, 3)
    Y = np.zeros((24, 512), np.float32)
    assert hip.m5_gemm_auto(5, lib.pf(X), lib.pu8(W), 24, 512, 2048, lib.pf(Y)) == 0
    G = np.stack([lib.gemv(5, X[t], W, 512, 2048) for t in range(24)])
    assert rel_err(Y, G) <= TOL


def test_gemm_unsupported_code_returns_minus_one(hip):
    from dracohip import lib
    X = np.zeros((2, 256), np.float32)
    W = np.zeros(4 * 110, np.uint8)
    Y = np.zeros((2, 4), np.float32)
    assert hip.m5_gemm_auto(2, lib.pf(X), lib.pu8(W), 2, 4, 256, lib.pf(Y)) == -1   # IQ3_S: caller falls back


@pytest.mark.parametrize("fname,code", [("q4k", 5), ("q6k", 4), ("q80", 0), ("q5k", 3)])
def test_fused_entries_equal_gemm_auto(hip, fname, code):
    """The per-format entries src/qwen35_prefill.py:76-80 looks up
    (src/m5/m5_gemm_fused.c:211-228) compute what m5_gemm_auto does."""
    from dracohip import lib
    T, n_out, n_in = 40, 96, 512
    W, X = _case(code, T, n_out, n_in, 77 + code)
    Y = np.full((T, n_out), np.nan, np.float32)
    getattr(hip, f"m5_gemm_{fname}")(lib.pf(X), lib.pu8(W), T, n_out, n_in, lib.pf(Y))
    Y2 = np.zeros_like(Y)
    assert hip.m5_gemm_auto(code, lib.pf(X), lib.pu8(W), T, n_out, n_in, lib.pf(Y2)) == 0
    assert np.array_equal(Y, Y2)


@pytest.mark.parametrize("fname", ["iq4xs", "iq3s"])
def test_fused_entries_not_carried_leave_nan(hip, fname):
    from dracohip import lib
    X = np.ones((2, 256), np.float32)
    W = np.zeros(4 * 136, np.uint8)
    Y = np.zeros((2, 4), np.float32)
    getattr(hip, f"m5_gemm_{fname}")(lib.pf(X), lib.pu8(W), 2, 4, 256, lib.pf(Y))
    assert np.isnan(Y).all()

