"""HIP GEMV through the m5 C ABI against the CPU oracle (same bytes, same x).

Bar: fp32 GEMV within 1e-5 relative error,
measured normwise as max|y_gpu - y_ref| / max|y_ref|.  With a single output
row the normwise error is the elementwise one, which cancellation can make
arbitrarily large (a 32-term Q8_0 dot of 2.0e-4 out of terms summing to 0.34
in magnitude: condition number ~1700); there the error is taken against the
dot product's absolute sum sum_i |w_i x_i|, the scale of its fp32 forward
error bound.  Range calls must leave rows outside [o0,o1) untouched.
"""
import numpy as np
import pytest

import gen_golden as gg
from helpers import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _check(oracle, code, n_out, n_in, seed, W=None, x=None):
    from dracohip import lib
    if W is None:
        W, x = gg.gemv_inputs(code, n_out, n_in, seed)
    print(f"[gemv] code={code} shape={n_out}x{n_in} seed={seed}", flush=True)
    y = lib.gemv(code, x, W, n_out, n_in)
    yr = oracle.gemv(code, x, W, n_out, n_in)
    if n_out == 1:
        from oracle.oracle import pf, pu8
        row = np.zeros(n_in, np.float32)
        assert oracle.lib.or_dequant_row(code, pu8(W), n_in, pf(row)) == 0
        scale = float(np.abs(row.astype(np.float64) * x.astype(np.float64)).sum())
        e = float(np.max(np.abs(y.astype(np.float64) - yr))) / max(scale, 1e-30)
    else:
        e = rel_err(y, yr)
    assert e <= TOL, (code, n_out, n_in, e)
    return W, x, y


@pytest.mark.parametrize("i", [i for i, c in enumerate(gg.GEMV_CASES) if c[1] in (0, 3, 4, 5, 7, 9)])
def test_gemv_golden_shapes(oracle, i):
    name, code, n_out, n_in = gg.GEMV_CASES[i]
    _check(oracle, code, n_out, n_in, 100 + i)


@pytest.mark.parametrize("code,n_out,n_in", [
    (5, 2048, 2048), (5, 512, 2048), (5, 8192, 2048), (4, 512, 2048), (4, 2048, 8192),
    (5, 4096, 14336), (5, 14336, 4096), (0, 960, 960), (0, 2560, 960), (0, 960, 2560),
    (0, 320, 960), (4, 3000, 2048), (5, 768, 2048), (4, 2048, 768),
    # one row, rows off the 16-row tile, n_in at the 16384 cap, a single super-block / Q8_0 block
    (5, 1, 4096), (5, 17, 16384), (4, 33, 256), (0, 1, 32), (4, 5, 16384),
    # Q5_K (src/m5_kern_scalar.c:91-114): model shapes, one row, ragged tiles, the cap
    (3, 2048, 2048), (3, 14336, 4096), (3, 4096, 14336), (3, 1, 4096), (3, 33, 256), (3, 17, 16384),
])
def test_gemv_model_shapes(oracle, code, n_out, n_in):
    _check(oracle, code, n_out, n_in, 7 + n_out + n_in)


@pytest.mark.parametrize("code", [0, 3, 4, 5])
def test_gemv_range_absolute_rows(oracle, code):
    from dracohip import lib
    n_out, n_in = 300, 512 if code else 512
    W, x = gg.gemv_inputs(code, n_out, n_in, 5)
    y = np.full(n_out, np.float32(-3.0))
    L = lib.load()
    rc = L.m5_gemv_range(code, lib.pf(x), lib.pu8(W), n_out, n_in, lib.pf(y), 37, 250)
    assert rc == 0, lib.last_error()
    yr = oracle.gemv(code, x, W, n_out, n_in)
    assert np.all(y[:37] == np.float32(-3.0)) and np.all(y[250:] == np.float32(-3.0))
    assert rel_err(y[37:250], yr[37:250]) <= TOL


@pytest.mark.parametrize("code", [0, 3, 4, 5])
def test_gemv_onehot_is_exact_column(oracle, code):
    """x = e_i returns column i of the decoded matrix exactly (the reference's
    own block-layout check, ROADMAP.md:568-580)."""
    from dracohip import lib
    n_out, n_in = 64, 1024
    W, _ = gg.gemv_inputs(code, n_out, n_in, 9)
    for col in (0, 31, 255, 256 + 77, 1023):
        x = np.zeros(n_in, np.float32)
        x[col] = 1.0
        y = lib.gemv(code, x, W, n_out, n_in)
        yr = oracle.gemv(code, x, W, n_out, n_in)
        assert np.array_equal(y, yr), (code, col)


def test_unsupported_code_fails_loudly():
    from dracohip import lib
    L = lib.load()
    x = np.zeros(256, np.float32)
    W = np.zeros(4096, np.uint8)
    y = np.zeros(4, np.float32)
    assert L.m5_gemv(2, lib.pf(x), lib.pu8(W), 4, 256, lib.pf(y)) == -1
    assert L.m5_scalar_supported(2) == 0 and L.m5_scalar_supported(5) == 1
    # the reference's scalar kernel serves 0, 3, 4, 5, 7, 9 (src/m5_kern_scalar.c:146-148)
    assert [c for c in range(10) if L.m5_scalar_supported(c)] == [0, 3, 4, 5, 7, 9]


def test_reregistered_address_is_not_stale(oracle):
    """A new buffer at a reused host address is re-uploaded (fingerprint check)."""
    from dracohip import lib
    n_out, n_in = 128, 512
    W1, x = gg.gemv_inputs(5, n_out, n_in, 1)
    W2, _ = gg.gemv_inputs(5, n_out, n_in, 2)
    buf = W1.copy()
    y1 = lib.gemv(5, x, buf, n_out, n_in)
    buf[:] = W2
    y2 = lib.gemv(5, x, buf, n_out, n_in)
    assert rel_err(y2, oracle.gemv(5, x, W2, n_out, n_in)) <= TOL
    assert not np.array_equal(y1, y2)
