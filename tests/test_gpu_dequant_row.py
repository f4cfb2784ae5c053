"""m5_dequant_row (src/m5/m5_gemm.c:55-235) on the GPU through the C ABI.

Rows of Q8_0 / Q4_K / Q5_K / Q6_K / F16 matrices are decoded on the device twice:
from the row's own bytes (matrix not registered) and from the resident copy
of a registered matrix (the embedding decoder of the device decode loop).
Both equal the oracle's or_dequant_row bit for bit; the oracle's decoder is
pinned by the golden one-hot GEMV columns and the numpy decoders
(tests/test_oracle_pins.py).  Codes the device does not carry return -1 as
the reference's unknown codes do.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [(0, 8, 2048), (5, 8, 2048), (4, 8, 2048), (7, 4, 512), (5, 3, 14336), (4, 2, 4096), (0, 5, 960),
         (3, 8, 2048), (3, 3, 14336)]


def _matrix(code, n_out, n_in, seed):
    from dracohip import lib
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n_out, n_in)) * 0.5).astype(np.float32)
    if code == 7:
        return x.astype(np.float16).view(np.uint8).reshape(-1).copy()
    return lib.quantize(code, x)


@pytest.mark.parametrize("code,n_out,n_in", CASES)
def test_dequant_row_matches_oracle(hip, oracle, code, n_out, n_in):
    from dracohip import lib
    W = _matrix(code, n_out, n_in, 1000 + code + n_in)
    rb = lib.row_bytes(code, n_in)
    ref = oracle.dequant(code, W, n_out, n_in)
    hip.draco_forget(W.ctypes.data)
    for resident in (False, True):
        if resident:  # a GEMV registers the matrix
            lib.gemv(code, np.ones(n_in, np.float32), W, n_out, n_in)
        print(f"[dequant_row] code {code} {n_out}x{n_in} resident {resident}", flush=True)
        for r in range(n_out):
            out = np.full(n_in, np.nan, np.float32)
            rc = hip.m5_dequant_row(code, lib.pu8(W[r * rb:(r + 1) * rb]), n_in, lib.pf(out))
            assert rc == 0, lib.last_error()
            np.testing.assert_array_equal(out, ref[r])
    hip.draco_forget(W.ctypes.data)


def test_dequant_row_codes_not_served(hip):
    from dracohip import lib
    row = np.zeros(256, np.uint8)
    out = np.zeros(256, np.float32)
    for code in (1, 2, 6, 9, 13, 99):
        assert hip.m5_dequant_row(code, lib.pu8(row), 256, lib.pf(out)) == -1
