"""Q8_K activations and the Q4_K / Q6_K x Q8_K GEMV on the GPU vs the oracle.

Bars: Q8_K bytes and integer super-block sums bit-exact; fp32 outputs within
1e-5 of max|y| (normwise over the output vector), through the C ABI.
"""
import numpy as np
import pytest

from helpers import rel_err

pytestmark = pytest.mark.gpu
Q8K = 292
TOL = 1e-5


def _x(n, nvec, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((nvec, n)).astype(np.float32) * np.float32(scale)
    # edge cases the quantizer must reproduce: an all-zero block, ties in |x|, exact halves
    if n >= 512:
        x[0, 256:512] = 0.0
    x[0, 3], x[0, 9] = 4.0, -4.0
    return x


@pytest.mark.parametrize("n,nvec", [(256, 1), (4096, 1), (14336, 1), (2048, 8), (768, 4)])
def test_q8k_quantize_bytes_bit_exact(hip, oracle, n, nvec):
    from dracohip import lib
    x = _x(n, nvec, n + nvec)
    got = np.zeros(nvec * (n // 256) * Q8K, np.uint8)
    lib.check(hip.draco_q8k_quantize(lib.pf(x), n, nvec, lib.pu8(got)), "draco_q8k_quantize")
    want = np.concatenate([oracle.quantize_q8k(x[v]) for v in range(nvec)])
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]


@pytest.mark.parametrize("code", [4, 5])
@pytest.mark.parametrize("n_out,n_in", [(16, 256), (37, 768), (300, 2048), (1000, 4096)])
def test_q8k_isums_bit_exact(hip, oracle, code, n_out, n_in):
    import ctypes as ct
    from dracohip import lib
    rng = np.random.default_rng(n_out + code)
    W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
    xq = oracle.quantize_q8k(_x(n_in, 1, 7)[0])
    nb = n_in // 256
    isc = np.zeros(n_out * nb, np.int32)
    imn = np.zeros(n_out * nb, np.int32)
    lib.check(hip.draco_q8k_isums(code, lib.pu8(xq), lib.pu8(W), n_out, n_in, lib.pi32(isc), lib.pi32(imn)),
              "draco_q8k_isums")
    bb = 144 if code == 5 else 210
    rs = nb * bb
    wi, wm = np.zeros_like(isc), np.zeros_like(imn)
    a, m = ct.c_int32(), ct.c_int32()
    for r in range(n_out):
        for b in range(nb):
            oracle.lib.or_q8k_block_isums(code, lib.pu8(W[r * rs + b * bb:r * rs + (b + 1) * bb]),
                                          lib.pu8(xq[b * Q8K:(b + 1) * Q8K]), ct.byref(a), ct.byref(m))
            wi[r * nb + b], wm[r * nb + b] = a.value, m.value
    assert np.array_equal(isc, wi)
    assert np.array_equal(imn, wm)


@pytest.mark.parametrize("code", [4, 5])
@pytest.mark.parametrize("n_out,n_in,nvec", [(64, 256, 1), (1000, 2048, 1), (512, 2048, 8), (200, 768, 4),
                                             (14336, 4096, 1), (4096, 14336, 1), (14336, 4096, 8),
                                             (4096, 14336, 8)])
def test_gemv_q8k_vs_oracle(hip, oracle, code, n_out, n_in, nvec):
    from dracohip import lib
    rng = np.random.default_rng(1)
    W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
    x = _x(n_in, nvec, 3)
    xq = np.concatenate([oracle.quantize_q8k(x[v]) for v in range(nvec)])
    y = np.zeros(nvec * n_out, np.float32)
    lib.check(hip.draco_gemv_q8k(code, lib.pu8(xq), nvec, lib.pu8(W), n_out, n_in, lib.pf(y)), "draco_gemv_q8k")
    y2 = np.zeros_like(y)
    lib.check(hip.draco_gemv_q8k_f32(code, lib.pf(x), nvec, lib.pu8(W), n_out, n_in, lib.pf(y2)),
              "draco_gemv_q8k_f32")
    for v in range(nvec):
        ref = oracle.gemv_q8k(code, xq[v * (n_in // 256) * Q8K:(v + 1) * (n_in // 256) * Q8K], W, n_out, n_in)
        assert rel_err(y[v * n_out:(v + 1) * n_out], ref) <= TOL
        # on-device quantization gives the same bytes, hence the same result
        assert np.array_equal(y2[v * n_out:(v + 1) * n_out], y[v * n_out:(v + 1) * n_out])


@pytest.mark.parametrize("code", [4, 5])
def test_gemv_q8k_f32_in_block_quantizer_edge_cases(hip, oracle, code):
    """One vector through draco_gemv_q8k_f32 (the GEMV launch quantizes x
    itself) equals the GEMV over the oracle's Q8_K bytes bit for bit on the
    quantizer's edge cases: an all-zero super-block (d = 0), a largest |x|
    held twice with opposite signs (the first index sets the sign), a negative
    maximum, products exactly halfway between integers (round half to even)
    and a value that clamps at 127."""
    from dracohip import lib
    n_out, n_in = 256, 1536
    rng = np.random.default_rng(5)
    W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(n_in).astype(np.float32)
    x[256:512] = 0.0                                    # all zero
    b = x[512:768]
    b[:] = rng.uniform(-1, 1, 256).astype(np.float32)
    b[10], b[200] = 3.0, -3.0                           # tie: +3 first
    c = x[768:1024]
    c[:] = rng.uniform(-1, 1, 256).astype(np.float32)
    c[77], c[78] = -3.0, 3.0                            # tie: -3 first
    d = x[1024:1280]
    d[:] = np.arange(256, dtype=np.float32) % 64 - 31.5  # iscale * x = n + 0.5 for m = -127
    d[5] = -127.0                                       # m = -127: iscale = 1
    e = x[1280:1536]
    e[:] = rng.uniform(-1, 1, 256).astype(np.float32)
    e[3] = -1.5                                         # negative max: iscale > 0, x = +1.5 -> ... clamps
    e[9] = 1.4999999
    xq = oracle.quantize_q8k(x)
    y = np.zeros(n_out, np.float32)
    lib.check(hip.draco_gemv_q8k(code, lib.pu8(xq), 1, lib.pu8(W), n_out, n_in, lib.pf(y)), "draco_gemv_q8k")
    y2 = np.zeros_like(y)
    lib.check(hip.draco_gemv_q8k_f32(code, lib.pf(x), 1, lib.pu8(W), n_out, n_in, lib.pf(y2)),
              "draco_gemv_q8k_f32")
    assert np.array_equal(y, y2)
    assert rel_err(y, oracle.gemv_q8k(code, xq, W, n_out, n_in)) <= TOL


def test_gemv_q8k_rejects_bad_input(hip):
    from dracohip import lib
    W = np.zeros(144 * 4, np.uint8)
    xq = np.zeros(Q8K * 4, np.uint8)
    y = np.zeros(16, np.float32)
    assert hip.draco_gemv_q8k(0, lib.pu8(xq), 1, lib.pu8(W), 4, 256, lib.pf(y)) == -1   # Q8_0 weights
    assert hip.draco_gemv_q8k(5, lib.pu8(xq), 3, lib.pu8(W), 4, 256, lib.pf(y)) == -1   # nvec 3
    assert hip.draco_gemv_q8k(5, lib.pu8(xq), 1, lib.pu8(W), 4, 100, lib.pf(y)) == -1   # n_in % 256
