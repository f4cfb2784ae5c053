"""Pins the oracle's Q8_K functions (or_quantize_q8k, or_q8k_block_isums,
or_gemv_q8k).  The reference has no Q8_K path, so these checks stand on the
block format's definition (llama.cpp b10819 quantize_row_q8_K_ref) and on
independent computations: numpy decoders (dracohip.gguf_np), int64 brute
force, fp64 dots of the dequantized operands, and hand-built blocks whose
answer is known in closed form.  Each check is chosen so that a plausible
slip (last-index tie-break, half-away rounding, a dropped min term, a wrong
nibble or scale index) fails it.
"""
import numpy as np
import pytest

Q8K = 292


def unpack(blocks):
    b = blocks.reshape(-1, Q8K)
    d = b[:, :4].copy().view(np.float32)[:, 0]
    qs = b[:, 4:260].view(np.int8).astype(np.int64)
    bs = b[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, qs, bs


def test_q8k_invariants(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(256 * 32).astype(np.float32) * np.float32(3.0)
    d, qs, bs = unpack(oracle.quantize_q8k(x))
    xb = x.reshape(-1, 256).astype(np.float64)
    assert np.all(np.abs(qs) <= 127)
    assert np.array_equal(bs, qs.reshape(-1, 16, 16).sum(axis=2))
    # reconstruction within half a step; the element of largest |x| maps to -127
    err = np.abs(xb - d[:, None].astype(np.float64) * qs)
    assert np.all(err <= np.abs(d[:, None]) * 0.5 * (1 + 1e-6))
    imax = np.argmax(np.abs(xb), axis=1)
    assert np.all(qs[np.arange(len(imax)), imax] == -127)
    # d = 1 / (-127 / max), computed in fp32
    mx = xb[np.arange(len(imax)), imax].astype(np.float32)
    assert np.array_equal(d, (np.float32(1.0) / (np.float32(-127.0) / mx)).astype(np.float32))


def test_q8k_zero_block(oracle):
    x = np.zeros(512, np.float32)
    x[256 + 5] = 1.0
    d, qs, bs = unpack(oracle.quantize_q8k(x))
    assert d[0] == 0.0 and not qs[0].any() and not bs[0].any()
    assert qs[1, 5] == -127 and qs[1].sum() == -127


def test_q8k_first_index_wins_ties(oracle):
    x = np.zeros(256, np.float32)
    x[3], x[7] = 2.0, -2.0  # equal |x|: the first (positive) one sets the sign of the scale
    d, qs, _ = unpack(oracle.quantize_q8k(x))
    assert qs[0, 3] == -127 and qs[0, 7] == 127 and d[0] < 0


def test_q8k_rounds_half_to_even(oracle):
    x = np.zeros(256, np.float32)
    x[0] = -127.0          # iscale = 1 exactly
    x[1], x[2], x[3], x[4] = 2.5, 3.5, -2.5, 0.5
    _, qs, _ = unpack(oracle.quantize_q8k(x))
    assert list(qs[0, 1:5]) == [2, 4, -2, 0]


def _brute_isums(code, wblk, qs, bs):
    """int64 brute force from the numpy decoders' integer fields."""
    from dracohip import gguf_np
    if code == 5:
        sc, mn = gguf_np._kscales(wblk[4:16].reshape(1, 12))
        sc, mn = sc[0].astype(np.int64), mn[0].astype(np.int64)
        q = np.zeros(256, np.int64)
        for j in range(8):
            seg = wblk[16 + (j // 2) * 32: 16 + (j // 2) * 32 + 32].astype(np.int64)
            q[j * 32:(j + 1) * 32] = (seg >> 4) if (j & 1) else (seg & 15)
        t = (q * qs).reshape(8, 32).sum(axis=1)
        isc = int((np.asarray(sc, np.int64) * t).sum())
        imn = int(sum(int(mn[j]) * int(bs[2 * j] + bs[2 * j + 1]) for j in range(8)))
        return isc, imn
    ql, qh = wblk[:128].astype(np.int64), wblk[128:192].astype(np.int64)
    sc = wblk[192:208].view(np.int8).astype(np.int64)
    q = np.zeros(256, np.int64)
    for p in range(256):
        lo = ql[(p >> 7) * 64 + (p & 63)]
        lo = (lo >> 4) if ((p >> 6) & 1) else (lo & 15)
        hi = (qh[(p >> 7) * 32 + (p & 31)] >> (((p >> 5) & 3) * 2)) & 3
        q[p] = (lo | (hi << 4)) - 32
    t = (q * qs).reshape(16, 16).sum(axis=1)
    return int((sc * t).sum()), 0


@pytest.mark.parametrize("code", [4, 5])
def test_block_isums_brute_force(oracle, code):
    from dracohip import lib
    import ctypes as ct
    rng = np.random.default_rng(code)
    W = lib.quantize(code, rng.standard_normal((6, 512), dtype=np.float32) * np.float32(0.5))
    xq = oracle.quantize_q8k(rng.standard_normal(512).astype(np.float32))
    _, qs, bs = unpack(xq)
    bb = 144 if code == 5 else 210
    for r in range(6):
        for b in range(2):
            wblk = W[r * 2 * bb + b * bb: r * 2 * bb + (b + 1) * bb]
            isc, imn = ct.c_int32(), ct.c_int32()
            oracle.lib.or_q8k_block_isums(code, lib.pu8(wblk), lib.pu8(xq[b * Q8K:(b + 1) * Q8K]),
                                          ct.byref(isc), ct.byref(imn))
            assert (isc.value, imn.value) == _brute_isums(code, wblk, qs[b], bs[b])


@pytest.mark.parametrize("code", [4, 5])
def test_gemv_q8k_matches_fp64_dot(oracle, code):
    from dracohip import gguf_np, lib
    rng = np.random.default_rng(10 + code)
    n_out, n_in = 40, 1024
    W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(n_in).astype(np.float32)
    xq = oracle.quantize_q8k(x)
    d, qs, _ = unpack(xq)
    xd = (d[:, None].astype(np.float64) * qs).reshape(-1)
    rb = W.size // n_out
    Wd = np.stack([gguf_np.dequant_row(code, W[r * rb:(r + 1) * rb]).astype(np.float64) for r in range(n_out)])
    ref = Wd @ xd
    y = oracle.gemv_q8k(code, xq, W, n_out, n_in)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
