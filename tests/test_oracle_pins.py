"""Pins for the oracle functions that no bitwise reference golden covers
directly: or_dequant_row (src/m5/m5_gemm.c:55-235), or_gemm (m5_gemm
semantics, src/m5/m5_gemm.c:249-272) and or_moe_tok (src/m6_moe_tok.c:44-161).

Each check is a function of an oracle build, so the same check runs on the
shipped oracle (must pass) and on builds with one planted slip (OR_MUTANT,
compiled into a temporary library here; must fail).  The slips are the
plausible mistakes each pin is meant to catch: a Q4_K nibble swap, a dropped
Q4_K min term, a Q6_K high-bit shift from the wrong index, a transposed GEMM
output and a token-batched MoE that weights every slot by slot 0's weight.
"""
import ctypes as ct
import os
import subprocess

import numpy as np
import pytest

import gen_golden as gg
from helpers import bits_equal, golden, rel_err
from dracohip import gguf_np
from oracle.oracle import HERE as ORACLE_DIR, Oracle, pf, pi32, pu8

DEQUANT_CODES = (0, 3, 4, 5, 7, 9)


def _same(code, a, b):
    """Bit for bit, except Q5_K: the reference's row decoder rounds
    (q*d)*sc - dmin*m (src/m5/m5_gemm.c:212-231) where its GEMV rounds
    (d*sc)*q - dmin*m (src/m5_kern_scalar.c:91-114), so the two agree to a
    couple of ulps of the product, not bitwise."""
    if code != 3:
        return bits_equal(a, b)
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return bool(np.all(np.abs(a - b) <= 2.0 ** -21 * np.maximum(np.abs(a), np.abs(b)) + 1e-30))


def check_dequant_row(orc):
    """Every row of or_dequant_row equals (a) the one-hot columns of or_gemv,
    which tests/test_oracle_golden.py pins bit for bit to the compiled scalar
    kernel (and (b) the golden column that kernel itself wrote), and (c) the
    numpy decoders of dracohip.gguf_np, bit for bit."""
    g = golden("gemv.npz")
    for i, (name, code, n_out, n_in) in enumerate(gg.GEMV_CASES):
        if code not in DEQUANT_CODES:
            continue
        W, _ = gg.gemv_inputs(code, n_out, n_in, 100 + i)
        D = orc.dequant(code, W, n_out, n_in)
        cols = np.empty((n_in, n_out), np.float32)
        e = np.zeros(n_in, np.float32)
        for c in range(n_in):
            e[c] = 1.0
            cols[c] = orc.gemv(code, e, W, n_out, n_in)
            e[c] = 0.0
        assert _same(code, np.ascontiguousarray(cols.T), D), (name, "one-hot columns")
        col = int(g[name + "_meta"][5])
        assert _same(code, np.ascontiguousarray(D[:, col]), g[name + "_col"]), (name, "reference column")
        rb = len(W) // n_out
        for r in range(n_out):
            assert bits_equal(gguf_np.dequant_row(code, W[r * rb:(r + 1) * rb]), D[r]), (name, "numpy row", r)


GEMM_CASES = [(5, 48, 512, 7), (4, 33, 768, 5), (0, 40, 960, 9), (5, 5, 2048, 3), (3, 24, 512, 4)]  # code, n_out, n_in, T


def _gemm(orc, code, X, W, n_out, n_in):
    T = X.shape[0]
    Y = np.zeros((T, n_out), np.float32)
    assert orc.lib.or_gemm(code, pf(np.ascontiguousarray(X)), pu8(W), T, n_out, n_in, pf(Y)) == 0
    return Y


def check_gemm(orc):
    """or_gemm == T stacked or_gemv up to summation order: the GEMM dots a
    dequantized row sequentially, the GEMV sums per block, so elementwise
    |Y_gemm - Y_gemv| <= 2 gamma_n sum|w||x| (gamma_n = n u / (1 - n u),
    u = 2^-24: each order is within gamma_n sum|w||x| of the exact dot).
    One-hot token rows return the weight columns exactly (T != n_out, so a
    transposed output cannot pass)."""
    u = 2.0 ** -24
    for k, (code, n_out, n_in, T) in enumerate(GEMM_CASES):
        rng = np.random.default_rng(900 + k)
        W = gg.dlib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
        X = rng.standard_normal((T, n_in)).astype(np.float32)
        Y = _gemm(orc, code, X, W, n_out, n_in)
        absW = np.abs(np.stack([gguf_np.dequant_row(code, W[r * (len(W) // n_out):(r + 1) * (len(W) // n_out)])
                                for r in range(n_out)]).astype(np.float64))
        gam = n_in * u / (1.0 - n_in * u)
        for t in range(T):
            yv = orc.gemv(code, X[t], W, n_out, n_in).astype(np.float64)
            bound = 2.0 * gam * (absW @ np.abs(X[t].astype(np.float64))) + 1e-30
            assert np.all(np.abs(Y[t].astype(np.float64) - yv) <= bound), (code, t)
        picks = rng.choice(n_in, T, replace=False)
        E = np.zeros((T, n_in), np.float32)
        E[np.arange(T), picks] = 1.0
        Y1 = _gemm(orc, code, E, W, n_out, n_in)
        for t in range(T):
            col = orc.gemv(code, E[t], W, n_out, n_in)
            assert _same(code, Y1[t], col), (code, "one-hot", t)


def _moe_tok(orc, T, n_used, inter, n_in, n_exp, X, order, wtop, ptrs, ec):
    y = np.zeros((T, n_in), np.float32)
    orc.lib.or_moe_tok(pf(X), pi32(order), pf(wtop), ct.c_void_p(ptrs.ctypes.data), pi32(ec), T, n_used, inter,
                       n_in, n_in, n_exp, pf(y))
    return y


def check_moe_tok(orc, tags=("small", "cfg3", "q6mix")):
    """(1) the compiled reference's m6_moe_tok (tests/golden/moetok.npz) within
    1e-5 normwise (its dots are 16-lane FMA trees); (2) token-batched ==
    token-serial bit for bit: with each token routed by or_moe_route, the
    batched FFN equals or_granite_moe run token by token."""
    import hashlib
    g = golden("moetok.npz")
    for tag, n_exp, n_used, inter, n_in, T, codes, seed in gg.MOETOK_CASES:
        if tag not in tags:
            continue
        mats, ptrs, ec, X, order, wtop = gg.moetok_inputs(n_exp, n_used, inter, n_in, T, codes, seed)
        assert hashlib.sha256(b"".join(m.tobytes() for m in mats)).digest() == g[f"{tag}_digest"].tobytes()
        y = _moe_tok(orc, T, n_used, inter, n_in, n_exp, X, order, wtop, ptrs, ec)
        assert rel_err(y, g[f"{tag}_y"]) <= 1e-5, (tag, rel_err(y, g[f"{tag}_y"]))
        # token-serial: route every token with the softmax router, then compare
        rng = np.random.default_rng(seed + 1)
        gate_inp = rng.standard_normal((n_exp, n_in), dtype=np.float32) * np.float32(0.05)
        probs = np.zeros(n_exp, np.float32)
        o2 = np.zeros((T, n_used), np.int32)
        w2 = np.zeros((T, n_used), np.float32)
        serial = np.zeros((T, n_in), np.float32)
        scratch = np.zeros(3 * n_used * inter + n_used * n_in + 64, np.float32)
        for t in range(T):
            idx = np.zeros(n_used, np.int32)
            wt = np.zeros(n_used, np.float32)
            orc.lib.or_moe_route(pf(X[t]), pf(gate_inp), n_exp, n_used, n_in, pf(probs), pi32(idx), pf(wt))
            o2[t], w2[t] = idx, wt
            orc.lib.or_granite_moe(pf(X[t]), ct.c_void_p(ptrs.ctypes.data), pi32(ec), pf(gate_inp), n_exp, n_used,
                                   inter, n_in, n_in, pf(scratch), pf(serial[t]))
        batched = _moe_tok(orc, T, n_used, inter, n_in, n_exp, X, o2, w2, ptrs, ec)
        assert bits_equal(batched, serial), (tag, "token-batched != token-serial")


def test_dequant_row_pinned(oracle):
    check_dequant_row(oracle)


def test_gemm_pinned(oracle):
    check_gemm(oracle)


def test_moe_tok_pinned(oracle):
    check_moe_tok(oracle)


MUTANTS = [(1, check_dequant_row), (2, check_dequant_row), (3, check_dequant_row), (4, check_gemm),
           (5, lambda o: check_moe_tok(o, tags=("small",)))]


@pytest.mark.parametrize("mutant,check", MUTANTS, ids=[f"mutant{m}" for m, _ in MUTANTS])
def test_pins_catch_planted_slips(tmp_path, mutant, check):
    """The oracle built with one planted slip (OR_MUTANT) fails its pin."""
    so = str(tmp_path / f"liboracle_m{mutant}.so")
    src = os.path.join(ORACLE_DIR, "draco_oracle.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-fopenmp",
                    f"-DOR_MUTANT={mutant}", "-o", so, src, "-lm"], check=True)
    with pytest.raises(AssertionError):
        check(Oracle(so))


def test_argmax_matches_numpy(oracle):
    """or_argmax is np.argmax over a float64 copy (src/smol_engine.py:212):
    the first maximum, and the first NaN whenever a value is NaN."""
    rng = np.random.default_rng(7)
    cases = [np.array([1.0, 3.0, 3.0, 2.0], np.float32), np.full(5, -np.inf, np.float32),
             np.full(4, np.nan, np.float32), np.array([np.inf, 1.0, np.inf], np.float32),
             np.array([-np.inf, np.nan, 5.0, np.nan], np.float32), np.array([2.0, np.inf, np.nan], np.float32)]
    for _ in range(200):
        v = rng.standard_normal(int(rng.integers(1, 300))).astype(np.float32)
        v[rng.integers(0, len(v), 3)] = v.max()  # ties of the maximum
        if rng.random() < 0.5:
            v[rng.integers(0, len(v), int(rng.integers(1, 3)))] = np.nan
        if rng.random() < 0.3:
            v[rng.integers(0, len(v))] = rng.choice([np.inf, -np.inf])
        cases.append(v)
    for v in cases:
        assert oracle.lib.or_argmax(pf(v), len(v)) == int(np.argmax(v.astype(np.float64))), v
