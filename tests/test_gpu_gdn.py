"""Gated-DeltaNet scan on the GPU through m6_gdn_scan (src/m6_gdn_scan.c:18-93).

Checks: the compiled reference's outputs (tests/golden/gdn.npz), the oracle at
the configs[4] head shape (32 V heads, 16 q/k heads, 128-wide), chunked ==
one-shot (state and tail carried through the ABI), and the beta = 0 closed
form (the state only decays).  Bars: ON and S within 1e-5 of max|ref|
(normwise); the conv tail is a copy of the last three inputs, bit-exact.
"""
import numpy as np
import pytest

import gen_golden as gg
from helpers import golden, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def scan(hip, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S):
    from dracohip import lib
    tail, S = tail.copy(), S.copy()
    ON = np.zeros((T, n_vh * 128), np.float32)
    work = np.zeros(8, np.float32)
    hip.m6_gdn_scan(lib.pf(QKV), lib.pf(Z), lib.pf(B), lib.pf(G), lib.pf(conv), lib.pf(ssm_norm), lib.pf(tail),
                    lib.pf(S), T, n_qkv, n_vh, lib.pf(ON), lib.pf(work))
    return ON, S, tail


def scan_oracle(oracle, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S):
    from dracohip import lib
    tail, S = tail.copy(), S.copy()
    ON = np.zeros((T, n_vh * 128), np.float32)
    work = np.zeros(n_qkv, np.float32)
    oracle.lib.or_gdn_scan(lib.pf(QKV), lib.pf(Z), lib.pf(B), lib.pf(G), lib.pf(conv), lib.pf(ssm_norm),
                           lib.pf(tail), lib.pf(S), T, n_qkv, n_vh, lib.pf(ON), lib.pf(work))
    return ON, S, tail


@pytest.mark.parametrize("tag", ["a", "b"])
def test_gdn_scan_vs_reference_golden(hip, oracle, tag):
    g = golden("gdn.npz")
    T, n_vh, nhq, seed = [int(v) for v in g[f"{tag}_meta"]]
    n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, n_vh, nhq, seed)
    ON, S2, tail2 = scan(hip, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    assert rel_err(ON, g[f"{tag}_ON"]) <= TOL
    assert rel_err(S2[::997], g[f"{tag}_S_sample"]) <= TOL
    _, So, tailo = scan_oracle(oracle, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    assert rel_err(S2, So) <= TOL
    assert np.array_equal(tail2, tailo)


def test_gdn_scan_configs4_heads(hip, oracle):
    T, n_vh, nhq = 64, 32, 16
    n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, n_vh, nhq, 41)
    ON, S2, tail2 = scan(hip, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    ONo, So, tailo = scan_oracle(oracle, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    assert rel_err(ON, ONo) <= TOL
    assert rel_err(S2, So) <= TOL
    assert np.array_equal(tail2, tailo)


def test_gdn_chunked_equals_one_shot(hip):
    T, n_vh, nhq = 48, 8, 4
    n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, n_vh, nhq, 43)
    ON1, S1, t1 = scan(hip, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    ON2 = np.zeros_like(ON1)
    St, tt = S.copy(), tail.copy()
    for t0 in range(0, T, 16):
        sl = slice(t0, t0 + 16)
        on, St, tt = scan(hip, 16, n_qkv, n_vh, np.ascontiguousarray(QKV[sl]), np.ascontiguousarray(Z[sl]),
                          np.ascontiguousarray(B[sl]), np.ascontiguousarray(G[sl]), conv, ssm_norm, tt, St)
        ON2[sl] = on
    assert np.array_equal(ON1, ON2) and np.array_equal(S1, St) and np.array_equal(t1, tt)


def test_gdn_beta_zero_only_decays(hip):
    T, n_vh, nhq = 7, 4, 2
    n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, n_vh, nhq, 44)
    B[:] = 0.0
    _, S2, _ = scan(hip, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    decay = np.prod(G.astype(np.float64), axis=0)  # [n_vh]
    want = S.reshape(n_vh, -1).astype(np.float64) * decay[:, None]
    assert rel_err(S2.reshape(n_vh, -1), want) <= 1e-6


def test_gdn_scan_configs4_4096_tokens_then_decode(hip, oracle):
    """configs[4]'s scan length: 4096 tokens in 64-token calls, then 64
    single-token calls (decode), at 32 V / 16 q-k heads of 128, the state and
    conv tail carried through the ABI; against the oracle's one-shot scan of
    all 4160 tokens.  Reports the worst normwise error of every call's outputs
    and of the final state (error growth over the recurrence)."""
    T, n_vh, nhq = 4096 + 64, 32, 16
    n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, n_vh, nhq, 45)
    S[:] = 0.0
    tail[:] = 0.0
    ONo, So, tailo = scan_oracle(oracle, T, n_qkv, n_vh, QKV, Z, B, G, conv, ssm_norm, tail, S)
    St, tt = S.copy(), tail.copy()
    worst, t0 = 0.0, 0
    while t0 < T:
        n = 64 if t0 < 4096 else 1
        sl = slice(t0, t0 + n)
        if t0 % 1024 == 0 or t0 >= 4096 and (t0 - 4096) % 16 == 0:
            print(f"[gdn] 4096-token scan: token {t0}, worst so far {worst:.2e}", flush=True)
        on, St, tt = scan(hip, n, n_qkv, n_vh, np.ascontiguousarray(QKV[sl]), np.ascontiguousarray(Z[sl]),
                          np.ascontiguousarray(B[sl]), np.ascontiguousarray(G[sl]), conv, ssm_norm, tt, St)
        e = rel_err(on, ONo[sl])
        worst = max(worst, e)
        assert e <= TOL, (t0, e)
        t0 += n
    es = rel_err(St, So)
    print(f"[gdn] 4096 + 64 tokens: worst per-call output error {worst:.2e}, final state {es:.2e}", flush=True)
    assert es <= TOL
    assert np.array_equal(tt, tailo)


@pytest.mark.parametrize("split", [1, 2, 4, 8])
@pytest.mark.parametrize("T", [2, 20])
def test_gdn_scan_column_split(hip, oracle, split, T):
    """The scan with each head's 128 state columns split over 1, 2, 4 or 8
    workgroups (the gated rms then in a second launch) against the oracle at
    the configs[4] head shape: outputs, state and tail.  (Single-token scans
    run unsplit; the split decode step is tested through m6_gdn_attn.)"""
    old = hip.draco_set_gdn_split(split, split)
    try:
        n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, 32, 16, 46 + T)
        print(f"[gdn] column split {split}, T {T}", flush=True)
        ON, S2, tail2 = scan(hip, T, n_qkv, 32, QKV, Z, B, G, conv, ssm_norm, tail, S)
    finally:
        hip.draco_set_gdn_split(old // 16, old % 16)
    ONo, So, tailo = scan_oracle(oracle, T, n_qkv, 32, QKV, Z, B, G, conv, ssm_norm, tail, S)
    assert rel_err(ON, ONo) <= TOL
    assert rel_err(S2, So) <= TOL
    assert np.array_equal(tail2, tailo)
