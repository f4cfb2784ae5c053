"""MoE on the GPU through the reference ABI: m6_granite_moe (src/m6_layer.c:771-802),
the qwen35moe shared expert m6_granite_shexp (src/m6_engine.c:1111-1127)
and m5_gemvn_q4k / m5_gemvn_q6k (src/m5/m5_batch8_k.c:80-183).

Checks: the compiled reference's own outputs (tests/golden/moe.npz, weights
regenerated from the recorded seed and checked by digest), the oracle at the
configs[3] shape with Q4_K experts, ties in the router, and the grouped GEMV
with shared and per-expert x.  Bar: max|dy| <= 1e-5 * max|y_ref|.
"""
import ctypes as ct
import hashlib

import numpy as np
import pytest

import gen_golden as gg
from helpers import golden, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def build_moe(n_exp, inter, n_in, n_out, seed, codes3=(5, 5, 4), digest_order=True):
    from dracohip import lib
    rng = np.random.default_rng(seed)
    gate_inp = rng.standard_normal((n_exp, n_in), dtype=np.float32) * np.float32(0.02)
    Wg = lib.quantize(codes3[0], rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02))
    Wu = lib.quantize(codes3[1], rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02))
    Wd = lib.quantize(codes3[2], rng.standard_normal((n_exp * n_out, inter), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(n_in, dtype=np.float32)
    pg, pu, pd = Wg.nbytes // n_exp, Wu.nbytes // n_exp, Wd.nbytes // n_exp
    ptrs = np.zeros(3 * n_exp, np.uint64)
    codes = np.zeros(3 * n_exp, np.int32)
    for e in range(n_exp):
        ptrs[3 * e:3 * e + 3] = (Wg.ctypes.data + e * pg, Wu.ctypes.data + e * pu, Wd.ctypes.data + e * pd)
        codes[3 * e:3 * e + 3] = codes3
    return dict(gate_inp=gate_inp, Wg=Wg, Wu=Wu, Wd=Wd, x=x, ptrs=ptrs, codes=codes)


def run_hip(hip, M, n_exp, n_used, inter, n_in, n_out):
    from dracohip import lib
    y = np.zeros(n_out, np.float32)
    scratch = np.zeros(8, np.float32)
    hip.m6_granite_moe(lib.pf(M["x"]), ct.c_void_p(M["ptrs"].ctypes.data), lib.pi32(M["codes"]),
                       lib.pf(M["gate_inp"]), n_exp, n_used, inter, n_in, n_out, lib.pf(scratch), lib.pf(y))
    return y


def run_oracle(oracle, M, n_exp, n_used, inter, n_in, n_out):
    from dracohip import lib
    y = np.zeros(n_out, np.float32)
    scratch = np.zeros(3 * n_used * inter + n_used * n_out + 64, np.float32)
    oracle.lib.or_granite_moe(lib.pf(M["x"]), ct.c_void_p(M["ptrs"].ctypes.data), lib.pi32(M["codes"]),
                              lib.pf(M["gate_inp"]), n_exp, n_used, inter, n_in, n_out, lib.pf(scratch), lib.pf(y))
    return y


@pytest.mark.parametrize("tag", ["small", "cfg4"])
def test_granite_moe_vs_reference_golden(hip, tag):
    g = golden("moe.npz")
    n_exp, n_used, inter, n_in, seed = [int(v) for v in g[f"{tag}_meta"]]
    M = build_moe(n_exp, inter, n_in, n_in, seed)
    assert hashlib.sha256(M["Wg"].tobytes() + M["Wu"].tobytes() + M["Wd"].tobytes()).digest() == \
        g[f"{tag}_digest"].tobytes()
    y = run_hip(hip, M, n_exp, n_used, inter, n_in, n_in)
    assert rel_err(y, g[f"{tag}_y"]) <= TOL


def test_granite_moe_configs3_q4k_experts(hip, oracle):
    # hidden 2048, 128 experts, top-8, expert FFN 768, Q4_K experts
    n_exp, n_used, inter, H = 128, 8, 768, 2048
    M = build_moe(n_exp, inter, H, H, 33, codes3=(5, 5, 5))
    for k in range(3):  # three tokens through the same registered experts
        M["x"] = np.random.default_rng(100 + k).standard_normal(H).astype(np.float32)
        y = run_hip(hip, M, n_exp, n_used, inter, H, H)
        ref = run_oracle(oracle, M, n_exp, n_used, inter, H, H)
        assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("n_exp,n_used", [(300, 6), (512, 16), (512, 1), (40, 8), (128, 24), (512, 64), (64, 64)])
def test_granite_moe_expert_counts(hip, oracle, n_exp, n_used):
    """Routers wider than the routing block (256 threads at n_in 512, so
    experts 256 and up are ranked in a second pass), the 512-expert limit,
    the largest top-k one down launch serves (16), top-1, and top-k above 16
    up to the reference's 64 (src/m6_layer.c:797: down launches of 16 slots
    chained in slot order), including every expert selected."""
    inter, H = 256, 512
    M = build_moe(n_exp, inter, H, H, 40 + n_used)
    y = run_hip(hip, M, n_exp, n_used, inter, H, H)
    ref = run_oracle(oracle, M, n_exp, n_used, inter, H, H)
    assert rel_err(y, ref) <= TOL, rel_err(y, ref)


def test_granite_moe_router_ties_pick_lowest_index(hip, oracle):
    n_exp, n_used, inter, H = 16, 4, 256, 512
    M = build_moe(n_exp, inter, H, H, 5)
    gi = M["gate_inp"]
    gi[3] = gi[11]  # experts 3 and 11 score identically; 5 and 6 too
    gi[6] = gi[5]
    gi[11] *= np.float32(4.0)  # make the tied pairs likely winners
    gi[3] = gi[11]
    y = run_hip(hip, M, n_exp, n_used, inter, H, H)
    ref = run_oracle(oracle, M, n_exp, n_used, inter, H, H)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("code", [4, 5])
@pytest.mark.parametrize("per_expert_x", [False, True])
def test_gemvn_grouped(hip, oracle, code, per_expert_x):
    from dracohip import lib
    n_tot, n_sel, n_out_e, n_in = 32, 8, 768, 2048
    rng = np.random.default_rng(code + 2 * per_expert_x)
    W = lib.quantize(code, rng.standard_normal((n_tot * n_out_e, n_in), dtype=np.float32) * np.float32(0.02))
    per = W.nbytes // n_tot
    idx = np.array(rng.choice(n_tot, n_sel, replace=False), np.int32)
    x_stride = n_in if per_expert_x else 0
    x = rng.standard_normal(n_sel * n_in if per_expert_x else n_in).astype(np.float32)
    y = np.zeros(n_sel * n_out_e, np.float32)
    fn = hip.m5_gemvn_q4k if code == 5 else hip.m5_gemvn_q6k
    assert fn(lib.pf(x), x_stride, lib.pu8(W), lib.pi32(idx), per, n_out_e, n_in, n_sel, lib.pf(y)) == 0
    ref = np.zeros_like(y)
    ofn = oracle.lib.or_gemvn_q4k if code == 5 else oracle.lib.or_gemvn_q6k
    assert ofn(lib.pf(x), x_stride, lib.pu8(W), lib.pi32(idx), per, n_out_e, n_in, n_sel, lib.pf(ref)) == 0
    for e in range(n_sel):
        assert rel_err(y[e * n_out_e:(e + 1) * n_out_e], ref[e * n_out_e:(e + 1) * n_out_e]) <= TOL


def test_gemvn_rejects_like_reference(hip):
    from dracohip import lib
    x = np.zeros(512, np.float32)
    W = np.zeros(144 * 2 * 16, np.uint8)
    idx = np.zeros(1, np.int32)
    y = np.zeros(16, np.float32)
    assert hip.m5_gemvn_q4k(lib.pf(x), 0, lib.pu8(W), lib.pi32(idx), 0, 16, 300, 1, lib.pf(y)) == -1


@pytest.mark.parametrize("n_exp,n_used,inter,H,T,codes3", [(16, 4, 256, 512, 20, (5, 5, 4)),
                                                           (128, 8, 768, 2048, 48, (5, 5, 5))])
def test_moe_tok_vs_oracle(hip, oracle, n_exp, n_used, inter, H, T, codes3):
    from dracohip import lib
    M = build_moe(n_exp, inter, H, H, 61 + T, codes3=codes3)
    rng = np.random.default_rng(T)
    X = rng.standard_normal((T, H)).astype(np.float32)
    # routing as the caller would pass it: distinct experts per token, softmax-like weights;
    # one invalid expert id (skipped by both) and experts with no tokens
    order = np.stack([rng.choice(n_exp // 2, n_used, replace=False) for _ in range(T)]).astype(np.int32)
    order[3, 1] = -1
    wtop = rng.random((T, n_used)).astype(np.float32)
    wtop /= wtop.sum(axis=1, keepdims=True)
    y = np.zeros((T, H), np.float32)
    z = np.zeros(8, np.float32)
    zi = np.zeros(8, np.int32)
    hip.m6_moe_tok(None, None, lib.pf(z), lib.pf(X), lib.pi32(order), lib.pf(wtop), ct.c_void_p(M["ptrs"].ctypes.data),
                   lib.pi32(M["codes"]), T, n_used, inter, H, H, n_exp, lib.pf(y), lib.pf(z), lib.pi32(zi))
    ref = np.zeros_like(y)
    oracle.lib.or_moe_tok(lib.pf(X), lib.pi32(order), lib.pf(wtop), ct.c_void_p(M["ptrs"].ctypes.data),
                          lib.pi32(M["codes"]), T, n_used, inter, H, H, n_exp, lib.pf(ref))
    assert rel_err(y, ref) <= TOL


def run_shexp(fn, ptrs, cds, x, shi, h):
    from dracohip import lib
    sg, sh, shg, y = (np.zeros(1, np.float32), np.zeros(2 * shi, np.float32), np.zeros(h, np.float32),
                      np.zeros(h, np.float32))
    fn(lib.pf(x), ct.c_void_p(ptrs.ctypes.data), lib.pi32(cds), lib.pf(sg), lib.pf(sh), lib.pf(shg), lib.pf(y),
       shi, h)
    return y, shg, sg, sh[:shi]


@pytest.mark.parametrize("tag", ["small", "q35", "mixed", "q8gate", "small"])
def test_granite_shexp_vs_reference_golden(hip, oracle, tag):
    """Golden from the compiled reference (Q4_K/Q6_K with an F32 gate row; a
    Q4_K/Q8_0 mix with an F16 gate row; Q8_0 gate with Q4_K up, which takes
    the two-launch gate/up path, and a Q8_0 gate row, which takes the one-row
    GEMV before the scale); "small" runs again after the other shapes so the
    cached descriptor is re-resolved."""
    import gen_golden as gg
    g = golden("shexp.npz")
    _, shi, h, codes, seed = [c for c in gg.SHEXP_CASES if c[0] == tag][0]
    ws, x, ptrs, cds = gg.shexp_inputs(shi, h, codes, seed)
    assert hashlib.sha256(b"".join(w.tobytes() for w in ws)).digest() == g[f"{tag}_digest"].tobytes()
    y, shg, sg, act = run_shexp(hip.m6_granite_shexp, ptrs, cds, x, shi, h)
    assert rel_err(y, g[f"{tag}_out"]) <= TOL, rel_err(y, g[f"{tag}_out"])
    assert rel_err(shg, g[f"{tag}_shg"]) <= TOL
    assert abs(float(sg[0]) - float(g[f"{tag}_sg"][0])) <= TOL * max(1.0, abs(float(g[f"{tag}_sg"][0])))
    assert rel_err(act, g[f"{tag}_act"]) <= TOL
    yo, _, _, _ = run_shexp(oracle.lib.or_granite_shexp, ptrs, cds, x, shi, h)
    assert rel_err(y, yo) <= TOL


@pytest.mark.parametrize("tag", [c[0] for c in __import__("gen_golden").MOETOK_CASES])
def test_moe_tok_vs_reference_golden(hip, tag):
    """m6_moe_tok against the compiled reference's token-batched MoE
    (tests/golden/moetok.npz): Q4_K / Q6_K experts, experts with no tokens and
    an invalid slot (-1)."""
    import gen_golden as gg
    from dracohip import lib
    g = golden("moetok.npz")
    _, n_exp, n_used, inter, H, T, codes, seed = [c for c in gg.MOETOK_CASES if c[0] == tag][0]
    mats, ptrs, ec, X, order, wtop = gg.moetok_inputs(n_exp, n_used, inter, H, T, codes, seed)
    assert hashlib.sha256(b"".join(m.tobytes() for m in mats)).digest() == g[f"{tag}_digest"].tobytes()
    y = np.zeros((T, H), np.float32)
    z = np.zeros(8, np.float32)
    zi = np.zeros(8, np.int32)
    print(f"[moe_tok] {tag} vs reference golden", flush=True)
    hip.m6_moe_tok(None, None, lib.pf(z), lib.pf(X), lib.pi32(order), lib.pf(wtop), ct.c_void_p(ptrs.ctypes.data),
                   lib.pi32(ec), T, n_used, inter, H, H, n_exp, lib.pf(y), lib.pf(z), lib.pi32(zi))
    assert rel_err(y, g[f"{tag}_y"]) <= TOL, rel_err(y, g[f"{tag}_y"])


def test_unserved_moe_inputs_leave_nan(hip):
    """The void MoE entry points cannot return an error code (as the
    reference's): for input they do not serve (IQ3_S experts, which the
    reference's qwen35 prefill passes to m6_moe_tok) they leave NaN in out
    instead of stale values."""
    from dracohip import lib
    n_exp, n_used, inter, H = 16, 4, 256, 512
    M = build_moe(n_exp, inter, H, H, 70)
    codes = M["codes"].copy()
    codes[:] = 2  # IQ3_S
    y = np.zeros(H, np.float32)
    scratch = np.zeros(8, np.float32)
    hip.m6_granite_moe(lib.pf(M["x"]), ct.c_void_p(M["ptrs"].ctypes.data), lib.pi32(codes), lib.pf(M["gate_inp"]),
                       n_exp, n_used, inter, H, H, lib.pf(scratch), lib.pf(y))
    assert np.all(np.isnan(y))
    T = 3
    X = np.ones((T, H), np.float32)
    order = np.tile(np.arange(n_used, dtype=np.int32), (T, 1))
    wtop = np.full((T, n_used), 1.0 / n_used, np.float32)
    out = np.zeros((T, H), np.float32)
    z = np.zeros(8, np.float32)
    zi = np.zeros(8, np.int32)
    hip.m6_moe_tok(None, None, lib.pf(z), lib.pf(X), lib.pi32(order), lib.pf(wtop), ct.c_void_p(M["ptrs"].ctypes.data),
                   lib.pi32(codes), T, n_used, inter, H, H, n_exp, lib.pf(out), lib.pf(z), lib.pi32(zi))
    assert np.all(np.isnan(out))


@pytest.mark.parametrize("tag", [c[0] for c in gg.MOE_BATCH4_CASES])
def test_moe_batch4_vs_reference_golden(hip, tag):
    """m6_moe_batch4 (src/m6_layer.c:656-690): given experts and weights,
    against the compiled reference's output on the same bytes."""
    from dracohip import lib
    g = golden("moe_batch4.npz")
    tag_, n, inter, n_in, n_out, codes, seed = [c for c in gg.MOE_BATCH4_CASES if c[0] == tag][0]
    M = gg.moe_batch4_inputs(n, inter, n_in, n_out, codes, seed)
    assert hashlib.sha256(M["Wg"].tobytes() + M["Wu"].tobytes() + M["Wd"].tobytes()).digest() == \
        g[f"{tag}_digest"].tobytes()
    y = np.full(n_out, np.nan, np.float32)
    print(f"[moe_batch4] {tag}: {n} experts {inter}x{n_in} -> {n_out}", flush=True)
    for _ in range(2):  # the second call reuses the registered experts
        hip.m6_moe_batch4(lib.pf(M["x"]), ct.c_void_p(M["ptrs"].ctypes.data), lib.pi32(M["codes"]), lib.pf(M["wtop"]),
                          n, inter, n_in, n_out, lib.pf(np.zeros(4, np.float32)), lib.pf(y))
        assert rel_err(y, g[f"{tag}_y"]) <= TOL


def test_moe_batch4_unserved_leaves_nan(hip):
    """More experts than the device path serves, or IQ formats: NaN, not stale values."""
    from dracohip import lib
    M = gg.moe_batch4_inputs(8, 256, 512, 512, (5, 5, 4), 70)
    y = np.zeros(512, np.float32)
    bad = M["codes"].copy()
    bad[2::3] = 2  # IQ3_S down projections
    hip.m6_moe_batch4(lib.pf(M["x"]), ct.c_void_p(M["ptrs"].ctypes.data), lib.pi32(bad), lib.pf(M["wtop"]),
                      8, 256, 512, 512, lib.pf(np.zeros(4, np.float32)), lib.pf(y))
    assert np.isnan(y).all()

