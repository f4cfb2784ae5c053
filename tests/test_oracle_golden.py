"""The CPU oracle (oracle/draco_oracle.c) against fixtures written by the
reference's own C (tests/golden/gen_golden.py drives oracle/_ref).

Bar: bit-identical outputs on identical inputs.
"""
import ctypes as ct

import numpy as np
import pytest

from helpers import bits_equal, golden
import gen_golden as gg
from dracohip import models
from dracohip.driver import LlamaDriver
from oracle.oracle import pf, pu8, pi32
from tests_oracle_engine import oracle_engine


@pytest.mark.parametrize("case", [c[0] for c in gg.GEMV_CASES])
def test_gemv_matches_reference(oracle, case):
    g = golden("gemv.npz")
    i = [c[0] for c in gg.GEMV_CASES].index(case)
    _, code, n_out, n_in = gg.GEMV_CASES[i]
    W, x = gg.gemv_inputs(code, n_out, n_in, 100 + i)
    y = oracle.gemv(code, x, W, n_out, n_in)
    assert bits_equal(y, g[case + "_y"]), (case, np.max(np.abs(y - g[case + "_y"])))
    code_, n_out_, n_in_, o0, o1, col = g[case + "_meta"]
    yr = np.full(n_out, np.float32(-7.0))
    oracle.gemv_range(code, x, W, n_out, n_in, int(o0), int(o1), yr)
    assert bits_equal(yr, g[case + "_yrange"])  # rows outside [o0,o1) untouched
    onehot = np.zeros(n_in, np.float32)
    onehot[int(col)] = 1.0
    assert bits_equal(oracle.gemv(code, onehot, W, n_out, n_in), g[case + "_col"])


def test_supported_codes(oracle):
    g = golden("gemv.npz")
    assert [oracle.lib.or_supported(c) for c in range(12)] == list(g["supported"])


@pytest.mark.parametrize("h", [960, 2048])
def test_rms_norm(oracle, h):
    g = golden("gemv.npz")
    x, w = g[f"rms{h}_x"], g[f"rms{h}_w"]
    o = np.zeros(h, np.float32)
    oracle.lib.or_rms_norm(pf(x), pf(w), h, ct.c_float(1e-5), pf(o))
    assert bits_equal(o, g[f"rms{h}_y"])


@pytest.mark.parametrize("i", range(len(gg.BATCH8K_CASES)))
def test_batch8k_lane_order(oracle, i):
    """AVX-512 grouped GEMV (src/m5/m5_batch8_k.c) restated lane by lane."""
    tag, code, perexp = gg.BATCH8K_CASES[i]
    W, x, idx, per, n_out_e, n_in, xstride = gg.batch8k_inputs(code, perexp, 40 + i)
    y = np.zeros(len(idx) * n_out_e, np.float32)
    fn = oracle.lib.or_gemvn_q4k if code == 5 else oracle.lib.or_gemvn_q6k
    assert fn(pf(x), xstride, pu8(W), pi32(idx), per, n_out_e, n_in, len(idx), pf(y)) == 0
    assert bits_equal(y, golden("batch8k.npz")[tag + "_y"])


@pytest.mark.parametrize("tag", ["a", "b"])
def test_gdn_scan(oracle, tag):
    import hashlib
    g = golden("gdn.npz")
    T, n_vh, nhq, seed = [int(v) for v in g[f"{tag}_meta"]]
    n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gg.gdn_inputs(T, n_vh, nhq, seed)
    ON = np.zeros((T, n_vh * 128), np.float32)
    work = np.zeros(n_qkv, np.float32)
    oracle.lib.or_gdn_scan(pf(QKV), pf(Z), pf(B), pf(G), pf(conv), pf(ssm_norm), pf(tail), pf(S),
                           T, n_qkv, n_vh, pf(ON), pf(work))
    assert bits_equal(ON, g[f"{tag}_ON"])
    assert hashlib.sha256(S.tobytes()).digest() == g[f"{tag}_S_sha"].tobytes()
    assert hashlib.sha256(tail.tobytes()).digest() == g[f"{tag}_tail_sha"].tobytes()


@pytest.mark.parametrize("tag", ["small", "cfg4"])
def test_granite_moe(oracle, tag):
    import hashlib
    from dracohip import lib as dlib
    g = golden("moe.npz")
    n_exp, n_used, inter, n_in, seed = [int(v) for v in g[f"{tag}_meta"]]
    rng = np.random.default_rng(seed)
    gate_inp = rng.standard_normal((n_exp, n_in), dtype=np.float32) * np.float32(0.02)
    Wg = dlib.quantize(5, rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02))
    Wu = dlib.quantize(5, rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02))
    Wd = dlib.quantize(4, rng.standard_normal((n_exp * n_in, inter), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(n_in, dtype=np.float32)
    assert hashlib.sha256(Wg.tobytes() + Wu.tobytes() + Wd.tobytes()).digest() == g[f"{tag}_digest"].tobytes()
    pg, pu, pd = Wg.nbytes // n_exp, Wu.nbytes // n_exp, Wd.nbytes // n_exp
    ptrs = np.zeros(3 * n_exp, np.uint64)
    codes = np.zeros(3 * n_exp, np.int32)
    for e in range(n_exp):
        ptrs[3 * e:3 * e + 3] = (Wg.ctypes.data + e * pg, Wu.ctypes.data + e * pu, Wd.ctypes.data + e * pd)
        codes[3 * e:3 * e + 3] = (5, 5, 4)
    scratch = np.zeros(3 * n_used * inter + n_used * n_in + 64, np.float32)
    y = np.zeros(n_in, np.float32)
    oracle.lib.or_granite_moe(pf(x), ct.c_void_p(ptrs.ctypes.data), pi32(codes), pf(gate_inp), n_exp,
                              n_used, inter, n_in, n_in, pf(scratch), pf(y))
    assert bits_equal(y, g[f"{tag}_y"])


@pytest.mark.parametrize("case", gg.SHEXP_CASES, ids=[c[0] for c in gg.SHEXP_CASES])
def test_granite_shexp(oracle, case):
    """qwen35moe shared expert (src/m6_engine.c:1111-1127): every array the
    reference writes (gated output, ungated product, gate logit, activation)."""
    import hashlib
    tag, shi, h, codes, seed = case
    g = golden("shexp.npz")
    ws, x, ptrs, cds = gg.shexp_inputs(shi, h, codes, seed)
    assert hashlib.sha256(b"".join(w.tobytes() for w in ws)).digest() == g[f"{tag}_digest"].tobytes()
    sg, sh, shg, y = (np.zeros(1, np.float32), np.zeros(2 * shi, np.float32), np.zeros(h, np.float32),
                      np.zeros(h, np.float32))
    oracle.lib.or_granite_shexp(pf(x), ct.c_void_p(ptrs.ctypes.data), pi32(cds), pf(sg), pf(sh), pf(shg), pf(y),
                                shi, h)
    assert bits_equal(y, g[f"{tag}_out"]) and bits_equal(shg, g[f"{tag}_shg"])
    assert bits_equal(sg, g[f"{tag}_sg"]) and bits_equal(sh[:shi], g[f"{tag}_act"])


@pytest.mark.parametrize("cfgname,fname", [("tiny-kquant", "llama_tiny_k.npz"), ("tiny-q8_0", "llama_tiny_q8.npz"),
                                          ("tiny-q5_k_m", "llama_tiny_q5.npz")])
def test_llama_decode_tiny(oracle, cfgname, fname):
    """Token-serial prefill + greedy decode through the descriptor ABI, bitwise."""
    g = golden(fname)
    cfg = models.CONFIGS[cfgname]
    model = models.build_llama(cfg, 0)
    assert model.digest() == g["digest"].tobytes().hex()
    drv = LlamaDriver(model, oracle_engine(oracle))
    toks, hidden, lg = drv.greedy(model.prompt(), cfg.n_gen, collect_logits=(0, 15))
    assert toks == list(g["tokens"])
    assert bits_equal(hidden, g["hidden"])
    assert bits_equal(lg[0], g["logits0"]) and bits_equal(lg[15], g["logits15"])


@pytest.mark.slow
def test_llama_decode_smol360m(oracle):
    """SmolLM2-360M-shaped Q8_0, 32 prompt + 64 greedy tokens, bitwise."""
    g = golden("smol360m.npz")
    cfg = models.SMOL360M
    model = models.build_llama(cfg, 0)
    assert model.digest() == g["digest"].tobytes().hex()
    drv = LlamaDriver(model, oracle_engine(oracle))
    toks, hidden, lg = drv.greedy(model.prompt(), cfg.n_gen, collect_logits=(0, 63))
    assert toks == list(g["tokens"])
    assert bits_equal(hidden, g["hidden"])
    assert bits_equal(lg[63][g["logits63_top_ids"]], g["logits63_top_vals"])


def _gdn_case(tag):
    g = golden("qwen35.npz")
    meta = [int(v) for v in g[f"gdn_{tag}_meta"]]
    return g, meta[0], tuple(meta[1:4]), meta[4], meta[5]


@pytest.mark.parametrize("tag", [c[0] for c in gg.QWEN_GDN_CASES])
def test_gdn_attn(oracle, tag):
    """m6_gdn_attn (src/m6_layer.c:205-364): the restatement reproduces the
    compiled reference over consecutive tokens.  Everything but the post-norm
    output is bitwise; x2n differs only by the order of the reference's
    per-thread partial sums of squares."""
    import hashlib
    from helpers import rel_err
    from dracohip import qwen35 as Q
    g, n_vh, codes, seed, steps = _gdn_case(tag)
    L = Q.gdn_layer(seed, n_vh, codes)
    h1 = Q.hidden(seed + 1000, steps)
    for s in range(steps):
        x2n, x2o = np.zeros(Q.H, np.float32), np.zeros(Q.H, np.float32)
        assert oracle.lib.or_gdn_attn(pf(h1[s]), L.ptr(), pf(L.ssm), pf(L.tail), pf(x2n), pf(x2o)) == 0
        assert bits_equal(x2o, g[f"gdn_{tag}_x2o_{s}"]), s
        assert rel_err(x2n, g[f"gdn_{tag}_x2n_{s}"]) < 1e-6, s
    assert bits_equal(L.tail, g[f"gdn_{tag}_tail"])
    assert hashlib.sha256(L.ssm.tobytes()).digest() == g[f"gdn_{tag}_ssm_sha"].tobytes()


@pytest.mark.parametrize("tag", [c[0] for c in gg.QWEN_FULL_CASES])
def test_full_attn(oracle, tag):
    """m6_full_attn (src/m6_layer.c:389-518): bitwise at every cache length,
    including pos0 != Told (rope position independent of the row count)."""
    from dracohip import qwen35 as Q
    case = [c for c in gg.QWEN_FULL_CASES if c[0] == tag][0]
    _, nh, codes, seed, steps = case
    g = golden("qwen35.npz")
    L = Q.full_layer(seed, nh, codes)
    for told, pos0 in steps:
        Kr, Vc = Q.kv_rows(seed + told, told)
        h1 = Q.hidden(seed + 2000 + told)[0]
        x2n, x2o = np.zeros(Q.H, np.float32), np.zeros(Q.H, np.float32)
        krn, vrn = np.zeros(512, np.float32), np.zeros(512, np.float32)
        assert oracle.lib.or_full_attn(pf(h1), L.ptr(), pf(Kr), pf(Vc), told, pos0, pf(x2n), pf(x2o),
                                       pf(krn), pf(vrn)) == 0
        k = f"full_{tag}_{told}_{pos0}"
        for name, v in (("x2n", x2n), ("x2o", x2o), ("krn", krn), ("vrn", vrn)):
            assert bits_equal(v, g[k + "_" + name]), (told, pos0, name)


def test_gdn_attn_closed_forms(oracle):
    """Invariants that do not lean on the reference: with every conv tap 0 the
    conv outputs are silu(0) = 0, so q = k = v = 0, the delta rule writes
    nothing and the state only decays, S_1 = exp(alpha) * S_0 per head (alpha
    recomputed here in float64 from the same inputs), and the layer output is
    the residual alone."""
    from dracohip import qwen35 as Q
    L = Q.gdn_layer(71, 16, (0, 0, 0))
    a = L.arrays
    a["conv"][:] = 0.0
    S0 = L.ssm.copy()
    h1 = Q.hidden(72)[0]
    x2n, x2o = np.zeros(Q.H, np.float32), np.zeros(Q.H, np.float32)
    assert oracle.lib.or_gdn_attn(pf(h1), L.ptr(), pf(L.ssm), pf(L.tail), pf(x2n), pf(x2o)) == 0
    xn = h1.astype(np.float64) / np.sqrt(np.mean(h1.astype(np.float64) ** 2) + 1e-6) * a["attn_norm"]
    av = xn @ a["alpha_wt"].astype(np.float64) + a["ssm_dt"]
    g = np.exp(np.logaddexp(0.0, av) * a["ssm_a"])
    S0 = S0.reshape(16, 128 * 128)
    S1 = L.ssm.reshape(16, 128 * 128)
    for h in range(16):
        np.testing.assert_allclose(S1[h], g[h] * S0[h], rtol=2e-5, atol=1e-9)
    # with q = k = v = 0 the output o is 0, so the layer adds ssm_out(0) = 0
    np.testing.assert_array_equal(x2o, h1)


def test_llama_attn_configs3_shape(oracle):
    """or_llama_attn_op at configs[3]'s attention shape (32 q / 4 kv heads of
    128, Q6_K, 480 cached rows + 4 steps), bitwise to the compiled reference."""
    g = golden("attn_cfg3.npz")
    cfg, model, krows, vrows, xs = gg.attn_cfg3_inputs()
    assert model.digest() == g["digest"].tobytes().hex()
    drv = LlamaDriver(model, oracle_engine(oracle))
    outs = gg.run_attn_steps(drv, oracle.lib.or_llama_attn_op, krows, vrows, xs, gg.ATTN_CFG3_T0)
    kd = cfg.n_kv * cfg.head_dim
    n = (gg.ATTN_CFG3_T0 + gg.ATTN_CFG3_STEPS) * kd
    assert bits_equal(outs, g["out"])
    assert bits_equal(drv.kc[0][gg.ATTN_CFG3_T0 * kd:n], g["knew"])
    assert bits_equal(drv.vc[0][gg.ATTN_CFG3_T0 * kd:n], g["vnew"])


def test_moe_stack_decode_tiny(oracle):
    """configs[3]'s layer (attention 32 q / 4 kv x 128 Q6_K + MoE FFN: 128
    experts, top 8, FFN 768) in two layers: token-serial prompt + greedy
    decode through the descriptor ABI with the MoE FFN as the layer's ffn op,
    bitwise to the compiled reference engine running its own m6_granite_moe."""
    g = golden("moe_tiny.npz")
    cfg = models.MOE_TINY
    model = models.build_llama(cfg, 0)
    assert model.digest() == g["digest"].tobytes().hex()
    drv = LlamaDriver(model, oracle_engine(oracle))
    toks, hidden, lg = drv.greedy(model.prompt(), cfg.n_gen, collect_logits=(0, 15))
    assert toks == list(g["tokens"])
    assert bits_equal(hidden, g["hidden"])
    assert bits_equal(lg[0], g["logits0"]) and bits_equal(lg[15], g["logits15"])


@pytest.mark.parametrize("name,fname,steps", [("qwen35-tiny", "qwen_tiny.npz", (0, 15)),
                                              ("qwen35-tiny-moe", "qwen_tiny_moe.npz", (0, 7))])
def test_qwen_stack_decode(oracle, name, fname, steps):
    """qwen35 hybrid stack (G G G F, dense or MoE FFN) decoded token by token
    the way src/qwen35_engine.py:310-327 composes the layer ops, against the
    compiled reference's ops: identical greedy tokens; hidden state and logits
    within 1e-5 (the reference's GDN post-norm sums squares in per-thread
    partials, so x2n differs in the last bits)."""
    from helpers import rel_err
    from dracohip import qwen35 as Q
    from tests_oracle_engine import oracle_qwen_ops
    g = golden(fname)
    cfg = Q.STACKS[name]
    stack = Q.build_stack(cfg, 0)
    assert list(stack.prompt()) == list(g["prompt"])
    drv = Q.QwenStackDriver(stack, oracle_qwen_ops(oracle))
    toks, hidden, lg = drv.greedy(stack.prompt(), cfg.n_gen, collect_logits=steps)
    assert toks == list(g["tokens"])
    assert rel_err(hidden, g["hidden"]) <= 1e-5
    for s in steps:
        assert rel_err(lg[s], g[f"logits{s}"]) <= 1e-5
