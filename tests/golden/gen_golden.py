"""Write the golden fixtures under tests/golden/ from the reference's own C.

Runs only where the reference tree exists and `make -C oracle ref` built
oracle/_ref/*.so (the reference's sources compiled in place).  Every output
array here is produced by the compiled reference (src/m5_kern_scalar.c,
src/m5/m5_batch8_k.c, src/m6_engine.c + m6_layer.c, src/m6_gdn_scan.c,
src/m6_moe_tok.c) on
seeded inputs; the inputs are regenerated deterministically by the tests
(weights via dracohip.models, vectors via numpy default_rng) or stored when
small.

usage: python tests/golden/gen_golden.py [--only NAME ...]
"""
import argparse
import ctypes as ct
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "dracomancer-llmengine_amd"))
sys.path.insert(0, ROOT)

from dracohip import lib as dlib  # noqa: E402
from dracohip import models  # noqa: E402
from dracohip.driver import EngineLib, LlamaDriver  # noqa: E402
from oracle.oracle import REF_DIR  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
f32p = ct.POINTER(ct.c_float)
u8p = ct.POINTER(ct.c_uint8)
i32p = ct.POINTER(ct.c_int)


def pf(a):
    return a.ctypes.data_as(f32p)


def pu8(a):
    return a.ctypes.data_as(u8p)


def ref(name):
    return ct.CDLL(os.path.join(REF_DIR, f"libref_{name}.so"))


# ---------------------------------------------------------------- inputs --
GEMV_CASES = [  # (name, code, n_out, n_in)
    ("q4k_48x512", 5, 48, 512), ("q4k_33x768", 5, 33, 768), ("q4k_5x2048", 5, 5, 2048),
    ("q6k_48x512", 4, 48, 512), ("q6k_33x768", 4, 33, 768), ("q6k_5x2048", 4, 5, 2048),
    ("q80_40x960", 0, 40, 960), ("q80_7x64", 0, 7, 64),
    ("q5k_16x512", 3, 16, 512), ("f16_10x96", 7, 10, 96), ("f32_10x96", 9, 10, 96),
]


def gemv_inputs(code, n_out, n_in, seed):
    """Seeded weight bytes + x.  Shared by the generator and the tests."""
    rng = np.random.default_rng(seed)
    if code in (0, 4, 5):
        W = dlib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
    elif code == 3:  # Q5_K: random qs/qh/scales with finite positive d, dmin
        nb = n_in // 256
        W = rng.integers(0, 256, n_out * nb * 176, dtype=np.uint8).reshape(-1, 176)
        d = (rng.random(W.shape[0]) * 1e-3 + 1e-4).astype(np.float16).view(np.uint8).reshape(-1, 2)
        dm = (rng.random(W.shape[0]) * 1e-3).astype(np.float16).view(np.uint8).reshape(-1, 2)
        W[:, 0:2] = d
        W[:, 2:4] = dm
        W = W.reshape(-1)
    elif code == 7:
        W = (rng.standard_normal(n_out * n_in) * 0.1).astype(np.float16).view(np.uint8)
    else:
        W = (rng.standard_normal(n_out * n_in) * 0.1).astype(np.float32).view(np.uint8)
    x = rng.standard_normal(n_in, dtype=np.float32)
    return np.ascontiguousarray(W), x


def gen_gemv():
    L = ref("scalar")
    L.m5_gemv.argtypes = [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, f32p]
    L.m5_gemv_range.argtypes = [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, f32p, ct.c_int, ct.c_int]
    L.m5_scalar_supported.argtypes = [ct.c_int]
    out = {}
    for i, (name, code, n_out, n_in) in enumerate(GEMV_CASES):
        W, x = gemv_inputs(code, n_out, n_in, 100 + i)
        y = np.zeros(n_out, np.float32)
        assert L.m5_gemv(code, pf(x), pu8(W), n_out, n_in, pf(y)) == 0
        yr = np.full(n_out, np.float32(-7.0))
        o0, o1 = n_out // 3, n_out - 1
        assert L.m5_gemv_range(code, pf(x), pu8(W), n_out, n_in, pf(yr), o0, o1) == 0
        onehot = np.zeros(n_in, np.float32)
        col = (n_in * 5) // 7
        onehot[col] = 1.0
        yc = np.zeros(n_out, np.float32)
        assert L.m5_gemv(code, pf(onehot), pu8(W), n_out, n_in, pf(yc)) == 0
        out[name + "_y"] = y
        out[name + "_yrange"] = yr
        out[name + "_meta"] = np.array([code, n_out, n_in, o0, o1, col], np.int64)
        out[name + "_col"] = yc
    out["supported"] = np.array([L.m5_scalar_supported(c) for c in range(12)], np.int32)
    # rms norm (src/m6_engine.c:31-37)
    E = ref("engine")
    E.m6_rms_norm.argtypes = [f32p, f32p, ct.c_int, ct.c_float, f32p]
    rng = np.random.default_rng(7)
    for h in (960, 2048):
        xx = rng.standard_normal(h, dtype=np.float32) * np.float32(3.0)
        ww = rng.standard_normal(h, dtype=np.float32)
        o = np.zeros(h, np.float32)
        E.m6_rms_norm(pf(xx), pf(ww), h, ct.c_float(1e-5), pf(o))
        out[f"rms{h}_x"], out[f"rms{h}_w"], out[f"rms{h}_y"] = xx, ww, o
    np.savez_compressed(os.path.join(OUT, "gemv.npz"), **out)
    print("gemv.npz", len(GEMV_CASES), "cases")


BATCH8K_CASES = [  # (tag, code, x_stride_kind)
    ("q4k_shared", 5, 0), ("q4k_perexp", 5, 1), ("q6k_shared", 4, 0), ("q6k_perexp", 4, 1),
]


def batch8k_inputs(code, perexp, seed):
    """Seeded inputs of m5_gemvn_q4k/q6k: 5 experts of 100x512, idx [3,0,4]."""
    rng = np.random.default_rng(seed)
    n_exp_all, n_out_e, n_in = 5, 100, 512
    W = dlib.quantize(code, rng.standard_normal((n_exp_all * n_out_e, n_in), dtype=np.float32)
                      * np.float32(0.02))
    idx = np.array([3, 0, 4], np.int32)
    xstride = n_in if perexp else 0
    x = rng.standard_normal((len(idx) if perexp else 1) * n_in, dtype=np.float32)
    return W, x, idx, W.nbytes // n_exp_all, n_out_e, n_in, xstride


def gen_batch8k():
    B = ref("batch8k")
    for fn in (B.m5_gemvn_q4k, B.m5_gemvn_q6k):
        fn.argtypes = [f32p, ct.c_long, u8p, i32p, ct.c_long, ct.c_int, ct.c_int, ct.c_int, f32p]
        fn.restype = ct.c_int
    out = {}
    for i, (tag, code, perexp) in enumerate(BATCH8K_CASES):
        W, x, idx, per, n_out_e, n_in, xstride = batch8k_inputs(code, perexp, 40 + i)
        fn = B.m5_gemvn_q4k if code == 5 else B.m5_gemvn_q6k
        y = np.zeros(len(idx) * n_out_e, np.float32)
        assert fn(pf(x), xstride, pu8(W), idx.ctypes.data_as(i32p), per, n_out_e, n_in, len(idx), pf(y)) == 0
        out[tag + "_y"] = y
    np.savez_compressed(os.path.join(OUT, "batch8k.npz"), **out)
    print("batch8k.npz")


def ref_engine():
    E = ref("engine")
    E.m6_init_dl.argtypes = [ct.c_char_p] * 5
    E.m6_init_dl.restype = ct.c_int
    sp = os.path.join(REF_DIR, "libref_scalar.so").encode()
    rc = E.m6_init_dl(sp, sp, sp, sp, sp)  # the reference's own scalar mode (src/m5sel.py:13-14)
    assert rc == 0, rc
    return E


_MOE_CALLBACKS = []  # keep the ctypes callbacks alive


def ref_engine_lib(E):
    """The compiled reference engine as an EngineLib.  Its MoE layers run the
    reference's own m6_granite_moe (src/m6_layer.c:771-802) through an ffn-op
    callback, as src/qwen35_engine.py:293-307 calls it per layer."""
    from dracohip.driver import DracoMoeP
    E.m6_granite_moe.argtypes = [f32p, ct.c_void_p, ct.c_void_p, f32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int,
                                 ct.c_int, f32p, f32p]
    E.m6_granite_moe.restype = None

    @ct.CFUNCTYPE(None, f32p, ct.c_void_p, f32p)
    def moe_op(xn, pv, out):
        p = ct.cast(pv, ct.POINTER(DracoMoeP)).contents
        E.m6_granite_moe(xn, p.ptrs, p.codes, p.gate_inp, p.n_exp, p.n_used, p.inter, p.n_in, p.n_out, p.scratch,
                         out)

    _MOE_CALLBACKS.append(moe_op)
    lib = EngineLib(E, name="ref", moe=None)
    lib.moe_ptr = ct.cast(moe_op, ct.c_void_p).value
    return lib


def gen_llama(cfg, fname, seed=0, logit_steps=(0,)):
    t0 = time.time()
    model = models.build_llama(cfg, seed)
    E = ref_engine_lib(ref_engine())
    drv = LlamaDriver(model, E)
    prompt = model.prompt()
    toks, hidden, lg = drv.greedy(prompt, cfg.n_gen, collect_logits=logit_steps)
    out = dict(tokens=np.array(toks, np.int32), hidden=hidden, prompt=prompt,
               digest=np.frombuffer(bytes.fromhex(model.digest()), np.uint8))
    for s, v in lg.items():
        # full logits only for small vocabularies; top-8 (ids + values) always
        top = np.argsort(-v.astype(np.float64), kind="stable")[:8]
        out[f"logits{s}_top_ids"] = top.astype(np.int32)
        out[f"logits{s}_top_vals"] = v[top]
        if cfg.vocab <= 4096:
            out[f"logits{s}"] = v
    np.savez_compressed(os.path.join(OUT, fname), **out)
    print(fname, cfg.name, f"{time.time() - t0:.1f}s", "tokens", toks[:8], "...")


def gen_moe():
    """m6_granite_moe (src/m6_layer.c:771-802) on a small and a cfg4-shaped layer."""
    E = ref_engine()
    E.m6_granite_moe.argtypes = [f32p, ct.c_void_p, i32p, f32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int,
                                 ct.c_int, f32p, f32p]
    out = {}
    for tag, n_exp, n_used, inter, n_in, seed in (("small", 16, 4, 256, 512, 21), ("cfg4", 128, 8, 768, 2048, 22)):
        rng = np.random.default_rng(seed)
        gate_inp = (rng.standard_normal((n_exp, n_in), dtype=np.float32) * np.float32(0.02))
        # expert bytes are regenerated by the test from the same seed stream
        Wg = dlib.quantize(5, rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02))
        Wu = dlib.quantize(5, rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02))
        Wd = dlib.quantize(4, rng.standard_normal((n_exp * n_in, inter), dtype=np.float32) * np.float32(0.02))
        x = rng.standard_normal(n_in, dtype=np.float32)
        pg, pu, pd = Wg.nbytes // n_exp, Wu.nbytes // n_exp, Wd.nbytes // n_exp
        ptrs = np.zeros(3 * n_exp, np.uint64)
        codes = np.zeros(3 * n_exp, np.int32)
        for e in range(n_exp):
            ptrs[3 * e] = Wg.ctypes.data + e * pg
            ptrs[3 * e + 1] = Wu.ctypes.data + e * pu
            ptrs[3 * e + 2] = Wd.ctypes.data + e * pd
            codes[3 * e:3 * e + 3] = (5, 5, 4)
        scratch = np.zeros(3 * n_used * inter + n_used * n_in + 64, np.float32)
        y = np.zeros(n_in, np.float32)
        E.m6_granite_moe(pf(x), ct.c_void_p(ptrs.ctypes.data), codes.ctypes.data_as(i32p), pf(gate_inp),
                         n_exp, n_used, inter, n_in, n_in, pf(scratch), pf(y))
        out[f"{tag}_y"] = y
        out[f"{tag}_meta"] = np.array([n_exp, n_used, inter, n_in, seed], np.int64)
        out[f"{tag}_digest"] = np.frombuffer(hashlib.sha256(Wg.tobytes() + Wu.tobytes() + Wd.tobytes()).digest(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "moe.npz"), **out)
    print("moe.npz")


MOE_BATCH4_CASES = [  # (tag, n experts, inter, n_in, n_out, codes (gate, up, down), seed)
    ("b8", 8, 256, 512, 512, (5, 5, 4), 61),
    ("b3q6", 3, 768, 2048, 2048, (4, 4, 5), 62),
    ("b20", 20, 256, 256, 256, (5, 5, 5), 63),
]


def moe_batch4_inputs(n, inter, n_in, n_out, codes, seed):
    """Expert bytes, their pointer / code tables, x and the (unnormalised)
    weights of one m6_moe_batch4 case, from one rng stream."""
    rng = np.random.default_rng(seed)
    Wg = dlib.quantize(codes[0], rng.standard_normal((n * inter, n_in), dtype=np.float32) * np.float32(0.02))
    Wu = dlib.quantize(codes[1], rng.standard_normal((n * inter, n_in), dtype=np.float32) * np.float32(0.02))
    Wd = dlib.quantize(codes[2], rng.standard_normal((n * n_out, inter), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(n_in, dtype=np.float32)
    wtop = (rng.random(n) * 0.5 + 0.05).astype(np.float32)
    pg, pu, pd = Wg.nbytes // n, Wu.nbytes // n, Wd.nbytes // n
    ptrs = np.zeros(3 * n, np.uint64)
    cds = np.zeros(3 * n, np.int32)
    for e in range(n):
        ptrs[3 * e:3 * e + 3] = (Wg.ctypes.data + e * pg, Wu.ctypes.data + e * pu, Wd.ctypes.data + e * pd)
        cds[3 * e:3 * e + 3] = codes
    return dict(Wg=Wg, Wu=Wu, Wd=Wd, x=x, wtop=wtop, ptrs=ptrs, codes=cds)


def gen_moe_batch4():
    """m6_moe_batch4 (src/m6_layer.c:656-690): given experts and weights."""
    E = ref_engine()
    # the C signature (src/m6_layer.c:656-658): 4 pointers, 4 ints, 2 pointers
    E.m6_moe_batch4.argtypes = [ct.c_void_p] * 4 + [ct.c_int] * 4 + [ct.c_void_p] * 2
    E.m6_moe_batch4.restype = None
    out = {}
    for tag, n, inter, n_in, n_out, codes, seed in MOE_BATCH4_CASES:
        M = moe_batch4_inputs(n, inter, n_in, n_out, codes, seed)
        scratch = np.zeros(3 * n * inter + n * n_out + 64, np.float32)
        y = np.full(n_out, np.nan, np.float32)
        E.m6_moe_batch4(M["x"].ctypes.data, M["ptrs"].ctypes.data, M["codes"].ctypes.data, M["wtop"].ctypes.data,
                        n, inter, n_in, n_out, scratch.ctypes.data, y.ctypes.data)
        out[f"{tag}_y"] = y
        out[f"{tag}_digest"] = np.frombuffer(hashlib.sha256(M["Wg"].tobytes() + M["Wu"].tobytes() +
                                                            M["Wd"].tobytes()).digest(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "moe_batch4.npz"), **out)
    print("moe_batch4.npz")


SHEXP_CASES = [  # (tag, shi, h, codes {gate, up, down, gate_inp}, seed)
    ("small", 256, 512, (5, 5, 4, 9), 51),
    ("q35", 512, 2048, (5, 5, 4, 9), 52),
    ("mixed", 128, 256, (5, 0, 0, 7), 53),
    ("q8gate", 256, 512, (0, 5, 4, 0), 54),
]


def shexp_inputs(shi, h, codes, seed):
    """Shared-expert weights {gate, up, down, gate_inp} encoded in `codes`
    (F32 / F16 rows as raw little-endian values) and x, from one rng stream."""
    rng = np.random.default_rng(seed)

    def enc(code, w):
        if code == 9:
            return np.ascontiguousarray(w, np.float32).view(np.uint8).ravel()
        if code == 7:
            return np.ascontiguousarray(w.astype(np.float16)).view(np.uint8).ravel()
        return dlib.quantize(code, w)
    shapes = [(shi, h), (shi, h), (h, shi), (1, h)]
    ws = [enc(c, rng.standard_normal(s, dtype=np.float32) * np.float32(0.02)) for c, s in zip(codes, shapes)]
    x = rng.standard_normal(h, dtype=np.float32)
    ptrs = np.array([w.ctypes.data for w in ws], np.uint64)
    return ws, x, ptrs, np.array(codes, np.int32)


def gen_shexp():
    """m6_granite_shexp (src/m6_engine.c:1111-1127) at three shapes / format mixes."""
    E = ref_engine()
    E.m6_granite_shexp.argtypes = [f32p, ct.c_void_p, i32p, f32p, f32p, f32p, f32p, ct.c_int, ct.c_int]
    E.m6_granite_shexp.restype = None
    out = {}
    for tag, shi, h, codes, seed in SHEXP_CASES:
        ws, x, ptrs, cds = shexp_inputs(shi, h, codes, seed)
        sg = np.zeros(1, np.float32)
        sh = np.zeros(2 * shi, np.float32)
        shg = np.zeros(h, np.float32)
        y = np.zeros(h, np.float32)
        E.m6_granite_shexp(pf(x), ct.c_void_p(ptrs.ctypes.data), cds.ctypes.data_as(i32p), pf(sg), pf(sh), pf(shg),
                           pf(y), shi, h)
        out[f"{tag}_out"] = y
        out[f"{tag}_shg"] = shg
        out[f"{tag}_sg"] = sg
        out[f"{tag}_act"] = sh[:shi].copy()
        out[f"{tag}_digest"] = np.frombuffer(hashlib.sha256(b"".join(w.tobytes() for w in ws)).digest(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "shexp.npz"), **out)
    print("shexp.npz")


def gdn_inputs(T, n_vh, nhq, seed):
    rng = np.random.default_rng(seed)
    n_qkv = n_vh * 128 + 2 * nhq * 128
    QKV = rng.standard_normal((T, n_qkv), dtype=np.float32)
    Z = rng.standard_normal((T, n_vh * 128), dtype=np.float32)
    B = (1.0 / (1.0 + np.exp(-rng.standard_normal((T, n_vh))))).astype(np.float32)
    G = np.exp(-np.logaddexp(0.0, rng.standard_normal((T, n_vh)))).astype(np.float32)
    conv = (rng.standard_normal((n_qkv, 4), dtype=np.float32) * np.float32(0.5))
    ssm_norm = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    tail = rng.standard_normal(n_qkv * 3, dtype=np.float32)
    S = (rng.standard_normal(n_vh * 128 * 128, dtype=np.float32) * np.float32(0.05))
    return n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S


def gen_gdn():
    L = ref("gdnscan")
    L.m6_gdn_scan.argtypes = [f32p] * 8 + [ct.c_int] * 3 + [f32p, f32p]
    out = {}
    for tag, T, n_vh, nhq, seed in (("a", 6, 2, 1, 31), ("b", 5, 4, 2, 32)):
        n_qkv, QKV, Z, B, G, conv, ssm_norm, tail, S = gdn_inputs(T, n_vh, nhq, seed)
        ON = np.zeros((T, n_vh * 128), np.float32)
        work = np.zeros(n_qkv, np.float32)
        L.m6_gdn_scan(pf(QKV), pf(Z), pf(B), pf(G), pf(conv), pf(ssm_norm), pf(tail), pf(S),
                      T, n_qkv, n_vh, pf(ON), pf(work))
        out[f"{tag}_ON"] = ON
        out[f"{tag}_S_sha"] = np.frombuffer(hashlib.sha256(S.tobytes()).digest(), np.uint8)
        out[f"{tag}_tail_sha"] = np.frombuffer(hashlib.sha256(tail.tobytes()).digest(), np.uint8)
        out[f"{tag}_S_sample"] = S[::997].copy()
        out[f"{tag}_meta"] = np.array([T, n_vh, nhq, seed], np.int64)
    np.savez_compressed(os.path.join(OUT, "gdn.npz"), **out)
    print("gdn.npz")


MOETOK_CASES = [  # (tag, n_exp, n_used, inter, n_in (= n_out), T, codes {gate, up, down}, seed)
    ("small", 16, 4, 256, 512, 20, (5, 5, 4), 81),
    ("cfg3", 128, 8, 768, 2048, 24, (5, 5, 5), 82),
    ("q6mix", 32, 6, 512, 1024, 12, (4, 5, 4), 83),
]


def moetok_inputs(n_exp, n_used, inter, n_in, T, codes, seed):
    """Seeded expert weights (3 per expert), token rows X[T][n_in] and routing
    (distinct experts per token from the lower half of the experts, so some
    experts get no token; weights normalised per token; slot 1 of token 3 holds
    the invalid id -1, which both sides skip)."""
    rng = np.random.default_rng(seed)
    mats = [dlib.quantize(codes[0], rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02)),
            dlib.quantize(codes[1], rng.standard_normal((n_exp * inter, n_in), dtype=np.float32) * np.float32(0.02)),
            dlib.quantize(codes[2], rng.standard_normal((n_exp * n_in, inter), dtype=np.float32) * np.float32(0.02))]
    ptrs = np.zeros(3 * n_exp, np.uint64)
    ec = np.zeros(3 * n_exp, np.int32)
    for e in range(n_exp):
        for k in range(3):
            ptrs[3 * e + k] = mats[k].ctypes.data + e * (mats[k].nbytes // n_exp)
            ec[3 * e + k] = codes[k]
    X = rng.standard_normal((T, n_in)).astype(np.float32)
    order = np.stack([rng.choice(n_exp // 2, n_used, replace=False) for _ in range(T)]).astype(np.int32)
    order[3, 1] = -1
    wtop = rng.random((T, n_used)).astype(np.float32)
    wtop /= wtop.sum(axis=1, keepdims=True)
    return mats, ptrs, ec, X, np.ascontiguousarray(order), np.ascontiguousarray(wtop)


def gen_moetok():
    """m6_moe_tok (src/m6_moe_tok.c:44-161) compiled from the reference, driven
    with GA = NULL (its row-dequantize + dot path) and DQ = the oracle's row
    decoder (the reference's own m5_dequant_row lives in src/m5/m5_gemm.c,
    which cannot be built here); the decoder is pinned bit for bit by
    tests/test_oracle_pins.py."""
    from oracle.oracle import Oracle
    orc = Oracle()
    M = ref("moetok")
    M.m6_moe_tok.restype = None
    M.m6_moe_tok.argtypes = [ct.c_void_p] * 8 + [ct.c_int] * 6 + [ct.c_void_p] * 3
    dq = ct.cast(orc.lib.or_dequant_row, ct.c_void_p)
    nth = 2 * (os.cpu_count() or 8)
    out = {}
    for tag, n_exp, n_used, inter, n_in, T, codes, seed in MOETOK_CASES:
        mats, ptrs, ec, X, order, wtop = moetok_inputs(n_exp, n_used, inter, n_in, T, codes, seed)
        y = np.zeros((T, n_in), np.float32)
        gwbuf = np.zeros(nth * ((max(n_in, inter) + 15) & ~15), np.float32)
        work = np.zeros(T * n_used * (n_in + 3 * inter + n_in), np.float32)
        iwork = np.zeros(T * n_used * 2 + n_exp + 1, np.int32)
        M.m6_moe_tok(dq, None, gwbuf.ctypes.data, X.ctypes.data, order.ctypes.data, wtop.ctypes.data,
                     ptrs.ctypes.data, ec.ctypes.data, T, n_used, inter, n_in, n_in, n_exp,
                     y.ctypes.data, work.ctypes.data, iwork.ctypes.data)
        out[f"{tag}_y"] = y
        out[f"{tag}_digest"] = np.frombuffer(hashlib.sha256(b"".join(m.tobytes() for m in mats)).digest(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "moetok.npz"), **out)
    print("moetok.npz")


ATTN_CFG3_T0 = 480      # cached rows before the first step
ATTN_CFG3_STEPS = 4


def attn_cfg3_inputs():
    """configs[3]'s attention (ATTN_CFG3, one layer): the layer's weights, a
    cache holding ATTN_CFG3_T0 seeded rows and the normalised inputs of
    ATTN_CFG3_STEPS tokens."""
    cfg = models.ATTN_CFG3
    model = models.build_llama(cfg, 7)
    rng = np.random.default_rng(77)
    kd = cfg.n_kv * cfg.head_dim
    krows = rng.standard_normal((ATTN_CFG3_T0, kd), dtype=np.float32)
    vrows = rng.standard_normal((ATTN_CFG3_T0, kd), dtype=np.float32)
    xs = rng.standard_normal((ATTN_CFG3_STEPS, cfg.hidden), dtype=np.float32)
    return cfg, model, krows, vrows, xs


def run_attn_steps(drv, attn_fn, krows, vrows, xs, pos0):
    """Drive one layer's attention op token by token from a pre-filled cache;
    returns the outputs [steps][hidden] and the appended K/V rows."""
    t0 = krows.shape[0]
    drv.kc[0][:krows.size] = krows.reshape(-1)
    drv.vc[0][:vrows.size] = vrows.reshape(-1)
    drv.tl[0][0] = t0
    outs = np.zeros((xs.shape[0], drv.H), np.float32)
    for s in range(xs.shape[0]):
        attn_fn(pf(np.ascontiguousarray(xs[s])), drv.descs[0].attn_p, pos0 + s, pf(outs[s]))
    return outs


def gen_attn_cfg3():
    """m6_llama_attn_op (src/m6_engine.c:425-517) at configs[3]'s attention
    shape: 32 q / 4 kv heads of 128 (GQA 8), Q6_K projections, 480 cached rows
    + 4 steps."""
    E = ref_engine()
    E.m6_llama_attn_op.argtypes = [f32p, ct.c_void_p, ct.c_int, f32p]
    E.m6_llama_attn_op.restype = None
    cfg, model, krows, vrows, xs = attn_cfg3_inputs()
    drv = LlamaDriver(model, EngineLib(E, name="ref"))
    outs = run_attn_steps(drv, E.m6_llama_attn_op, krows, vrows, xs, ATTN_CFG3_T0)
    kd = cfg.n_kv * cfg.head_dim
    n = (ATTN_CFG3_T0 + ATTN_CFG3_STEPS) * kd
    np.savez_compressed(os.path.join(OUT, "attn_cfg3.npz"), out=outs,
                        knew=drv.kc[0][ATTN_CFG3_T0 * kd:n].copy(), vnew=drv.vc[0][ATTN_CFG3_T0 * kd:n].copy(),
                        digest=np.frombuffer(bytes.fromhex(model.digest()), np.uint8))
    print("attn_cfg3.npz")


# qwen35 layer ops: (tag, n_vh, codes, seed) and (tag, nh, codes, seed, [(told, pos0), ...])
QWEN_GDN_CASES = [("cfg5", 32, (5, 5, 5), 51), ("q80", 16, (0, 0, 0), 52), ("mixed", 16, (5, 4, 4), 53)]
QWEN_FULL_CASES = [("cfg5", 16, (5, 5, 4, 5), 61, [(0, 0), (7, 7), (300, 300), (40, 45)]),
                   ("q80", 8, (0, 0, 0, 0), 62, [(0, 0), (33, 33)])]
GDN_STEPS = 3


def gen_qwen35():
    """m6_gdn_attn (src/m6_layer.c:205-364) over GDN_STEPS consecutive tokens
    and m6_full_attn (src/m6_layer.c:389-518) at several cache lengths."""
    from dracohip import qwen35 as Q
    E = ref_engine()
    E.m6_gdn_attn.argtypes = [f32p, ct.c_void_p, f32p, f32p, f32p, f32p, f32p]
    E.m6_full_attn.argtypes = [f32p, ct.c_void_p, f32p, f32p, ct.c_int, ct.c_int, f32p, f32p, f32p, f32p,
                               f32p, f32p]
    out = {}
    for tag, n_vh, codes, seed in QWEN_GDN_CASES:
        L = Q.gdn_layer(seed, n_vh, codes)
        ssm, tail = L.fresh_state()
        h1 = Q.hidden(seed + 1000, GDN_STEPS)
        buf = np.zeros(40000, np.float32)  # the reference's scratch (>= 28672, buf[39000] = 0)
        for s in range(GDN_STEPS):
            x2n = np.zeros(Q.H, np.float32)
            x2o = np.zeros(Q.H, np.float32)
            E.m6_gdn_attn(pf(h1[s]), L.ptr(), pf(ssm), pf(tail), pf(buf), pf(x2n), pf(x2o))
            out[f"gdn_{tag}_x2n_{s}"] = x2n
            out[f"gdn_{tag}_x2o_{s}"] = x2o
        out[f"gdn_{tag}_ssm_sample"] = ssm[::61].copy()
        out[f"gdn_{tag}_ssm_sha"] = np.frombuffer(hashlib.sha256(ssm.tobytes()).digest(), np.uint8)
        out[f"gdn_{tag}_tail"] = tail.copy()
        out[f"gdn_{tag}_meta"] = np.array([n_vh, *codes, seed, GDN_STEPS], np.int64)
    for tag, nh, codes, seed, steps in QWEN_FULL_CASES:
        L = Q.full_layer(seed, nh, codes)
        for told, pos0 in steps:
            Kr, Vc = Q.kv_rows(seed + told, told)
            h1 = Q.hidden(seed + 2000 + told)[0]
            buf = np.zeros(40000, np.float32)
            scores = np.zeros(nh * (told + 1), np.float32)
            x2n, x2o = np.zeros(Q.H, np.float32), np.zeros(Q.H, np.float32)
            krn, vrn = np.zeros(512, np.float32), np.zeros(512, np.float32)
            E.m6_full_attn(pf(h1), L.ptr(), pf(Kr), pf(Vc), told, pos0, pf(buf), pf(scores), pf(x2n), pf(x2o),
                           pf(krn), pf(vrn))
            k = f"full_{tag}_{told}_{pos0}"
            out[k + "_x2n"], out[k + "_x2o"], out[k + "_krn"], out[k + "_vrn"] = x2n, x2o, krn, vrn
        out[f"full_{tag}_meta"] = np.array([nh, *codes, seed], np.int64)
    np.savez_compressed(os.path.join(OUT, "qwen35.npz"), **out)
    print("qwen35.npz")


def ref_qwen_ops(E, max_t):
    """The compiled reference's qwen35 per-layer ops (src/m6_layer.c:205-518,
    src/m6_engine.c:275-303 and :373-391, m6_granite_moe through the MoE
    callback) as a QwenStackDriver op table, with the host scratch they need
    (buf >= 40000 floats with buf[39000] = 0, scores [nh][max_t])."""
    from dracohip import qwen35 as Q
    E.m6_gdn_attn.argtypes = [f32p, ct.c_void_p, f32p, f32p, f32p, f32p, f32p]
    E.m6_gdn_attn.restype = None
    E.m6_full_attn.argtypes = [f32p, ct.c_void_p, f32p, f32p, ct.c_int, ct.c_int, f32p, f32p, f32p, f32p, f32p, f32p]
    E.m6_full_attn.restype = None
    E.m6_dense_op.argtypes = [f32p, ct.c_void_p, f32p]
    E.m6_dense_op.restype = None
    lib = ref_engine_lib(E)
    buf = np.zeros(40000, np.float32)
    scores = np.zeros(32 * max_t, np.float32)
    moe = ct.cast(lib.moe_ptr, ct.CFUNCTYPE(None, f32p, ct.c_void_p, f32p))
    return {"gdn": lambda h1, w, ssm, tail, x2n, x2o: E.m6_gdn_attn(h1, w, ssm, tail, pf(buf), x2n, x2o),
            "full": lambda h1, w, Kr, Vc, told, pos0, x2n, x2o, krn, vrn:
                E.m6_full_attn(h1, w, Kr, Vc, told, pos0, pf(buf), pf(scores), x2n, x2o, krn, vrn),
            "dense": E.m6_dense_op, "moe": moe, "head": lib.head_op, "_keep": (buf, scores, lib)}


def gen_qwen_stack(name, fname, logit_steps, record=()):
    """A qwen35 stack (dracohip.qwen35 STACKS[name]) decoded token by token
    through the compiled reference's per-layer ops exactly as
    src/qwen35_engine.py:310-327 composes them (the caller appends KRN / VRN
    to its caches), then greedy tokens.  `record`: layers after which the
    last token's hidden state is kept (depth{il})."""
    from dracohip import qwen35 as Q
    t0 = time.time()
    cfg = Q.STACKS[name]
    stack = Q.build_stack(cfg, 0)
    ops = ref_qwen_ops(ref_engine(), cfg.max_t)
    drv = Q.QwenStackDriver(stack, ops)
    drv.record = tuple(record)
    toks, hidden, lg = drv.greedy(stack.prompt(), cfg.n_gen, collect_logits=logit_steps)
    out = dict(tokens=np.array(toks, np.int32), hidden=hidden, prompt=stack.prompt())
    for il, v in drv.depth.items():
        out[f"depth{il}"] = v
    for s, v in lg.items():
        if cfg.vocab <= 4096:
            out[f"logits{s}"] = v
        top = np.argsort(-v.astype(np.float64), kind="stable")[:8]
        out[f"logits{s}_top_ids"] = top.astype(np.int32)
        out[f"logits{s}_top_vals"] = v[top]
    np.savez_compressed(os.path.join(OUT, fname), **out)
    print(fname, name, f"{time.time() - t0:.1f}s", "tokens", toks[:8], "...")


JOBS = {
    "gemv": gen_gemv,
    "batch8k": gen_batch8k,
    "moe": gen_moe,
    "moe_batch4": gen_moe_batch4,
    "tiny_q5": lambda: gen_llama(models.TINY_Q5, "llama_tiny_q5.npz", logit_steps=(0, 15)),
    "moetok": gen_moetok,
    "attn_cfg3": gen_attn_cfg3,
    "shexp": gen_shexp,
    "gdn": gen_gdn,
    "qwen35": gen_qwen35,
    "tiny_k": lambda: gen_llama(models.TINY_K, "llama_tiny_k.npz", logit_steps=(0, 15)),
    "tiny_q8": lambda: gen_llama(models.TINY_Q8, "llama_tiny_q8.npz", logit_steps=(0, 15)),
    "smol360m": lambda: gen_llama(models.SMOL360M, "smol360m.npz", logit_steps=(0, 63)),
    "llama1b": lambda: gen_llama(models.LLAMA1B, "llama1b.npz", logit_steps=(0, 63)),
    "moe_tiny": lambda: gen_llama(models.MOE_TINY, "moe_tiny.npz", logit_steps=(0, 15)),
    "qwen_tiny": lambda: gen_qwen_stack("qwen35-tiny", "qwen_tiny.npz", logit_steps=(0, 15)),
    "qwen_tiny_moe": lambda: gen_qwen_stack("qwen35-tiny-moe", "qwen_tiny_moe.npz", logit_steps=(0, 7)),
    "qwen48": lambda: gen_qwen_stack("qwen35-gdn-stack-48-short", "qwen48_short.npz", logit_steps=(0, 7),
                                     record=range(3, 48, 4)),
    "moe8": lambda: gen_llama(models.QWEN3_MOE8, "moe_stack8.npz", seed=3, logit_steps=(0, 7)),
}

if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", nargs="*", default=[k for k in JOBS if k != "llama1b"])
    a = ap.parse_args()
    for k in a.only:
        JOBS[k]()
    with open(os.path.join(OUT, "README.json"), "w") as f:
        json.dump({k: "generated by gen_golden.py from oracle/_ref (the reference's C compiled in place)"
                   for k in JOBS}, f, indent=1)
