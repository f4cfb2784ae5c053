"""qwen35 (Qwen3.5 / Qwen3-Next hybrid) layer descriptors and seeded layers.

GdnW and FullW are field-for-field the reference's ctypes structs
(src/qwen35_engine.py:137-157, C side src/m6_layer.c:189-202 and :375-387):
the same descriptor drives the reference's m6_gdn_attn / m6_full_attn, the
oracle's restatement and this library's device path.

Seeded layers (the reference defines no synthetic qwen35 layer; fixed here):
  * one np.random.default_rng(seed) per layer, tensors drawn in field order;
  * projection matrices N(0, 0.02) encoded by draco_quantize;
  * norm weights 1 + 0.1 N(0, 1); conv taps 0.5 N(0, 1);
  * beta / alpha projections N(0, 0.02) stored [2048][n_vh] (the reference's
    pre-transposed layout, src/qwen35_engine.py:190-199); dt 0.3 N(0, 1);
    ssm_a = -exp(0.3 N(0, 1)), so the decay exp(softplus(.) * a) lies in (0, 1);
  * initial recurrent state 0.05 N(0, 1), conv tail N(0, 1);
  * full attention: rope_inv[t] = 1e7^(-2t/64) (float64, then float32, as
    src/qwen35_engine.py:172), cached K / V rows N(0, 1).
"""
import ctypes as ct
from dataclasses import dataclass, field

import numpy as np

from . import lib as _lib

Q8_0, Q6_K, Q4_K = 0, 4, 5
H = 2048      # hidden width fixed by the reference ops (src/m6_layer.c:11-13)
NKH = 16      # q/k heads of the GDN layer
SV = 128      # GDN head width
HD_A = 256    # full-attention head dim
NKV_A = 2     # full-attention KV heads

f32p = ct.POINTER(ct.c_float)


class GdnW(ct.Structure):
    _fields_ = [("attn_norm", f32p),
                ("qkv_buf", ct.c_void_p), ("qkv_code", ct.c_int),
                ("gate_buf", ct.c_void_p), ("gate_code", ct.c_int),
                ("beta_wt", f32p), ("alpha_wt", f32p),
                ("ssm_a", f32p), ("ssm_dt", f32p),
                ("conv", f32p), ("ssm_norm", f32p),
                ("ssm_out_buf", ct.c_void_p), ("ssm_out_code", ct.c_int),
                ("post_norm", f32p),
                ("n_qkv", ct.c_int), ("n_vh", ct.c_int), ("d_in", ct.c_int)]


class FullW(ct.Structure):
    _fields_ = [("attn_norm", f32p),
                ("q_buf", ct.c_void_p), ("q_code", ct.c_int),
                ("k_buf", ct.c_void_p), ("k_code", ct.c_int),
                ("v_buf", ct.c_void_p), ("v_code", ct.c_int),
                ("q_norm", f32p), ("k_norm", f32p),
                ("o_buf", ct.c_void_p), ("o_code", ct.c_int),
                ("post_norm", f32p), ("rope_inv", f32p),
                ("nh", ct.c_int)]


def _pf(a):
    return a.ctypes.data_as(f32p)


def _norm(rng, n):
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def _mat(rng, code, n_out, n_in, wscale=0.02):
    return _lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(wscale))


@dataclass
class GdnLayer:
    n_vh: int
    codes: tuple
    arrays: dict = field(default_factory=dict)
    w: GdnW = None
    ssm: np.ndarray = None
    tail: np.ndarray = None

    @property
    def n_qkv(self):
        return 2 * NKH * SV + self.n_vh * SV

    def ptr(self):
        return ct.cast(ct.pointer(self.w), ct.c_void_p)

    def fresh_state(self):
        """Copies of the initial state (ssm, tail)."""
        return self.arrays["ssm0"].copy(), self.arrays["tail0"].copy()


def gdn_layer(seed, n_vh=32, codes=(Q4_K, Q4_K, Q4_K)):
    """codes = (qkv, gate, ssm_out)."""
    rng = np.random.default_rng(seed)
    n_qkv = 2 * NKH * SV + n_vh * SV
    a = {}
    a["attn_norm"] = _norm(rng, H)
    a["qkv"] = _mat(rng, codes[0], n_qkv, H)
    a["gate"] = _mat(rng, codes[1], n_vh * SV, H)
    a["beta_wt"] = rng.standard_normal((H, n_vh), dtype=np.float32) * np.float32(0.02)
    a["alpha_wt"] = rng.standard_normal((H, n_vh), dtype=np.float32) * np.float32(0.02)
    a["ssm_a"] = (-np.exp(0.3 * rng.standard_normal(n_vh))).astype(np.float32)
    a["ssm_dt"] = (0.3 * rng.standard_normal(n_vh)).astype(np.float32)
    a["conv"] = rng.standard_normal((n_qkv, 4), dtype=np.float32) * np.float32(0.5)
    a["ssm_norm"] = _norm(rng, SV)
    a["ssm_out"] = _mat(rng, codes[2], H, n_vh * SV)
    a["post_norm"] = _norm(rng, H)
    a["ssm0"] = rng.standard_normal(n_vh * SV * SV, dtype=np.float32) * np.float32(0.05)
    a["tail0"] = rng.standard_normal(n_qkv * 3, dtype=np.float32)
    w = GdnW()
    w.attn_norm = _pf(a["attn_norm"])
    w.qkv_buf, w.qkv_code = a["qkv"].ctypes.data, codes[0]
    w.gate_buf, w.gate_code = a["gate"].ctypes.data, codes[1]
    w.beta_wt, w.alpha_wt = _pf(a["beta_wt"]), _pf(a["alpha_wt"])
    w.ssm_a, w.ssm_dt = _pf(a["ssm_a"]), _pf(a["ssm_dt"])
    w.conv, w.ssm_norm = _pf(a["conv"]), _pf(a["ssm_norm"])
    w.ssm_out_buf, w.ssm_out_code = a["ssm_out"].ctypes.data, codes[2]
    w.post_norm = _pf(a["post_norm"])
    w.n_qkv, w.n_vh, w.d_in = n_qkv, n_vh, n_vh * SV
    L = GdnLayer(n_vh=n_vh, codes=tuple(codes), arrays=a, w=w)
    L.ssm, L.tail = L.fresh_state()
    return L


@dataclass
class FullLayer:
    nh: int
    codes: tuple
    arrays: dict = field(default_factory=dict)
    w: FullW = None

    def ptr(self):
        return ct.cast(ct.pointer(self.w), ct.c_void_p)


def rope_inv(base=1e7, rot=64):
    return np.array([base ** (-2.0 * t / rot) for t in range(rot // 2)], np.float32)


def full_layer(seed, nh=16, codes=(Q4_K, Q4_K, Q6_K, Q4_K)):
    """codes = (q+gate, k, v, o)."""
    rng = np.random.default_rng(seed)
    a = {}
    a["attn_norm"] = _norm(rng, H)
    a["q"] = _mat(rng, codes[0], nh * 2 * HD_A, H)
    a["k"] = _mat(rng, codes[1], NKV_A * HD_A, H)
    a["v"] = _mat(rng, codes[2], NKV_A * HD_A, H)
    a["q_norm"] = _norm(rng, HD_A)
    a["k_norm"] = _norm(rng, HD_A)
    a["o"] = _mat(rng, codes[3], H, nh * HD_A)
    a["post_norm"] = _norm(rng, H)
    a["rope_inv"] = rope_inv()
    w = FullW()
    w.attn_norm = _pf(a["attn_norm"])
    w.q_buf, w.q_code = a["q"].ctypes.data, codes[0]
    w.k_buf, w.k_code = a["k"].ctypes.data, codes[1]
    w.v_buf, w.v_code = a["v"].ctypes.data, codes[2]
    w.q_norm, w.k_norm = _pf(a["q_norm"]), _pf(a["k_norm"])
    w.o_buf, w.o_code = a["o"].ctypes.data, codes[3]
    w.post_norm, w.rope_inv = _pf(a["post_norm"]), _pf(a["rope_inv"])
    w.nh = nh
    return FullLayer(nh=nh, codes=tuple(codes), arrays=a, w=w)


def kv_rows(seed, told):
    """Seeded cached K / V rows [told][2*256] for full-attention tests."""
    rng = np.random.default_rng(seed)
    Kr = rng.standard_normal((max(told, 1), NKV_A * HD_A), dtype=np.float32)
    Vc = rng.standard_normal((max(told, 1), NKV_A * HD_A), dtype=np.float32)
    return Kr, Vc


def hidden(seed, n=1):
    return np.random.default_rng(seed).standard_normal((n, H), dtype=np.float32)


# ------------------------------------------------------------ the stack --
# A qwen35 hybrid stack as the reference's driver runs it (src/qwen35_engine.py:
# 159-327): per layer a GDN or full-attention op, then the FFN of x2n added
# to x2_out; the token embedding and the head (m6_head_op) around them.
# Layer il is full attention when (il + 1) % interval == 0 (3:1 GDN:full at
# interval 4).  Each layer is the seeded layer above (seed + il); its state
# starts from zero (the reference's reset, src/qwen35_engine.py:335-337).

FFN_NONE, FFN_DENSE, FFN_MOE = 0, 1, 2


class DracoQwenLayer(ct.Structure):
    """include/draco_hip.h DracoQwenLayer."""
    _fields_ = [("kind", ct.c_int), ("w", ct.c_void_p), ("state0", f32p), ("state1", f32p), ("max_t", ct.c_int),
                ("ffn_kind", ct.c_int), ("ffn", ct.c_void_p)]


@dataclass
class QwenStackConfig:
    name: str
    n_layer: int
    vocab: int
    interval: int = 4
    n_vh: int = 32
    nh: int = 16
    gdn_codes: tuple = (Q4_K, Q4_K, Q4_K)       # qkv, gate, ssm_out
    full_codes: tuple = (Q4_K, Q4_K, Q4_K, Q4_K)  # q+gate, k, v, o
    emb_code: int = Q4_K
    out_code: int = Q6_K
    eps: float = 1e-6
    max_t: int = 64
    n_prompt: int = 20
    n_gen: int = 16
    ffn: int = FFN_NONE
    n_ff: int = 0                                 # dense FFN rows
    ffn_codes: tuple = (Q4_K, Q4_K, Q6_K)        # dense gate, up, down
    n_exp: int = 0
    n_used: int = 0
    exp_ff: int = 0


# configs[4] of BASELINE.json: 48 layers at 3:1 GDN:full attention, GDN of 16
# q/k and 32 V heads of 128, full attention of 16 q heads and 2 KV heads of
# 256, Q4_K projections, hidden 2048; 4096-token prompt in 64-token chunks,
# then 64 decode steps.  The configuration names no FFN (the stack is the
# mixers) and no vocabulary (Qwen3-Next's 151936, untied Q6_K head).
QWEN35_GDN48 = QwenStackConfig(name="qwen35-gdn-stack-48", n_layer=48, vocab=151936, max_t=4096 + 64,
                               n_prompt=4096, n_gen=64)

# four layers (G G G F) with a dense FFN: the parity cases of the stack
QWEN35_TINY = QwenStackConfig(name="qwen35-tiny", n_layer=4, vocab=1024, max_t=64, n_prompt=20, n_gen=16,
                              ffn=FFN_DENSE, n_ff=512)
QWEN35_TINY_MOE = QwenStackConfig(name="qwen35-tiny-moe", n_layer=4, vocab=1024, max_t=64, n_prompt=12, n_gen=8,
                                  ffn=FFN_MOE, n_exp=32, n_used=4, exp_ff=512)

# the same 48 layers (the same weights: seed 0) with a short prompt: the
# full-depth parity case against the compiled reference
QWEN35_GDN48_SHORT = QwenStackConfig(name="qwen35-gdn-stack-48-short", n_layer=48, vocab=151936, max_t=64,
                                     n_prompt=8, n_gen=8)

STACKS = {c.name: c for c in (QWEN35_GDN48, QWEN35_TINY, QWEN35_TINY_MOE, QWEN35_GDN48_SHORT)}


@dataclass
class QwenStack:
    cfg: QwenStackConfig
    seed: int
    layers: list = field(default_factory=list)   # GdnLayer / FullLayer
    ffn: list = field(default_factory=list)      # per layer: dict of FFN arrays (or None)
    emb: np.ndarray = None
    head: np.ndarray = None
    onorm: np.ndarray = None

    def is_full(self, il):
        return (il + 1) % self.cfg.interval == 0

    def prompt(self, n=None):
        n = self.cfg.n_prompt if n is None else n
        return np.random.default_rng(self.seed + 1000).integers(0, self.cfg.vocab, n).astype(np.int32)

    def nbytes(self):
        tot = self.emb.nbytes + self.head.nbytes
        for L in self.layers:
            tot += sum(v.nbytes for k, v in L.arrays.items() if k not in ("ssm0", "tail0"))
        for f in self.ffn:
            if f:
                tot += sum(v.nbytes for v in f.values() if isinstance(v, np.ndarray))
        return tot


def build_stack(cfg, seed=0):
    from . import models as _models
    s = QwenStack(cfg=cfg, seed=seed)
    rng = np.random.default_rng(seed)
    s.emb = _models._tensor(rng, cfg.emb_code, cfg.vocab, H)
    s.head = _models._tensor(rng, cfg.out_code, cfg.vocab, H)
    s.onorm = _norm(rng, H)
    for il in range(cfg.n_layer):
        if s.is_full(il):
            s.layers.append(full_layer(seed * 1000 + il, cfg.nh, cfg.full_codes))
        else:
            L = gdn_layer(seed * 1000 + il, cfg.n_vh, cfg.gdn_codes)
            L.ssm[:] = 0.0
            L.tail[:] = 0.0
            s.layers.append(L)
        frng = np.random.default_rng(seed * 1000 + 500 + il)
        if cfg.ffn == FFN_DENSE:
            c = cfg.ffn_codes
            s.ffn.append({"g": _mat(frng, c[0], cfg.n_ff, H), "u": _mat(frng, c[1], cfg.n_ff, H),
                          "d": _mat(frng, c[2], H, cfg.n_ff)})
        elif cfg.ffn == FFN_MOE:
            E, F = cfg.n_exp, cfg.exp_ff
            s.ffn.append({"gi": frng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02),
                          "gate": _models._random_q4k(frng, E * F, H, 0.02),
                          "up": _models._random_q4k(frng, E * F, H, 0.02),
                          "down": _models._random_q4k(frng, E * H, F, 0.02)})
        else:
            s.ffn.append(None)
    return s


class QwenStackDriver:
    """Runs a QwenStack through an engine, the way src/qwen35_engine.py:310-327
    does per token (layer op, cache append by the caller, FFN, residual, head),
    or on the device (draco_qwen_* entry points, engine "hip" only).

    `ops` is a dict of callables: gdn(h1, w, ssm, tail, x2n, x2o),
    full(h1, w, Kr, Vc, told, pos0, x2n, x2o, krn, vrn), dense(xn, p, out),
    moe(xn, p, out), head(x, norm, h, eps, head, code, vocab, logits, scratch)."""

    def __init__(self, stack, ops, lib=None):
        from .driver import DracoMoeP, M6DenseP
        cfg = stack.cfg
        self.stack, self.cfg, self.ops, self.lib = stack, cfg, ops, lib
        self.keep = []
        self.kr, self.vc = {}, {}
        self.descs = (DracoQwenLayer * cfg.n_layer)()
        self.ffn_p = []
        for il, L in enumerate(stack.layers):
            d = self.descs[il]
            if isinstance(L, FullLayer):
                kr = np.zeros(cfg.max_t * NKV_A * HD_A, np.float32)
                vc = np.zeros(cfg.max_t * NKV_A * HD_A, np.float32)
                self.kr[il], self.vc[il] = kr, vc
                d.kind, d.w, d.state0, d.state1, d.max_t = 1, L.ptr().value, _pf(kr), _pf(vc), cfg.max_t
                self.keep += [kr, vc]
            else:
                d.kind, d.w, d.state0, d.state1, d.max_t = 0, L.ptr().value, _pf(L.ssm), _pf(L.tail), 0
            f = stack.ffn[il]
            if cfg.ffn == FFN_DENSE:
                p = M6DenseP()
                p.g, p.u, p.d = f["g"].ctypes.data, f["u"].ctypes.data, f["d"].ctypes.data
                p.cg, p.cu, p.cd = cfg.ffn_codes
                p.n_ff, p.h = cfg.n_ff, H
                d.ffn_kind, d.ffn = FFN_DENSE, ct.addressof(p)
            elif cfg.ffn == FFN_MOE:
                E, F = cfg.n_exp, cfg.exp_ff
                ptrs = np.zeros(3 * E, np.uint64)
                codes = np.full(3 * E, Q4_K, np.int32)
                for k, nm in enumerate(("gate", "up", "down")):
                    per = f[nm].nbytes // E
                    ptrs[k::3] = f[nm].ctypes.data + per * np.arange(E, dtype=np.uint64)
                scratch = np.zeros(3 * cfg.n_used * F + cfg.n_used * H + 64, np.float32)
                p = DracoMoeP()
                p.ptrs, p.codes, p.gate_inp = ptrs.ctypes.data, codes.ctypes.data, _pf(f["gi"])
                p.n_exp, p.n_used, p.inter, p.n_in, p.n_out = E, cfg.n_used, F, H, H
                p.scratch = _pf(scratch)
                self.keep += [ptrs, codes, scratch]
                d.ffn_kind, d.ffn = FFN_MOE, ct.addressof(p)
            else:
                p = None
                d.ffn_kind, d.ffn = FFN_NONE, None
            self.ffn_p.append(p)
            self.keep.append(p)
        self.x = np.zeros(H, np.float32)
        self.x2n = np.zeros(H, np.float32)
        self.x2o = np.zeros(H, np.float32)
        self.ffo = np.zeros(H, np.float32)
        self.krn = np.zeros(NKV_A * HD_A, np.float32)
        self.vrn = np.zeros(NKV_A * HD_A, np.float32)
        self.logits = np.zeros(cfg.vocab, np.float32)
        self.hsc = np.zeros(H, np.float32)
        self.emb_row = stack.emb.nbytes // cfg.vocab
        # layers after which forward() keeps a copy of the hidden state
        # (depth[il]: the last token's), for per-depth comparisons
        self.record = ()
        self.depth = {}

    # -- the reference's per-token forward, op by op (host state) --
    def embed(self, tok):
        from . import gguf_np
        return gguf_np.dequant_row(self.cfg.emb_code, self.stack.emb[tok * self.emb_row:(tok + 1) * self.emb_row])

    def forward(self, tok, pos):
        cfg, o = self.cfg, self.ops
        self.x[:] = self.embed(int(tok))
        row = NKV_A * HD_A
        for il, L in enumerate(self.stack.layers):
            if isinstance(L, FullLayer):
                o["full"](_pf(self.x), L.ptr(), _pf(self.kr[il]), _pf(self.vc[il]), pos, pos, _pf(self.x2n),
                          _pf(self.x2o), _pf(self.krn), _pf(self.vrn))
                self.kr[il][pos * row:(pos + 1) * row] = self.krn
                self.vc[il][pos * row:(pos + 1) * row] = self.vrn
            else:
                o["gdn"](_pf(self.x), L.ptr(), _pf(L.ssm), _pf(L.tail), _pf(self.x2n), _pf(self.x2o))
            p = self.ffn_p[il]
            if cfg.ffn == FFN_DENSE:
                o["dense"](_pf(self.x2n), ct.cast(ct.pointer(p), ct.c_void_p), _pf(self.ffo))
            elif cfg.ffn == FFN_MOE:
                o["moe"](_pf(self.x2n), ct.cast(ct.pointer(p), ct.c_void_p), _pf(self.ffo))
            else:
                self.ffo[:] = 0.0
            self.x[:] = self.x2o + self.ffo
            if il in self.record:
                self.depth[il] = self.x.copy()
        return self.x

    def logits_of_x(self, x=None):
        x = self.x if x is None else np.ascontiguousarray(x, np.float32)
        rc = self.ops["head"](_pf(x), _pf(self.stack.onorm), H, np.float32(self.cfg.eps),
                              ct.c_void_p(self.stack.head.ctypes.data), self.cfg.out_code, self.cfg.vocab,
                              _pf(self.logits), _pf(self.hsc))
        if rc:
            raise RuntimeError(f"head op rc={rc}")
        return self.logits

    def greedy(self, prompt, n_gen, collect_logits=()):
        for pos, t in enumerate(prompt):
            self.forward(t, pos)
        out, saved = [], {}
        lg = self.logits_of_x()
        if 0 in collect_logits:
            saved[0] = lg.copy()
        nid = int(np.argmax(lg.astype(np.float64)))
        out.append(nid)
        for s in range(1, n_gen):
            self.forward(nid, len(prompt) + s - 1)
            lg = self.logits_of_x()
            if s in collect_logits:
                saved[s] = lg.copy()
            nid = int(np.argmax(lg.astype(np.float64)))
            out.append(nid)
        return out, self.x.copy(), saved

    def reset(self):
        """src/qwen35_engine.py:335-337: zero every state array; with the device
        stack, push the zeroed arrays to the device state too."""
        for L in self.stack.layers:
            if isinstance(L, GdnLayer):
                L.ssm[:] = 0.0
                L.tail[:] = 0.0
        for a in list(self.kr.values()) + list(self.vc.values()):
            a[:] = 0.0
        if self.lib is not None:
            self._check(self.lib.draco_qwen_state_push(self._dp(), self.cfg.n_layer, self.cfg.max_t),
                        "draco_qwen_state_push")

    # -- the device stack --
    def _dp(self):
        return ct.cast(self.descs, ct.c_void_p)

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} rc={rc}: {self.lib.draco_last_error().decode()}")

    def forward_device(self, tok, pos):
        self.x[:] = self.embed(int(tok))
        self._check(self.lib.draco_qwen_forward(_pf(self.x), H, int(pos), self._dp(), self.cfg.n_layer),
                    "draco_qwen_forward")
        return self.x

    def prefill_device(self, ids, pos0):
        ids = np.ascontiguousarray(ids, np.int32)
        self._check(self.lib.draco_qwen_prefill(self._dp(), self.cfg.n_layer, H, ct.c_void_p(self.stack.emb.ctypes.data),
                                                self.cfg.emb_code, self.cfg.vocab,
                                                ids.ctypes.data_as(ct.POINTER(ct.c_int)), len(ids), int(pos0),
                                                _pf(self.x)), "draco_qwen_prefill")
        return self.x

    def generate_device(self, prompt, n_gen, pos0=0, use_graph=True):
        prompt = np.ascontiguousarray(prompt, np.int32)
        toks = np.zeros(n_gen, np.int32)
        hidden = np.zeros(H, np.float32)
        stats = np.zeros(4, np.float32)
        self._check(self.lib.draco_qwen_generate(
            self._dp(), self.cfg.n_layer, H, np.float32(self.cfg.eps), _pf(self.stack.onorm),
            ct.c_void_p(self.stack.head.ctypes.data), self.cfg.out_code, self.cfg.vocab,
            ct.c_void_p(self.stack.emb.ctypes.data), self.cfg.emb_code, int(pos0),
            prompt.ctypes.data_as(ct.POINTER(ct.c_int)), len(prompt), n_gen, int(use_graph),
            toks.ctypes.data_as(ct.POINTER(ct.c_int)), _pf(hidden), _pf(stats)), "draco_qwen_generate")
        self.x[:] = hidden
        return [int(t) for t in toks], hidden, (float(stats[0]), float(stats[1]))

    def pull_state(self, rows):
        self._check(self.lib.draco_qwen_state_pull(self._dp(), self.cfg.n_layer, int(rows)), "draco_qwen_state_pull")


def hip_ops(lib):
    """The HIP library's per-layer ops with the reference's signatures."""
    return {"gdn": lambda h1, w, ssm, tail, x2n, x2o: lib.m6_gdn_attn(h1, w, ssm, tail, None, x2n, x2o),
            "full": lambda h1, w, Kr, Vc, told, pos0, x2n, x2o, krn, vrn:
                lib.m6_full_attn(h1, w, Kr, Vc, told, pos0, None, None, x2n, x2o, krn, vrn),
            "dense": lib.m6_dense_op, "moe": lib.draco_moe_ffn_op, "head": lib.m6_head_op}
