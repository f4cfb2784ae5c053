"""Llama-family driver over the m6 engine ABI.

Mirrors the reference driver src/smol_engine.py:97-195: it owns the weights
(byte arrays), the per-layer KV caches and `tlen` counters, fills the
reference's ctypes structures (M6LayerDesc, M6LlamaAttnP, M6DenseP -- field
for field the layouts of src/m6_engine.c:21-28, :270-273, :396-406) and runs
one m6_forward_token + m6_head_op per token, greedy-picking with argmax.

The engine library is pluggable: anything exporting the m6 ABI (the HIP
library here; tests also plug in the CPU checkers) is wrapped by an
`EngineLib`, whose op function pointers go into the descriptors exactly as
src/smol_engine.py:117-118 takes them from the same .so.
"""
import ctypes as ct

import numpy as np

from . import gguf_np

f32p = ct.POINTER(ct.c_float)


def pf(a):
    return a.ctypes.data_as(f32p)


class M6LayerDesc(ct.Structure):
    _fields_ = [("attn_norm", f32p), ("ffn_norm", f32p),
                ("attn", ct.c_void_p), ("attn_p", ct.c_void_p),
                ("ffn", ct.c_void_p), ("ffn_p", ct.c_void_p)]


class M6LlamaAttnP(ct.Structure):
    _fields_ = [("wq", ct.c_void_p), ("wk", ct.c_void_p), ("wv", ct.c_void_p), ("wo", ct.c_void_p),
                ("cq", ct.c_int), ("ck", ct.c_int), ("cv", ct.c_int), ("co", ct.c_int),
                ("n_head", ct.c_int), ("n_kv", ct.c_int), ("head_dim", ct.c_int),
                ("hidden", ct.c_int), ("rot", ct.c_int),
                ("rope_base", ct.c_float),
                ("kcache", f32p), ("vcache", f32p),
                ("tlen", ct.POINTER(ct.c_int)), ("max_t", ct.c_int),
                ("work", f32p)]


class M6DenseP(ct.Structure):
    _fields_ = [("g", ct.c_void_p), ("u", ct.c_void_p), ("d", ct.c_void_p),
                ("cg", ct.c_int), ("cu", ct.c_int), ("cd", ct.c_int),
                ("n_ff", ct.c_int), ("h", ct.c_int)]


class DracoMoeP(ct.Structure):
    """Parameters of the MoE FFN op (include/draco_hip.h DracoMoeP): the
    arguments of m6_granite_moe (src/m6_layer.c:771) in one struct."""
    _fields_ = [("ptrs", ct.c_void_p), ("codes", ct.c_void_p), ("gate_inp", f32p),
                ("n_exp", ct.c_int), ("n_used", ct.c_int), ("inter", ct.c_int), ("n_in", ct.c_int),
                ("n_out", ct.c_int), ("scratch", f32p)]


class EngineLib:
    """An m6-ABI library: forward_token, head_op and the op pointers (the MoE
    FFN op is optional: `moe=None` for libraries without one; a caller may set
    `moe_ptr` to a callback of its own)."""

    def __init__(self, cdll, forward="m6_forward_token", head="m6_head_op",
                 attn="m6_llama_attn_op", dense="m6_dense_op", name="hip", moe="draco_moe_ffn_op"):
        self.cdll = cdll
        self.name = name
        self.forward_token = getattr(cdll, forward)
        self.forward_token.argtypes = [f32p, ct.c_int, ct.c_float, ct.c_int, ct.c_void_p, ct.c_int, f32p]
        self.forward_token.restype = ct.c_int
        self.head_op = getattr(cdll, head)
        self.head_op.argtypes = [f32p, f32p, ct.c_int, ct.c_float, ct.c_void_p, ct.c_int, ct.c_int,
                                 f32p, f32p]
        self.head_op.restype = ct.c_int
        self.attn_ptr = ct.cast(getattr(cdll, attn), ct.c_void_p).value
        self.dense_ptr = ct.cast(getattr(cdll, dense), ct.c_void_p).value
        self.moe_ptr = ct.cast(getattr(cdll, moe), ct.c_void_p).value if moe and hasattr(cdll, moe) else None


def hip_engine_lib():
    from . import lib as _lib
    return EngineLib(_lib.load(), name="hip")


class LlamaDriver:
    """Per-token llama decode through an m6-ABI engine (src/smol_engine.py:134-195)."""

    def __init__(self, model, engine, max_t=None):
        cfg = model.cfg
        self.model, self.cfg, self.engine = model, cfg, engine
        self.H, self.NL = cfg.hidden, cfg.n_layer
        self.max_t = max_t or cfg.max_t
        NH, NKV, HD = cfg.n_head, cfg.n_kv, cfg.head_dim
        self.keep = []
        self.kc, self.vc, self.tl = [], [], []
        self.descs = (M6LayerDesc * self.NL)()
        T = model.tensors
        for il in range(self.NL):
            p = f"blk.{il}."
            an, fn = model.norms[p + "attn_norm.weight"], model.norms[p + "ffn_norm.weight"]
            self.descs[il].attn_norm = pf(an)
            self.descs[il].ffn_norm = pf(fn)
            a = M6LlamaAttnP()
            for fld, cfld, tname in (("wq", "cq", "attn_q"), ("wk", "ck", "attn_k"),
                                     ("wv", "cv", "attn_v"), ("wo", "co", "attn_output")):
                buf, code = T[p + tname + ".weight"][:2]
                setattr(a, fld, buf.ctypes.data)
                setattr(a, cfld, code)
            a.n_head, a.n_kv, a.head_dim, a.hidden, a.rot = NH, NKV, HD, self.H, cfg.rot
            a.rope_base = cfg.rope_base
            kc = np.zeros(self.max_t * NKV * HD, np.float32)
            vc = np.zeros(self.max_t * NKV * HD, np.float32)
            tl = np.zeros(1, np.int32)
            wk = np.zeros(NH * HD + 2 * NKV * HD + NH * self.max_t + 64, np.float32)
            a.kcache, a.vcache = pf(kc), pf(vc)
            a.tlen = tl.ctypes.data_as(ct.POINTER(ct.c_int))
            a.max_t = self.max_t
            a.work = pf(wk)
            self.keep += [an, fn, kc, vc, tl, wk, a]
            self.kc.append(kc)
            self.vc.append(vc)
            self.tl.append(tl)
            self.descs[il].attn = engine.attn_ptr
            self.descs[il].attn_p = ct.cast(ct.pointer(a), ct.c_void_p)
            if cfg.moe:
                self._moe_layer(il, p, T, engine)
                continue
            d = M6DenseP()
            for fld, cfld, tname in (("g", "cg", "ffn_gate"), ("u", "cu", "ffn_up"), ("d", "cd", "ffn_down")):
                buf, code = T[p + tname + ".weight"][:2]
                setattr(d, fld, buf.ctypes.data)
                setattr(d, cfld, code)
            d.n_ff, d.h = cfg.n_ff, self.H
            self.keep.append(d)
            self.descs[il].ffn = engine.dense_ptr
            self.descs[il].ffn_p = ct.cast(ct.pointer(d), ct.c_void_p)
        self.onorm = model.norms["output_norm.weight"]
        self.head_buf, self.head_code = model.head()[:2]
        emb = T["token_embd.weight"]
        self.emb_buf, self.emb_code = emb[0], emb[1]
        self.emb_row = emb[0].nbytes // cfg.vocab
        self.scratch = np.zeros(3 * (self.H + 64), np.float32)
        self.x = np.zeros(self.H, np.float32)
        self.logits = np.zeros(cfg.vocab, np.float32)
        self.hrms = np.zeros(self.H, np.float32)

    def _moe_layer(self, il, p, T, engine):
        """The MoE FFN of layer il as the descriptor's ffn op: the expert
        table as src/qwen35_engine.py:262-275 builds it (3 host pointers and
        codes per expert into the 3-D expert tensors), the fp32 router."""
        if engine.moe_ptr is None:
            raise RuntimeError(f"engine {engine.name} has no MoE FFN op")
        cfg = self.cfg
        E, F = cfg.n_exp, cfg.exp_ff
        ptrs = np.zeros(3 * E, np.uint64)
        codes = np.zeros(3 * E, np.int32)
        for k, tname in enumerate(("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")):
            buf, code = T[p + tname + ".weight"][:2]
            per = buf.nbytes // E
            ptrs[k::3] = buf.ctypes.data + per * np.arange(E, dtype=np.uint64)
            codes[k::3] = code
        gi = T[p + "ffn_gate_inp.weight"][0].view(np.float32)
        scratch = np.zeros(3 * cfg.n_used * F + cfg.n_used * self.H + 64, np.float32)
        mp = DracoMoeP()
        mp.ptrs, mp.codes, mp.gate_inp = ptrs.ctypes.data, codes.ctypes.data, pf(gi)
        mp.n_exp, mp.n_used, mp.inter, mp.n_in, mp.n_out = E, cfg.n_used, F, self.H, self.H
        mp.scratch = pf(scratch)
        self.keep += [ptrs, codes, gi, scratch, mp]
        self.descs[il].ffn = engine.moe_ptr
        self.descs[il].ffn_p = ct.cast(ct.pointer(mp), ct.c_void_p)

    def reset(self):
        """src/draco_engine_server.py:125-132: zero the state arrays and tlen."""
        for a in self.kc + self.vc:
            a[:] = 0
        for t in self.tl:
            t[0] = 0

    def embed(self, tok):
        r = self.emb_buf[tok * self.emb_row:(tok + 1) * self.emb_row]
        return gguf_np.dequant_row(self.emb_code, r)

    def forward(self, tok, pos):
        self.x[:] = self.embed(int(tok))
        rc = self.engine.forward_token(pf(self.x), self.H, np.float32(self.cfg.eps), int(pos),
                                       ct.cast(self.descs, ct.c_void_p), self.NL, pf(self.scratch))
        if rc != 0:
            raise RuntimeError(f"m6_forward_token rc={rc}")
        return self.x

    def logits_of_x(self):
        rc = self.engine.head_op(pf(self.x), pf(self.onorm), self.H, np.float32(self.cfg.eps),
                                 ct.c_void_p(self.head_buf.ctypes.data), self.head_code, self.cfg.vocab,
                                 pf(self.logits), pf(self.hrms))
        if rc != 0:
            raise RuntimeError(f"m6_head_op rc={rc}")
        return self.logits

    def generate_device(self, prompt, n_gen, use_graph=True):
        """The same greedy loop run entirely on the device (draco_llama_generate).

        Returns (tokens, final hidden x, stats) with stats = (decode ms, prefill ms).
        Only valid with the HIP engine library."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        toks = np.zeros(n_gen, np.int32)
        hidden = np.zeros(self.H, np.float32)
        stats = np.zeros(4, np.float32)
        L = self.engine.cdll
        rc = L.draco_llama_generate(
            ct.cast(self.descs, ct.c_void_p), self.NL, self.H, np.float32(self.cfg.eps), pf(self.onorm),
            ct.c_void_p(self.head_buf.ctypes.data), self.head_code, self.cfg.vocab,
            ct.c_void_p(self.emb_buf.ctypes.data), self.emb_code,
            prompt.ctypes.data_as(ct.POINTER(ct.c_int)), len(prompt), n_gen, int(use_graph),
            toks.ctypes.data_as(ct.POINTER(ct.c_int)), pf(hidden), pf(stats))
        if rc != 0:
            raise RuntimeError(f"draco_llama_generate rc={rc}: {L.draco_last_error().decode()}")
        self.x[:] = hidden
        return [int(t) for t in toks], hidden, (float(stats[0]), float(stats[1]))

    def prefill_chunk(self, ids, pos0):
        """Chunked prefill (the forward_chunk contract of src/qwen35_prefill.py:209-239
        and src/draco_engine_server.py:836-842, here for the llama family): leaves
        the engine state of forward(ids[i], pos0 + i) run token by token and
        returns the last position's logits.  Only valid with the HIP engine."""
        ids = np.ascontiguousarray(ids, np.int32)
        L = self.engine.cdll
        rc = L.draco_llama_prefill(ct.cast(self.descs, ct.c_void_p), self.NL, self.H, np.float32(self.cfg.eps),
                                   ct.c_void_p(self.emb_buf.ctypes.data), self.emb_code, self.cfg.vocab,
                                   ids.ctypes.data_as(ct.POINTER(ct.c_int)), len(ids), int(pos0), pf(self.x))
        if rc != 0:
            raise RuntimeError(f"draco_llama_prefill rc={rc}: {L.draco_last_error().decode()}")
        return self.logits_of_x()

    def greedy(self, prompt, n_gen, collect_logits=()):
        """Token-serial prefill then greedy decode (src/smol_engine.py:203-213)."""
        for pos, t in enumerate(prompt):
            self.forward(t, pos)
        out, saved = [], {}
        lg = self.logits_of_x()
        nid = int(np.argmax(lg.astype(np.float64)))
        if 0 in collect_logits:
            saved[0] = lg.copy()
        out.append(nid)
        for s in range(1, n_gen):
            self.forward(nid, len(prompt) + s - 1)
            lg = self.logits_of_x()
            if s in collect_logits:
                saved[s] = lg.copy()
            nid = int(np.argmax(lg.astype(np.float64)))
            out.append(nid)
        return out, self.x.copy(), saved
