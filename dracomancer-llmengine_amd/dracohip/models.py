"""Seeded synthetic models of the benchmark configurations, in GGUF byte format.

Convention (the reference defines none; fixed here and used everywhere):
  * one numpy Generator per model, np.random.default_rng(seed);
  * tensors are drawn in GGUF tensor order -- token_embd, then per layer
    attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down, then
    output (only when the head is not tied to the embedding);
  * each tensor is rng.standard_normal((n_out, n_in), dtype=float32) * wscale
    (0.02 for every benchmark configuration) and is encoded by draco_quantize (libdraco_hip.so, host code);
  * every RMSNorm weight is 1.0;
  * prompt ids: np.random.default_rng(seed + 1000).integers(0, vocab, n_prompt).

The GPU path and the CPU oracle consume the same bytes, so the encoder only
needs to be a valid GGUF encoder.
"""
import hashlib
import os
from dataclasses import dataclass, field

import numpy as np

from . import lib as _lib

Q8_0, Q5_K, Q6_K, Q4_K, F16, F32 = 0, 3, 4, 5, 7, 9


@dataclass
class LlamaConfig:
    name: str
    hidden: int
    n_layer: int
    n_head: int
    n_kv: int
    head_dim: int
    n_ff: int
    vocab: int
    eps: float
    rope_base: float
    codes: dict  # tensor kind -> format code (q, k, v, o, gate, up, down, emb, out)
    tied: bool = True
    n_prompt: int = 32
    n_gen: int = 64
    max_t: int = 1024
    chunk: int = 256
    wscale: float = 0.02
    # MoE FFN (n_exp > 0): softmax router over n_exp experts, top n_used,
    # experts of exp_ff SwiGLU rows (m6_granite_moe semantics) instead of the
    # dense gate/up/down
    n_exp: int = 0
    n_used: int = 0
    exp_ff: int = 0

    @property
    def rot(self):
        return self.head_dim

    @property
    def moe(self):
        return self.n_exp > 0


# configs[0] of BASELINE.json: SmolLM2-360M shape, all Q8_0, tied head.
SMOL360M = LlamaConfig(
    name="smollm2-360m-q8_0", hidden=960, n_layer=32, n_head=15, n_kv=5, head_dim=64, n_ff=2560,
    vocab=49152, eps=1e-5, rope_base=100000.0,
    codes=dict(q=Q8_0, k=Q8_0, v=Q8_0, o=Q8_0, gate=Q8_0, up=Q8_0, down=Q8_0, emb=Q8_0, out=Q8_0),
    tied=True, n_prompt=32, n_gen=64, max_t=1024)

# configs[2] of BASELINE.json: Llama-3.2-1B shape, Q4_K_M-style, tied head (Q6_K).
LLAMA1B = LlamaConfig(
    name="llama-3.2-1b-q4_k_m", hidden=2048, n_layer=16, n_head=32, n_kv=8, head_dim=64, n_ff=8192,
    vocab=128256, eps=1e-5, rope_base=500000.0,
    codes=dict(q=Q4_K, k=Q4_K, v=Q6_K, o=Q4_K, gate=Q4_K, up=Q4_K, down=Q6_K, emb=Q6_K, out=Q6_K),
    tied=True, n_prompt=960, n_gen=64, max_t=1024)

# small shapes for tests
TINY_K = LlamaConfig(
    name="tiny-kquant", hidden=512, n_layer=2, n_head=8, n_kv=2, head_dim=64, n_ff=1024, vocab=1000,
    eps=1e-5, rope_base=10000.0,
    codes=dict(q=Q4_K, k=Q4_K, v=Q6_K, o=Q4_K, gate=Q4_K, up=Q4_K, down=Q6_K, emb=Q6_K, out=Q6_K),
    tied=True, n_prompt=8, n_gen=16, max_t=64, wscale=0.25)

TINY_Q8 = LlamaConfig(
    name="tiny-q8_0", hidden=192, n_layer=2, n_head=3, n_kv=1, head_dim=64, n_ff=256, vocab=600,
    eps=1e-5, rope_base=100000.0,
    codes=dict(q=Q8_0, k=Q8_0, v=Q8_0, o=Q8_0, gate=Q8_0, up=Q8_0, down=Q8_0, emb=Q8_0, out=Q8_0),
    tied=True, n_prompt=8, n_gen=16, max_t=64, wscale=0.25)

# Q5_K_M-style mix (Q5_K for q/k/o/gate/up and the embedding, Q6_K for
# v/down and the untied head): the Q5_K parity cases
TINY_Q5 = LlamaConfig(
    name="tiny-q5_k_m", hidden=512, n_layer=2, n_head=8, n_kv=2, head_dim=64, n_ff=1024, vocab=1000,
    eps=1e-5, rope_base=10000.0,
    codes=dict(q=Q5_K, k=Q5_K, v=Q6_K, o=Q5_K, gate=Q5_K, up=Q5_K, down=Q6_K, emb=Q5_K, out=Q6_K),
    tied=False, n_prompt=8, n_gen=16, max_t=64, wscale=0.25)

# configs[3]'s attention block (32 q / 4 kv heads of 128, Q6_K projections,
# cache of 512 rows) as a one-layer llama model: the attention parity cases
ATTN_CFG3 = LlamaConfig(
    name="attn-cfg3-q6k", hidden=2048, n_layer=1, n_head=32, n_kv=4, head_dim=128, n_ff=256, vocab=256,
    eps=1e-6, rope_base=1000000.0,
    codes=dict(q=Q6_K, k=Q6_K, v=Q6_K, o=Q6_K, gate=Q4_K, up=Q4_K, down=Q4_K, emb=Q6_K, out=Q6_K),
    tied=True, n_prompt=8, n_gen=8, max_t=512)

# configs[3] of BASELINE.json: Qwen3-30B-A3B-shaped MoE stack -- 48 layers of
# attention (32 q / 4 kv heads of 128, Q6_K) + MoE FFN (128 experts, top 8,
# expert FFN 768, Q4_K experts, fp32 router N(0, 0.02)), hidden 2048, decode
# at context 512.  The configuration names no vocabulary; Qwen3's 151936 with
# an untied Q6_K head (Q4_K embedding) gives the greedy loop its tokens.
QWEN3_MOE = LlamaConfig(
    name="qwen3-30b-a3b-moe-stack", hidden=2048, n_layer=48, n_head=32, n_kv=4, head_dim=128, n_ff=0,
    vocab=151936, eps=1e-6, rope_base=1000000.0,
    codes=dict(q=Q6_K, k=Q6_K, v=Q6_K, o=Q6_K, gate=Q4_K, up=Q4_K, down=Q4_K, emb=Q4_K, out=Q6_K),
    tied=False, n_prompt=448, n_gen=64, max_t=512, n_exp=128, n_used=8, exp_ff=768)

# configs[3]'s first 8 layers (the same layer weights: seed 3 draws them first)
# with a short prompt: the deeper MoE parity case against the compiled reference
QWEN3_MOE8 = LlamaConfig(
    name="qwen3-moe-stack-8", hidden=2048, n_layer=8, n_head=32, n_kv=4, head_dim=128, n_ff=0,
    vocab=151936, eps=1e-6, rope_base=1000000.0,
    codes=dict(q=Q6_K, k=Q6_K, v=Q6_K, o=Q6_K, gate=Q4_K, up=Q4_K, down=Q4_K, emb=Q4_K, out=Q6_K),
    tied=False, n_prompt=8, n_gen=8, max_t=64, n_exp=128, n_used=8, exp_ff=768)

# the same layer shape in two layers with a small vocabulary: MoE parity cases
MOE_TINY = LlamaConfig(
    name="moe-tiny", hidden=2048, n_layer=2, n_head=32, n_kv=4, head_dim=128, n_ff=0, vocab=1024, eps=1e-6,
    rope_base=1000000.0,
    codes=dict(q=Q6_K, k=Q6_K, v=Q6_K, o=Q6_K, gate=Q4_K, up=Q4_K, down=Q4_K, emb=Q4_K, out=Q6_K),
    tied=False, n_prompt=8, n_gen=16, max_t=64, n_exp=128, n_used=8, exp_ff=768)

CONFIGS = {c.name: c for c in (SMOL360M, LLAMA1B, TINY_K, TINY_Q8, TINY_Q5, ATTN_CFG3, QWEN3_MOE, MOE_TINY,
                                QWEN3_MOE8)}


@dataclass
class LlamaModel:
    cfg: LlamaConfig
    seed: int
    tensors: dict = field(default_factory=dict)  # name -> (uint8 bytes, code, n_out, n_in)
    norms: dict = field(default_factory=dict)    # name -> float32

    def head(self):
        name = "token_embd.weight" if self.cfg.tied else "output.weight"
        return self.tensors[name]

    def digest(self):
        h = hashlib.sha256()
        for name in sorted(self.tensors):
            h.update(name.encode())
            h.update(self.tensors[name][0].tobytes())
        return h.hexdigest()

    def prompt(self, n=None):
        n = self.cfg.n_prompt if n is None else n
        return np.random.default_rng(self.seed + 1000).integers(0, self.cfg.vocab, n).astype(np.int32)

    def nbytes(self):
        return sum(t[0].nbytes for t in self.tensors.values())


def _draw(rng, n_out, n_in, wscale):
    w = rng.standard_normal((n_out, n_in), dtype=np.float32)
    w *= np.float32(wscale)
    return w


def _tensor(rng, code, n_out, n_in, wscale=0.02, rows_per_chunk=16384):
    out = np.empty(n_out * _lib.row_bytes(code, n_in), np.uint8)
    rb = _lib.row_bytes(code, n_in)
    # draw in row chunks (same stream order as one big draw) to bound memory
    for r0 in range(0, n_out, rows_per_chunk):
        r1 = min(n_out, r0 + rows_per_chunk)
        w = _draw(rng, r1 - r0, n_in, wscale)
        out[r0 * rb:r1 * rb] = _lib.quantize(code, w)
    return out


def _random_q4k(rng, n_rows, n_in, wscale):
    """Random Q4_K rows without drawing floats: every byte of each 144-byte
    super-block uniform (nibbles q, 6-bit scales sc and mins m), then d and
    dmin set so that w = d*sc*q - dmin*m has mean ~0 (dmin = 7.5 d) and
    standard deviation ~wscale (about 255 d for uniform q, sc, m).  Used for
    MoE experts, whose N(0, wscale) draws would take minutes at the configs[3]
    size (29 G values); the kernels' work and bytes do not depend on the
    values, and GPU and CPU consume the same bytes."""
    nblk = n_rows * (n_in // 256)
    words = rng.bit_generator.random_raw((nblk * 144 + 7) // 8)  # uniform 64-bit words of the generator
    blk = words.view(np.uint8)[:nblk * 144].reshape(nblk, 144)
    d = np.float16(wscale / 255.0)
    dmin = np.float16(7.5 * float(d))
    blk[:, 0:2] = np.frombuffer(d.tobytes(), np.uint8)
    blk[:, 2:4] = np.frombuffer(dmin.tobytes(), np.uint8)
    return blk.reshape(-1)


def build_llama(cfg, seed=0):
    rng = np.random.default_rng(seed)
    m = LlamaModel(cfg=cfg, seed=seed)
    H, QD, KD = cfg.hidden, cfg.n_head * cfg.head_dim, cfg.n_kv * cfg.head_dim
    c = cfg.codes
    ws = cfg.wscale
    m.tensors["token_embd.weight"] = (_tensor(rng, c["emb"], cfg.vocab, H, ws), c["emb"], cfg.vocab, H)
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output",
             "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down"}
    for il in range(cfg.n_layer):
        p = f"blk.{il}."
        for kind, n_out, n_in in (("q", QD, H), ("k", KD, H), ("v", KD, H), ("o", H, QD)):
            m.tensors[p + names[kind] + ".weight"] = (_tensor(rng, c[kind], n_out, n_in, ws), c[kind], n_out, n_in)
        if cfg.moe:
            # router fp32 [n_exp][H] N(0, wscale); experts as random Q4_K blocks,
            # each 3-D tensor [n_exp][rows][cols] stored as n_exp * rows rows
            E, F = cfg.n_exp, cfg.exp_ff
            gi = _draw(rng, E, H, ws)
            m.tensors[p + "ffn_gate_inp.weight"] = (gi.view(np.uint8).reshape(-1), F32, E, H)
            for kind, rows, n_in in (("gate", F, H), ("up", F, H), ("down", H, F)):
                if c[kind] != Q4_K:
                    raise ValueError("MoE experts are generated as Q4_K")
                m.tensors[p + names[kind] + "_exps.weight"] = (_random_q4k(rng, E * rows, n_in, ws), c[kind],
                                                               E * rows, n_in)
        else:
            for kind, n_out, n_in in (("gate", cfg.n_ff, H), ("up", cfg.n_ff, H), ("down", H, cfg.n_ff)):
                m.tensors[p + names[kind] + ".weight"] = (_tensor(rng, c[kind], n_out, n_in, ws), c[kind], n_out,
                                                          n_in)
        m.norms[p + "attn_norm.weight"] = np.ones(H, np.float32)
        m.norms[p + "ffn_norm.weight"] = np.ones(H, np.float32)
    if not cfg.tied:
        m.tensors["output.weight"] = (_tensor(rng, c["out"], cfg.vocab, H, ws), c["out"], cfg.vocab, H)
    m.norms["output_norm.weight"] = np.ones(H, np.float32)
    return m


# ------------------------------------------------------------ GGUF files --
# Metadata keys are the llama family's, as the reference driver reads them
# (src/smol_engine.py:26-40: llama.block_count, .embedding_length,
# .attention.head_count(_kv), .attention.layer_norm_rms_epsilon,
# .rope.dimension_count, .rope.freq_base, .feed_forward_length, .vocab_size).

def save_llama_gguf(model, path):
    """Write a LlamaModel as a GGUF v3 file (tensor data as stored, norms as F32)."""
    from . import gguf
    cfg = model.cfg
    fields = {
        "general.architecture": "llama", "general.name": cfg.name,
        "llama.block_count": cfg.n_layer, "llama.embedding_length": cfg.hidden,
        "llama.attention.head_count": cfg.n_head, "llama.attention.head_count_kv": cfg.n_kv,
        "llama.attention.layer_norm_rms_epsilon": float(cfg.eps), "llama.rope.dimension_count": cfg.rot,
        "llama.rope.freq_base": float(cfg.rope_base), "llama.feed_forward_length": cfg.n_ff,
        "llama.vocab_size": cfg.vocab, "llama.context_length": cfg.max_t,
        "dracomancer.seed": int(model.seed), "dracomancer.n_prompt": cfg.n_prompt, "dracomancer.n_gen": cfg.n_gen,
    }
    tensors = []
    for name, (buf, code, n_out, n_in) in model.tensors.items():
        tensors.append((name, gguf.GGML_OF_M5[code], (n_in, n_out), buf))
    for name, w in model.norms.items():
        tensors.append((name, "F32", (w.size,), np.ascontiguousarray(w, np.float32)))
    gguf.write_gguf(path, fields, tensors)


def load_llama_gguf(path, max_t=None):
    """A LlamaModel whose tensors are zero-copy views of the mapped file
    (the engine registers them by those addresses)."""
    from . import gguf
    r = gguf.FastGGUF(path)

    def kv(key, default=None):
        f = r.fields.get("llama." + key)
        return default if f is None else f.contents()

    T = {t.name: t for t in r.tensors}
    kind = {"attn_q": "q", "attn_k": "k", "attn_v": "v", "attn_output": "o", "ffn_gate": "gate",
            "ffn_up": "up", "ffn_down": "down"}
    codes = {"emb": gguf.M5_CODE[T["token_embd.weight"].tensor_type.name]}
    for tname, k in kind.items():
        codes[k] = gguf.M5_CODE[T["blk.0." + tname + ".weight"].tensor_type.name]
    tied = "output.weight" not in T
    codes["out"] = codes["emb"] if tied else gguf.M5_CODE[T["output.weight"].tensor_type.name]
    seed_f = r.fields.get("dracomancer.seed")
    np_f, ng_f = r.fields.get("dracomancer.n_prompt"), r.fields.get("dracomancer.n_gen")
    gen = r.fields.get("general.name")
    H, NH = int(kv("embedding_length")), int(kv("attention.head_count"))
    cfg = LlamaConfig(
        name=gen.contents() if gen else os.path.basename(path), hidden=H, n_layer=int(kv("block_count")),
        n_head=NH, n_kv=int(kv("attention.head_count_kv")), head_dim=H // NH, n_ff=int(kv("feed_forward_length")),
        vocab=int(kv("vocab_size", T["token_embd.weight"].shape[1])),
        eps=float(kv("attention.layer_norm_rms_epsilon")), rope_base=float(kv("rope.freq_base")), codes=codes,
        tied=tied, n_prompt=int(np_f.contents()) if np_f else 32, n_gen=int(ng_f.contents()) if ng_f else 64,
        max_t=int(max_t or kv("context_length", 1024)))
    if int(kv("rope.dimension_count", cfg.head_dim)) != cfg.head_dim:
        raise ValueError("partial rope (rope.dimension_count != head_dim) is not served by this driver")
    m = LlamaModel(cfg=cfg, seed=int(seed_f.contents()) if seed_f else 0)
    for name, t in T.items():
        if t.tensor_type.name == "F32" and len(t.shape) == 1:
            m.norms[name] = t.data
        else:
            m.tensors[name] = (t.data.reshape(-1), gguf.M5_CODE[t.tensor_type.name], int(t.shape[1]), int(t.shape[0]))
    return m
