"""Adapter: the oracle's llama entry points as an m6-ABI engine (test helper)."""
from dracohip.driver import EngineLib


def oracle_engine(oracle):
    return EngineLib(oracle.lib, forward="or_forward_token", head="or_head_op",
                     attn="or_llama_attn_op", dense="or_dense_op", name="oracle", moe="or_moe_ffn_op")


def oracle_qwen_ops(oracle):
    """The oracle's qwen35 per-layer ops as a QwenStackDriver op table."""
    import ctypes as ct
    L = oracle.lib
    u8p = ct.POINTER(ct.c_uint8)
    return {"gdn": L.or_gdn_attn, "full": L.or_full_attn, "dense": L.or_dense_op, "moe": L.or_moe_ffn_op,
            "head": lambda x, nw, h, eps, head, code, vocab, lg, sc:
                L.or_head_op(x, nw, h, eps, ct.cast(head, u8p), code, vocab, lg, sc)}
