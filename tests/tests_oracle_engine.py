"""Adapter: the oracle's llama entry points as an m6-ABI engine (test helper)."""
from dracohip.driver import EngineLib


def oracle_engine(oracle):
    return EngineLib(oracle.lib, forward="or_forward_token", head="or_head_op",
                     attn="or_llama_attn_op", dense="or_dense_op", name="oracle", moe="or_moe_ffn_op")
