"""The qwen35 hybrid stack on the GPU (G G G F layers of the configs[4] shape,
with a dense or a MoE FFN), against the compiled reference's per-layer ops
composed as src/qwen35_engine.py:310-327 does (tests/golden/qwen_tiny*.npz)
and against the oracle.

Paths: the drop-in per-layer ops with host state (m6_gdn_attn / m6_full_attn
/ m6_dense_op / draco_moe_ffn_op / m6_head_op, as the reference's driver
calls them), the device-resident token forward (draco_qwen_forward), the
graph-replayed greedy loop (draco_qwen_generate, prompt token by token or in
chunks) and the chunked prefill (draco_qwen_prefill, the forward_chunk
contract of src/qwen35_prefill.py:209-239).

Bars: greedy tokens identical; logits within 1e-4 normwise; hidden state and
device state (GDN recurrent state and conv tail, K / V cache rows) within
1e-4 normwise of the reference / oracle (each GEMV is within 1e-5; four
layers of reordered fp32 sums and a 20-token recurrence compound it).
"""
import ctypes as ct

import numpy as np
import pytest

from helpers import golden, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-4
STACKS = [("qwen35-tiny", "qwen_tiny.npz", (0, 15)), ("qwen35-tiny-moe", "qwen_tiny_moe.npz", (0, 7))]


def _stack(name, hip):
    from dracohip import qwen35 as Q
    hip.draco_reset()
    cfg = Q.STACKS[name]
    return cfg, Q.build_stack(cfg, 0)


@pytest.mark.parametrize("name,fname,steps", STACKS)
def test_per_layer_ops_host_state(hip, name, fname, steps):
    from dracohip import qwen35 as Q
    g = golden(fname)
    cfg, stack = _stack(name, hip)
    drv = Q.QwenStackDriver(stack, Q.hip_ops(hip))
    print(f"[qwen stack] {name} per-layer ops", flush=True)
    toks, hidden, lg = drv.greedy(stack.prompt(), cfg.n_gen, collect_logits=steps)
    assert toks == list(g["tokens"])
    assert rel_err(hidden, g["hidden"]) <= TOL
    for s in steps:
        assert rel_err(lg[s], g[f"logits{s}"]) <= TOL


@pytest.mark.parametrize("use_graph", [False, True])
@pytest.mark.parametrize("chunk", [0, 8])
@pytest.mark.parametrize("name,fname,steps", STACKS)
def test_device_generate(hip, name, fname, steps, chunk, use_graph):
    """draco_qwen_generate: prompt token by token (chunk 0) or in 8-token
    chunks (MoE stacks always go token by token), greedy decode on the device."""
    from dracohip import qwen35 as Q
    g = golden(fname)
    cfg, stack = _stack(name, hip)
    drv = Q.QwenStackDriver(stack, Q.hip_ops(hip), lib=hip)
    old = hip.draco_set_qwen_chunk(chunk)
    try:
        print(f"[qwen stack] {name} device generate chunk {chunk} graph {use_graph}", flush=True)
        toks, hidden, _ = drv.generate_device(stack.prompt(), cfg.n_gen, use_graph=use_graph)
    finally:
        hip.draco_set_qwen_chunk(old)
    assert toks == list(g["tokens"])
    assert rel_err(hidden, g["hidden"]) <= TOL


def test_device_forward_and_state_match_oracle(hip, oracle):
    """draco_qwen_forward token by token against the oracle's per-layer ops:
    hidden after every token, then every layer's device state pulled back."""
    from dracohip import qwen35 as Q
    from tests_oracle_engine import oracle_qwen_ops
    cfg, stack = _stack("qwen35-tiny", hip)
    dev = Q.QwenStackDriver(stack, Q.hip_ops(hip), lib=hip)
    ref_stack = Q.build_stack(cfg, 0)
    ref = Q.QwenStackDriver(ref_stack, oracle_qwen_ops(oracle))
    p = stack.prompt()
    for pos, t in enumerate(p[:12]):
        print(f"[qwen stack] forward token {pos}", flush=True)
        x = dev.forward_device(t, pos).copy()
        xr = ref.forward(t, pos)
        assert rel_err(x, xr) <= TOL, (pos, rel_err(x, xr))
    dev.pull_state(12)
    _compare_state(dev, ref, stack, ref_stack, 12)


def _compare_state(dev, ref, stack, ref_stack, rows):
    from dracohip import qwen35 as Q
    n = rows * Q.NKV_A * Q.HD_A
    for il, (L, Lr) in enumerate(zip(stack.layers, ref_stack.layers)):
        if isinstance(L, Q.FullLayer):
            assert rel_err(dev.kr[il][:n], ref.kr[il][:n]) <= TOL, il
            assert rel_err(dev.vc[il][:n], ref.vc[il][:n]) <= TOL, il
        else:
            assert rel_err(L.ssm, Lr.ssm) <= TOL, il
            assert rel_err(L.tail, Lr.tail) <= TOL, il


@pytest.mark.parametrize("chunk", [8, 64])
def test_chunked_prefill_matches_token_serial(hip, oracle, chunk):
    """draco_qwen_prefill (f16-MFMA projections over the chunk, token-serial
    scan, causal gated attention) leaves the state of the oracle's token-serial
    forward: the last hidden row and every layer's state; a decode step after
    it gives the oracle's next hidden state."""
    from dracohip import qwen35 as Q
    from tests_oracle_engine import oracle_qwen_ops
    cfg, stack = _stack("qwen35-tiny", hip)
    dev = Q.QwenStackDriver(stack, Q.hip_ops(hip), lib=hip)
    ref_stack = Q.build_stack(cfg, 0)
    ref = Q.QwenStackDriver(ref_stack, oracle_qwen_ops(oracle))
    p = stack.prompt()
    n = 19
    old = hip.draco_set_qwen_chunk(chunk)
    try:
        print(f"[qwen stack] chunked prefill chunk {chunk}", flush=True)
        x = dev.prefill_device(p[:n], 0).copy()
    finally:
        hip.draco_set_qwen_chunk(old)
    for pos in range(n):
        xr = ref.forward(p[pos], pos)
    assert rel_err(x, xr) <= TOL, rel_err(x, xr)
    dev.pull_state(n)
    _compare_state(dev, ref, stack, ref_stack, n)
    x = dev.forward_device(p[n], n).copy()
    xr = ref.forward(p[n], n)
    assert rel_err(x, xr) <= TOL


def test_state_reset_and_repeat(hip):
    """The reference's reset (zero every state array) followed by a push
    restarts the device state: two generations give the same tokens."""
    from dracohip import qwen35 as Q
    cfg, stack = _stack("qwen35-tiny", hip)
    drv = Q.QwenStackDriver(stack, Q.hip_ops(hip), lib=hip)
    a = drv.generate_device(stack.prompt(), 6)[0]
    drv.reset()
    b = drv.generate_device(stack.prompt(), 6)[0]
    assert a == b
