"""Llama layer shapes outside the benchmark configurations, and the greedy
pick's NaN semantics, on the GPU against the oracle engine.

The reference's llama_attn_core takes any GQA ratio and head dim
(src/m6_engine.c:425-511) and its greedy pick is np.argmax over the logits
(src/smol_engine.py:212).  Cases:
- an o projection of 24 super-blocks (48 q heads x 128): a width the split-K
  launch does not cover, so the layer takes the plain launch;
- head dim 128 with 16 q heads per kv head (64 q / 4 kv): the per-head
  attention kernel;
- head dims 80 and 96 and 32 q heads per kv head: the generic attention
  kernel, and the token-serial path of draco_llama_prefill;
- logits with NaN rows: the first NaN's index wins; all NaN gives token 0 and
  the state still advances.
Bars: greedy tokens identical; final hidden state within the decode bar;
prefill logits within 1e-4 normwise.
"""
import dataclasses

import numpy as np
import pytest

from helpers import rel_err
from dracohip import models
from dracohip.driver import LlamaDriver, hip_engine_lib

pytestmark = pytest.mark.gpu


def hid_tol(ref):
    return 1e-3 * max(1.0, float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2))))


SHAPES = [  # name, hidden, n_head, n_kv, head_dim
    ("o-24-superblocks", 2048, 48, 8, 128),
    ("gqa16-hd128", 2048, 64, 4, 128),
    ("hd80", 512, 16, 4, 80),
    ("hd96-gqa32", 512, 32, 1, 96),
]


def _model(name, hidden, n_head, n_kv, head_dim, seed):
    cfg = dataclasses.replace(models.TINY_K, name=name, hidden=hidden, n_head=n_head, n_kv=n_kv,
                              head_dim=head_dim, n_layer=2, n_ff=1024, n_prompt=12, n_gen=8, max_t=64,
                              wscale=0.25 if hidden <= 512 else 0.05)
    return cfg, models.build_llama(cfg, seed)


@pytest.mark.parametrize("use_graph", [False, True])
@pytest.mark.parametrize("name,hidden,n_head,n_kv,head_dim", SHAPES, ids=[s[0] for s in SHAPES])
def test_attention_shapes_match_oracle(oracle, name, hidden, n_head, n_kv, head_dim, use_graph):
    from tests_oracle_engine import oracle_engine
    from dracohip import lib
    cfg, model = _model(name, hidden, n_head, n_kv, head_dim, 11)
    ref = LlamaDriver(model, oracle_engine(oracle))
    rt, rh, _ = ref.greedy(model.prompt(), cfg.n_gen)
    lib.load().draco_reset()
    drv = LlamaDriver(model, hip_engine_lib())
    print(f"[shapes] {name} device generate graph={use_graph}", flush=True)
    toks, hidden_d, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    assert toks == rt
    assert np.max(np.abs(hidden_d - rh)) <= hid_tol(rh)
    lib.load().draco_reset()
    drv2 = LlamaDriver(model, hip_engine_lib())
    print(f"[shapes] {name} per-token drop-in", flush=True)
    t2, h2, _ = drv2.greedy(model.prompt(), cfg.n_gen)
    assert t2 == rt
    assert np.max(np.abs(h2 - rh)) <= hid_tol(rh)


@pytest.mark.parametrize("name,hidden,n_head,n_kv,head_dim", SHAPES, ids=[s[0] for s in SHAPES])
def test_prefill_chunk_shapes_match_oracle(oracle, name, hidden, n_head, n_kv, head_dim):
    """draco_llama_prefill (forward_chunk) at every shape: batched where the
    prefill attention kernel serves it, token by token otherwise; the
    logits after the prompt and one more decode token match the oracle's."""
    from tests_oracle_engine import oracle_engine
    from dracohip import lib
    cfg, model = _model(name, hidden, n_head, n_kv, head_dim, 12)
    p = model.prompt()
    ref = LlamaDriver(model, oracle_engine(oracle))
    for pos, t in enumerate(p):
        ref.forward(t, pos)
    lr = ref.logits_of_x().copy()
    ref.forward(3, len(p))
    lr2 = ref.logits_of_x().copy()
    lib.load().draco_reset()
    drv = LlamaDriver(model, hip_engine_lib())
    print(f"[shapes] {name} prefill chunk", flush=True)
    lg = drv.prefill_chunk(p, 0).copy()
    assert rel_err(lg, lr) <= 1e-4
    assert drv.tl[0][0] == len(p)
    drv.forward(3, len(p))
    assert rel_err(drv.logits_of_x(), lr2) <= 1e-4


def _nan_rows(model, rows):
    """Q6_K head rows whose first block scale is the f16 NaN 0x7e00 (the
    block's last two bytes): those logits are NaN, the others finite."""
    buf, code = model.head()[:2]
    assert code == models.Q6_K
    rb = buf.nbytes // model.cfg.vocab
    for r in rows:
        buf[r * rb + 208:r * rb + 210] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)


@pytest.mark.parametrize("use_graph", [False, True])
def test_greedy_first_nan_wins(oracle, use_graph):
    """Rows 7 and 3 of the (untied) head give NaN logits: np.argmax picks 3,
    the first NaN; the device loop's fused argmax does the same at every
    step, token for token with the oracle engine's np.argmax loop."""
    from tests_oracle_engine import oracle_engine
    from dracohip import lib
    cfg = dataclasses.replace(models.TINY_K, name="nan-rows", tied=False, n_gen=6)
    model = models.build_llama(cfg, 21)
    _nan_rows(model, (7, 3))
    ref = LlamaDriver(model, oracle_engine(oracle))
    rt, _, _ = ref.greedy(model.prompt(), cfg.n_gen)
    assert rt[0] == 3
    lib.load().draco_reset()
    drv = LlamaDriver(model, hip_engine_lib())
    print(f"[shapes] first-NaN greedy graph={use_graph}", flush=True)
    toks, _, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    assert toks == rt


@pytest.mark.parametrize("use_graph", [False, True])
def test_all_nan_logits_give_token_zero(use_graph):
    """A final-norm weight of NaN makes every logit NaN: np.argmax returns 0
    (the first NaN), the loop feeds token 0 on and the state advances by
    every step (no out-of-range embedding row)."""
    from dracohip import lib
    cfg = dataclasses.replace(models.TINY_K, name="nan-all", n_gen=5)
    model = models.build_llama(cfg, 22)
    lib.load().draco_reset()
    drv = LlamaDriver(model, hip_engine_lib())
    drv.onorm = drv.onorm.copy()
    drv.onorm[0] = np.nan
    print(f"[shapes] all-NaN logits graph={use_graph}", flush=True)
    toks, _, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    assert toks == [0] * cfg.n_gen
    assert drv.tl[0][0] == cfg.n_prompt + cfg.n_gen - 1


Q8_HEADS = [(960, 15, 5, 16403), (2048, 32, 8, 20000)]  # 30 / 64 Q8_0 blocks per row, ragged last row group


def _q8_nan_rows(model, rows):
    """Q8_0 head rows whose first block scale is the f16 NaN 0x7e00 (the
    block's first two bytes): those logits are NaN, the others finite."""
    buf, code = model.head()[:2]
    assert code == models.Q8_0
    rb = buf.nbytes // model.cfg.vocab
    for r in rows:
        buf[r * rb:r * rb + 2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)


@pytest.mark.parametrize("hidden,nh,nkv,vocab", Q8_HEADS, ids=[f"h{s[0]}-v{s[3]}" for s in Q8_HEADS])
def test_q8_head_row_groups_match_oracle(oracle, hidden, nh, nkv, vocab):
    """Q8_0 heads of at least 16384 rows run the persistent row-group kernel
    (x staged once per block, row groups of 32 rows): the per-token drop-in
    path's logits within 1e-5 of the oracle engine's with the kernel on and
    off (k_seg), greedy tokens equal; the device loop's fused argmax gives the
    oracle engine's tokens, also with NaN rows in the head (the first NaN
    wins, as np.argmax)."""
    from tests_oracle_engine import oracle_engine
    from dracohip import lib
    L = lib.load()
    cfg = dataclasses.replace(models.SMOL360M, name=f"q8-head-{hidden}-{vocab}", hidden=hidden, n_head=nh, n_kv=nkv,
                              n_layer=2, n_ff=1024, vocab=vocab, tied=False, n_prompt=8, n_gen=6, max_t=64)
    model = models.build_llama(cfg, 51)
    ref = LlamaDriver(model, oracle_engine(oracle))
    rt, _, rl = ref.greedy(model.prompt(), cfg.n_gen, collect_logits=(0, 3))
    old = L.draco_set_seg_rows(-1)
    try:
        for rows in (2, 0):
            L.draco_set_seg_rows(rows)
            L.draco_reset()
            drv = LlamaDriver(model, hip_engine_lib())
            print(f"[shapes] q8 head h{hidden} v{vocab} seg_rows {rows}", flush=True)
            toks, _, lg = drv.greedy(model.prompt(), cfg.n_gen, collect_logits=(0, 3))
            assert toks == rt
            for s in (0, 3):
                assert rel_err(lg[s], rl[s]) <= 1e-5
            L.draco_reset()
            drv = LlamaDriver(model, hip_engine_lib())
            toks, _, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=True)
            assert toks == rt
        _q8_nan_rows(model, (vocab - 5, 40))
        ref = LlamaDriver(model, oracle_engine(oracle))
        rt, _, _ = ref.greedy(model.prompt(), cfg.n_gen)
        assert rt[0] == 40
        L.draco_set_seg_rows(2)
        L.draco_reset()
        drv = LlamaDriver(model, hip_engine_lib())
        print(f"[shapes] q8 head h{hidden} v{vocab} NaN rows", flush=True)
        toks, _, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=True)
        assert toks == rt
    finally:
        L.draco_set_seg_rows(old)
