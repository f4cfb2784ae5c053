"""Chunked prefill of the llama family (draco_llama_prefill, and the prompt of
draco_llama_generate) against token-serial decoding.

The contract is the reference's forward_chunk (src/qwen35_prefill.py:209-210,
src/draco_engine_server.py:836-842): afterwards the engine state is the one
forward(ids[i], pos0 + i) leaves when run token by token, and the call returns
the last position's logits.  Checked here against the compiled-reference
oracle's token-serial run (logits, KV caches), against this library's own
token-serial device path, across chunk boundaries (ragged chunks, a second
call at pos0 > 0), at head dims 64 and 128 and GQA ratios 1-5, and through the
goldens of whole greedy decodes (the device-generate tests, whose prompts go
through the chunked prefill by default).

Bars: logits 1e-4 normwise (every layer's products are reordered fp32 sums,
as in the per-token deep-layer KV bar); KV rows 1e-5 for layer 0 (one GEMM +
rope from the input) and 1e-4 deeper; greedy continuations identical.
"""
import ctypes as ct
import dataclasses

import numpy as np
import pytest

from helpers import golden, rel_err
from dracohip import lib, models
from dracohip.driver import LlamaDriver, hip_engine_lib

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _restore_chunk():
    L = lib.load()
    old = L.draco_set_prefill_chunk(-1)
    yield
    L.draco_set_prefill_chunk(old)


def _pair(cfg, oracle):
    from tests_oracle_engine import oracle_engine
    model = models.build_llama(cfg, 0)
    lib.load().draco_reset()
    return model, LlamaDriver(model, hip_engine_lib()), LlamaDriver(model, oracle_engine(oracle))


def _serial_logits(drv, ids, pos0):
    for i, t in enumerate(ids):
        drv.forward(int(t), pos0 + i)
    return drv.logits_of_x().copy()


@pytest.mark.parametrize("chunk", [256, 7, 1])
@pytest.mark.parametrize("cfgname", ["tiny-kquant", "tiny-q8_0"])
def test_prefill_matches_oracle_serial(oracle, cfgname, chunk):
    """40 tokens in one call (chunks of `chunk` tokens, the last one ragged)
    against the oracle's token-serial run: logits, every layer's KV rows,
    tlen, and 6 greedy continuation tokens."""
    cfg = dataclasses.replace(models.CONFIGS[cfgname], max_t=64)
    model, drv, ref = _pair(cfg, oracle)
    L = lib.load()
    L.draco_set_prefill_chunk(chunk)
    ids = np.random.default_rng(7).integers(0, cfg.vocab, 40).astype(np.int32)
    print(f"[prefill] {cfgname} chunk {chunk}", flush=True)
    lg = drv.prefill_chunk(ids, 0).copy()
    lr = _serial_logits(ref, ids, 0)
    assert rel_err(lg, lr) <= 1e-4
    assert drv.tl[0][0] == ref.tl[0][0] == len(ids)
    assert L.draco_state_pull(ct.cast(drv.descs, ct.c_void_p), drv.NL) == 0
    n = len(ids) * cfg.n_kv * cfg.head_dim
    for l in range(cfg.n_layer):
        tol = 1e-5 if l == 0 else 1e-4
        assert rel_err(drv.kc[l][:n], ref.kc[l][:n]) <= tol
        assert rel_err(drv.vc[l][:n], ref.vc[l][:n]) <= tol
    # greedy continuation from the prefilled state, token by token on both
    a, b = [int(np.argmax(lg))], [int(np.argmax(lr))]
    assert a == b
    for s in range(5):
        pos = len(ids) + s
        drv.forward(a[-1], pos)
        ref.forward(b[-1], pos)
        a.append(int(np.argmax(drv.logits_of_x())))
        b.append(int(np.argmax(ref.logits_of_x())))
    assert a == b


def test_prefill_second_call_at_offset(oracle):
    """Two calls (20 tokens, then 17 at pos0 = 20, chunk 8): the second
    chunk's queries attend the first call's cache rows."""
    cfg = dataclasses.replace(models.TINY_K, max_t=64)
    model, drv, ref = _pair(cfg, oracle)
    lib.load().draco_set_prefill_chunk(8)
    ids = np.random.default_rng(11).integers(0, cfg.vocab, 37).astype(np.int32)
    drv.prefill_chunk(ids[:20], 0)
    lg = drv.prefill_chunk(ids[20:], 20).copy()
    lr = _serial_logits(ref, ids, 0)
    assert rel_err(lg, lr) <= 1e-4
    assert drv.tl[-1][0] == 37


@pytest.mark.parametrize("hd,nh,nkv", [(128, 3, 1), (128, 2, 2), (64, 5, 1), (64, 8, 1)])
def test_prefill_head_shapes(oracle, hd, nh, nkv):
    """Head dim 128 and GQA ratios 1, 2(rep 1), 5 and 8 through the chunk
    attention kernel, 48 tokens in chunks of 16 against the oracle."""
    cfg = dataclasses.replace(models.TINY_Q8, name=f"pf-{hd}-{nh}-{nkv}", head_dim=hd, n_head=nh, n_kv=nkv,
                              max_t=128)
    model, drv, ref = _pair(cfg, oracle)
    lib.load().draco_set_prefill_chunk(16)
    ids = np.random.default_rng(13).integers(0, cfg.vocab, 48).astype(np.int32)
    print(f"[prefill] hd {hd} nh {nh} nkv {nkv}", flush=True)
    lg = drv.prefill_chunk(ids, 0).copy()
    lr = _serial_logits(ref, ids, 0)
    assert rel_err(lg, lr) <= 1e-4


@pytest.mark.parametrize("cfgname,fname", [("tiny-kquant", "llama_tiny_k.npz"), ("tiny-q8_0", "llama_tiny_q8.npz")])
def test_generate_token_serial_prompt(cfgname, fname):
    """draco_llama_generate with the chunked prefill switched off feeds the
    prompt token by token (graph-replayed steps): still the golden tokens."""
    g = golden(fname)
    cfg = models.CONFIGS[cfgname]
    model = models.build_llama(cfg, 0)
    L = lib.load()
    L.draco_reset()
    L.draco_set_prefill_chunk(0)
    drv = LlamaDriver(model, hip_engine_lib())
    toks, hidden, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=True)
    assert toks == list(g["tokens"])


def test_llama1b_chunked_matches_serial_device():
    """the 960-token prompt through 256-token chunks against the
    same prompt through token-serial device steps: identical greedy tokens,
    final hidden states within 1e-3."""
    cfg = models.LLAMA1B
    model = models.build_llama(cfg, 0)
    L = lib.load()
    L.draco_reset()
    out = {}
    for chunk in (256, 0):
        L.draco_set_prefill_chunk(chunk)
        drv = LlamaDriver(model, hip_engine_lib())
        drv.reset()
        L.draco_state_push(ct.cast(drv.descs, ct.c_void_p), drv.NL)
        toks, hidden, st = drv.generate_device(model.prompt(), 16, use_graph=True)
        print(f"[prefill] llama1b chunk {chunk}: prefill {st[1]:.1f} ms", flush=True)
        out[chunk] = (toks, hidden.copy())
    assert out[256][0] == out[0][0]
    assert np.max(np.abs(out[256][1] - out[0][1])) <= 1e-3
