"""The benchmark stacks at depth on the GPU, against the compiled reference.

- configs[4]'s 48-layer qwen35 stack (3:1 GDN : full attention, the
  benchmark's own weights) with an 8-token prompt and 8 greedy tokens: the
  reference's per-layer ops composed as src/qwen35_engine.py:310-327 does
  (tests/golden/qwen48_short.npz), compared after every fourth layer of the
  last token, at the end, and through the device-resident greedy loop;
- configs[3]'s first 8 MoE layers (the benchmark's layer weights) with an
  8-token prompt and 8 greedy tokens (tests/golden/moe_stack8.npz), the
  reference engine running its own m6_granite_moe per layer.

Bars: greedy tokens identical; final hidden state within 1e-3 max|diff| (the
north star's bar for the final layer); the per-depth errors are printed so
the growth over 48 layers is on record.
"""
import numpy as np
import pytest

from helpers import golden, rel_err

pytestmark = pytest.mark.gpu
HID_TOL = 1e-3


def test_qwen48_per_layer_ops_by_depth(hip):
    from dracohip import qwen35 as Q
    g = golden("qwen48_short.npz")
    hip.draco_reset()
    cfg = Q.STACKS["qwen35-gdn-stack-48-short"]
    stack = Q.build_stack(cfg, 0)
    drv = Q.QwenStackDriver(stack, Q.hip_ops(hip))
    drv.record = tuple(range(3, 48, 4))
    print("[depth] qwen35 48 layers, per-layer ops", flush=True)
    toks, hidden, lg = drv.greedy(stack.prompt(), cfg.n_gen, collect_logits=(0, 7))
    errs = {il: float(np.max(np.abs(drv.depth[il] - g[f"depth{il}"]))) for il in drv.record}
    print("[depth] max|dh| after layer: " + ", ".join(f"{il + 1}: {e:.2e}" for il, e in errs.items()), flush=True)
    assert toks == list(g["tokens"])
    assert np.max(np.abs(hidden - g["hidden"])) <= HID_TOL
    assert max(errs.values()) <= HID_TOL
    for s in (0, 7):
        top = g[f"logits{s}_top_ids"]
        assert rel_err(lg[s][top], g[f"logits{s}_top_vals"]) <= 1e-4


@pytest.mark.parametrize("use_graph", [True])
def test_qwen48_device_generate(hip, use_graph):
    from dracohip import qwen35 as Q
    g = golden("qwen48_short.npz")
    hip.draco_reset()
    cfg = Q.STACKS["qwen35-gdn-stack-48-short"]
    stack = Q.build_stack(cfg, 0)
    drv = Q.QwenStackDriver(stack, Q.hip_ops(hip), lib=hip)
    print(f"[depth] qwen35 48 layers, device generate graph {use_graph}", flush=True)
    toks, hidden, _ = drv.generate_device(stack.prompt(), cfg.n_gen, use_graph=use_graph)
    print(f"[depth] qwen35 48 layers device loop: final max|dh| {np.max(np.abs(hidden - g['hidden'])):.2e}",
          flush=True)
    assert toks == list(g["tokens"])
    assert np.max(np.abs(hidden - g["hidden"])) <= HID_TOL


@pytest.mark.parametrize("use_graph", [False, True])
def test_moe8_device_generate(hip, use_graph):
    from dracohip import models
    from dracohip.driver import LlamaDriver, hip_engine_lib
    g = golden("moe_stack8.npz")
    hip.draco_reset()
    cfg = models.QWEN3_MOE8
    model = models.build_llama(cfg, 3)
    assert model.digest() == g["digest"].tobytes().hex()
    drv = LlamaDriver(model, hip_engine_lib())
    print(f"[depth] MoE 8 layers, device generate graph {use_graph}", flush=True)
    toks, hidden, _ = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    print(f"[depth] MoE 8 layers: final max|dh| {np.max(np.abs(hidden - g['hidden'])):.2e}", flush=True)
    assert toks == list(g["tokens"])
    assert np.max(np.abs(hidden - g["hidden"])) <= HID_TOL


def test_moe8_dropin_per_token(hip):
    from dracohip import models
    from dracohip.driver import LlamaDriver, hip_engine_lib
    g = golden("moe_stack8.npz")
    hip.draco_reset()
    cfg = models.QWEN3_MOE8
    model = models.build_llama(cfg, 3)
    drv = LlamaDriver(model, hip_engine_lib())
    print("[depth] MoE 8 layers, drop-in per token", flush=True)
    toks, hidden, lg = drv.greedy(model.prompt(), cfg.n_gen, collect_logits=(0, 7))
    assert toks == list(g["tokens"])
    assert np.max(np.abs(hidden - g["hidden"])) <= HID_TOL
    for s in (0, 7):
        top = g[f"logits{s}_top_ids"]
        assert rel_err(lg[s][top], g[f"logits{s}_top_vals"]) <= 1e-4
