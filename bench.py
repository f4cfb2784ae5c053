"""Benchmark: decode tok/s at batch 1, context ~1024, on one MI355X.

Workload: Llama-3.2-1B-shaped decoder, random-init
N(0,0.02) from seed 0, Q4_K_M-style (Q4_K q/k/o/gate/up, Q6_K v/down/tied
head), a 960-token random prompt through the 256-token chunked prefill, then
greedy decode at positions 960..1023.  One "step" is one decode token
(embedding -> 16 layers -> head -> argmax), run by the device-resident loop
(draco_llama_generate, graph-replayed); the prompt is fed before every timed
run and is not part of `value`.  value = timed tokens / timed seconds (HIP
events on the decode stream).  configs2_prefill reports the prompt's chunked
prefill time (and the token-serial time of the same prompt for scale).

roofline: the Q4_K GEMV of configs[1] (W 14336x4096 from seed 1, fp32 x),
one HIP event pair around each graph replay of 200 launches rotating 10
distinct weight copies (330 MB > the 256 MB MALL), the median of five
replays after a warm one.  decode_roofline: the
configs[2] decode's bytes per token x tok/s against the same HBM peak.
Further legs: configs[0], [1], [3] and [4] (see each function).

cpu_baseline: the reference's own C engine (src/m6_engine.c + the scalar
kernels of src/m5_kern_scalar.c, compiled from source into oracle/_ref),
decoding from the same context on this host's cores (all granted, and one),
in a child process; plus the reference's AVX-512 Q4_K row kernel
(src/m5/m5_batch8_k.c) at the configs[1] shapes.

usage: python bench.py [--gpus 1] [--steps 64] [--warmup 8]
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dracomancer-llmengine_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of the roofline kernel from the FETCH_SIZE / WRITE_SIZE
# counter passes (rocprofv3 --pmc, scaled by a device copy of known size:
# 2046.5 B per FETCH_SIZE unit, 1024 B per WRITE_SIZE unit): 16299.2 * 2046.48
# + 56.0 * 1024 bytes (profiles/gemv_q4k_14336x4096_roofline.md)
TRAFFIC_BYTES = 33413287
CTX_START = 960
MAX_DECODE = 64  # positions 960..1023 (max_t 1024)


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def q4k_gemv_roofline(lib, n_copies=10, iters=200):
    """configs[1] Q4_K GEMV 14336x4096, fp32 activations (the decode path's kernel, k_dq).

    Average launch duration = one HIP event pair around a graph replay of
    `iters` launches rotating over `n_copies` weight copies (330 MB > the
    256 MB MALL), so kernels run back to back on the launch stream; the
    median of five replays after a warm one.  The
    other configs[1] shape (4096x14336, fp32 x) is timed the same way and
    reported under "other_shape"; the top-level figures are the 14336x4096
    launch's.
    """
    def one(n_out, n_in):
        rng = np.random.default_rng(1)
        W = lib.quantize(5, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
        out = np.zeros(8, np.float32)
        rc = lib.load().draco_bench_gemv(5, lib.pu8(W), n_out, n_in, n_copies, iters, lib.pf(out))
        if rc != 0:
            raise RuntimeError(lib.last_error())
        us = float(out[4])
        alg_bytes = W.nbytes + 4 * n_in + 4 * n_out  # weights + fp32 x + fp32 y
        return us, alg_bytes, float(out[0])

    us, alg_bytes, us_ev = one(14336, 4096)
    gbs = alg_bytes / us / 1e3
    us2, alg2, _ = one(4096, 14336)
    gbs2 = alg2 / us2 / 1e3
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_BYTES,
            "kernel": "k_dq<8,1,false> (W 14336x4096 Q4_K, fp32 x, 10 rotating copies)",
            "alg_bytes_per_launch": alg_bytes, "us_per_launch": round(us, 3),
            "us_per_launch_event_pairs": round(us_ev, 3),
            "other_shape": {"shape": "4096x14336", "kernel": "k_dq<16,1,false> (W 4096x14336 Q4_K, fp32 x)",
                            "alg_bytes_per_launch": alg2, "us_per_launch": round(us2, 3),
                            "achieved": round(gbs2, 1), "frac": round(gbs2 / PEAK_HBM_GBS, 4)}}


def q8k_gemv_configs1(lib, n_copies=10, iters=200):
    """Q4_K GEMV with on-device Q8_K activations, both FFN shapes, bs1 and bs8.

    Algorithmic bytes per launch = Q4_K weights + Q8_K activation blocks + fp32 y.
    """
    out = {}
    for n_out, n_in in ((14336, 4096), (4096, 14336)):
        rng = np.random.default_rng(1)
        W = lib.quantize(5, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
        for nvec in (1, 8):
            o = np.zeros(4, np.float32)
            rc = lib.load().draco_bench_gemv_q8k(5, lib.pu8(W), n_out, n_in, nvec, n_copies, iters, lib.pf(o))
            if rc != 0:
                raise RuntimeError(lib.last_error())
            alg = W.nbytes + nvec * (n_in // 256) * 292 + 4 * nvec * n_out
            us = float(o[0])
            rec = {"us_per_launch": round(us, 3), "GB_s": round(alg / us / 1e3, 1),
                   "frac_of_peak": round(alg / us / 1e3 / PEAK_HBM_GBS, 4),
                   "us_quantize_plus_gemv": round(float(o[1]), 3), "alg_bytes": alg}
            if nvec == 1 and o[2] > 0:
                # the fp32-x path draco_gemv_q8k_f32 runs for rows up to 4096 wide:
                # one launch that quantizes x itself
                rec["us_fp32_x_fused"] = round(float(o[2]), 3)
            out[f"{n_out}x{n_in}_bs{nvec}"] = rec
    return out


def moe_ffn_configs3(lib, iters=100):
    """configs[3] MoE FFN: hidden 2048, 128 experts (Q4_K gate/up/down, FFN 768), top-8, fp32 router.

    One FFN = router GEMV + routed gate/up (+SwiGLU) + down (+weighted combine),
    timed as a graph replay of `iters` FFNs.  Bytes per FFN = 8 experts' three
    Q4_K matrices + the fp32 router.
    """
    import ctypes as ct
    n_exp, n_used, inter, H = 128, 8, 768, 2048
    rng = np.random.default_rng(3)
    gate_inp = rng.standard_normal((n_exp, H), dtype=np.float32) * np.float32(0.02)
    mats = []
    for rows, cols in ((inter, H), (inter, H), (H, inter)):
        chunks = [lib.quantize(5, rng.standard_normal((16 * rows, cols), dtype=np.float32) * np.float32(0.02))
                  for _ in range(n_exp // 16)]
        mats.append(np.concatenate(chunks))
    per = [m.nbytes // n_exp for m in mats]
    ptrs = np.zeros(3 * n_exp, np.uint64)
    codes = np.full(3 * n_exp, 5, np.int32)
    for e in range(n_exp):
        for k in range(3):
            ptrs[3 * e + k] = mats[k].ctypes.data + e * per[k]
    x = rng.standard_normal(H).astype(np.float32)
    o = np.zeros(4, np.float32)
    rc = lib.load().draco_bench_granite_moe(lib.pf(x), ct.c_void_p(ptrs.ctypes.data), lib.pi32(codes),
                                           lib.pf(gate_inp), n_exp, n_used, inter, H, H, iters, lib.pf(o))
    if rc != 0:
        raise RuntimeError(lib.last_error())
    lib.load().draco_reset()
    us, nbytes = float(o[0]), float(o[1])
    return {"us_per_ffn": round(us, 3), "bytes_per_ffn": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
            "frac_of_peak": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
            "shape": "128 experts top-8, FFN 768, hidden 2048, Q4_K experts, fp32 router"}


def shexp_qwen35moe(lib, iters=200, n_copies=160):
    """qwen35moe shared expert (m6_granite_shexp) at hidden 2048, FFN 512: Q4_K
    gate/up, Q6_K down, fp32 gate row.  One call = gate/up (+SwiGLU), down, and
    the gate row's dot with the sigmoid scale (three launches), graph-replayed with the weights rotated over
    n_copies device copies (~2.05 MB each, 330 MB in all: past the MALL)."""
    import ctypes as ct
    shi, H = 512, 2048
    rng = np.random.default_rng(5)
    ws = [lib.quantize(5, rng.standard_normal((shi, H), dtype=np.float32) * np.float32(0.02)),
          lib.quantize(5, rng.standard_normal((shi, H), dtype=np.float32) * np.float32(0.02)),
          lib.quantize(4, rng.standard_normal((H, shi), dtype=np.float32) * np.float32(0.02)),
          (rng.standard_normal(H, dtype=np.float32) * np.float32(0.02)).view(np.uint8)]
    ptrs = np.array([w.ctypes.data for w in ws], np.uint64)
    codes = np.array([5, 5, 4, 9], np.int32)
    x = rng.standard_normal(H).astype(np.float32)
    o = np.zeros(2, np.float32)
    rc = lib.load().draco_bench_shexp(lib.pf(x), ct.c_void_p(ptrs.ctypes.data), lib.pi32(codes), shi, H, n_copies,
                                      iters, lib.pf(o))
    if rc != 0:
        raise RuntimeError(lib.last_error())
    lib.load().draco_reset()
    us, nbytes = float(o[0]), float(o[1])
    return {"us_per_call": round(us, 3), "bytes_per_call": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
            "frac_of_peak": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "launches": 3,
            "shape": "shared expert FFN 512, hidden 2048, Q4_K gate/up, Q6_K down, fp32 gate row"}


def gdn_scan_configs4(lib):
    """configs[4] GDN scan: 32 V heads / 16 q-k heads of 128, T = 4096 scanned in 64-token
    launches, then 64 single-token (decode) steps; us per token, state bytes per token."""
    T, n_vh, nhq = 4096, 32, 16
    n_qkv = n_vh * 128 + 2 * nhq * 128
    rng = np.random.default_rng(4)
    QKV = rng.standard_normal((T, n_qkv), dtype=np.float32)
    Z = rng.standard_normal((T, n_vh * 128), dtype=np.float32)
    B = (1.0 / (1.0 + np.exp(-rng.standard_normal((T, n_vh))))).astype(np.float32)
    G = np.exp(-np.logaddexp(0.0, rng.standard_normal((T, n_vh)))).astype(np.float32)
    conv = rng.standard_normal((n_qkv, 4), dtype=np.float32) * np.float32(0.5)
    ssm_norm = np.ones(128, np.float32)
    tail = np.zeros(n_qkv * 3, np.float32)
    S = np.zeros(n_vh * 128 * 128, np.float32)
    o = np.zeros(4, np.float32)
    rc = lib.load().draco_bench_gdn_scan(lib.pf(QKV), lib.pf(Z), lib.pf(B), lib.pf(G), lib.pf(conv),
                                         lib.pf(ssm_norm), lib.pf(tail), lib.pf(S), T, n_qkv, n_vh, 64, 64,
                                         lib.pf(o))
    if rc != 0:
        raise RuntimeError(lib.last_error())
    return {"us_per_token_prefill_64chunks": round(float(o[0]), 3), "us_per_decode_step": round(float(o[1]), 3),
            "prefill_tok_s_one_layer": round(1e6 / float(o[0]), 1),
            "shape": "32 V heads, 16 q/k heads, head 128, T 4096 in 64-token launches + 64 decode steps"}


def qwen35_ops_configs4(lib, told=4096, iters=50):
    """configs[4] hybrid stack, one decode token per layer kind: the GDN layer op
    (m6_gdn_attn: qkv+gate GEMVs, gates, conv, delta rule on the 32x128x128
    state, gated rms, ssm_out GEMV + residual, post-norm) and the full-attention
    op (m6_full_attn: q+gate/k/v GEMVs, q/k norm + rope, attention over `told`
    cached rows + the new one, sigmoid gate, o GEMV + residual, post-norm), Q4_K
    projections (v in Q6_K), graph replay with device-resident state."""
    from dracohip import qwen35 as Q
    L = lib.load()
    h1 = Q.hidden(5)[0]
    out = np.zeros(4, np.float32)
    res = {}
    G = Q.gdn_layer(81, 32, (5, 5, 5))
    if L.draco_bench_qwen_op(0, G.ptr(), lib.pf(h1), lib.pf(G.ssm), lib.pf(G.tail), 0, iters, lib.pf(out)):
        raise RuntimeError(lib.last_error())
    res["gdn_op"] = {"us_per_token": round(float(out[0]), 3), "bytes_per_token": int(out[2]),
                     "GB_s": round(float(out[2]) / float(out[0]) / 1e3, 1),
                     "frac_of_peak": round(float(out[2]) / float(out[0]) / 1e3 / PEAK_HBM_GBS, 4)}
    F = Q.full_layer(82, 16, (5, 5, 4, 5))
    Kr, Vc = Q.kv_rows(83, told)
    if L.draco_bench_qwen_op(1, F.ptr(), lib.pf(h1), lib.pf(Kr), lib.pf(Vc), told, iters, lib.pf(out)):
        raise RuntimeError(lib.last_error())
    res["full_attn_op"] = {"us_per_token": round(float(out[0]), 3), "bytes_per_token": int(out[2]),
                           "cached_rows": told, "GB_s": round(float(out[2]) / float(out[0]) / 1e3, 1),
                           "frac_of_peak": round(float(out[2]) / float(out[0]) / 1e3 / PEAK_HBM_GBS, 4)}
    res["shape"] = ("GDN: 16 q/k + 32 V heads of 128, n_qkv 8192, hidden 2048; full attention: 16 q heads, "
                    "2 KV heads of 256, hidden 2048")
    return res


def llama_bytes_per_token(model, first_pos, n_gen):
    """Algorithmic HBM bytes of one decode token of a llama-family model: every
    layer matrix and the head once, one embedding row, and the K / V rows read
    (mean over positions first_pos .. first_pos + n_gen - 1, rows 0..pos)."""
    cfg = model.cfg
    T = model.tensors
    layers = sum(v[0].nbytes for k, v in T.items() if k.startswith("blk."))
    head = model.head()[0].nbytes
    emb_row = T["token_embd.weight"][0].nbytes // cfg.vocab
    rows = np.arange(first_pos, first_pos + n_gen) + 1
    kv = cfg.n_layer * 2 * cfg.n_kv * cfg.head_dim * 4 * float(rows.mean())
    return layers + head + emb_row + kv


def smol_decode_configs0(lib, use_graph=True):
    """SmolLM2-360M-shaped Q8_0, 32-token prompt + 64 greedy tokens
    on the device loop (graph-replayed); tokens checked against the reference
    golden; tok/s and GB/s against the HBM roof."""
    import ctypes as ct
    from dracohip import models
    from dracohip.driver import LlamaDriver, hip_engine_lib
    cfg = models.SMOL360M
    model = models.build_llama(cfg, 0)
    L = lib.load()
    drv = LlamaDriver(model, hip_engine_lib())
    drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    drv.reset()
    L.draco_state_push(ct.cast(drv.descs, ct.c_void_p), drv.NL)
    toks, _, (dec_ms, _) = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    gpath = os.path.join(ROOT, "tests", "golden", "smol360m.npz")
    match = bool(list(np.load(gpath)["tokens"]) == toks) if os.path.exists(gpath) else None
    per_tok = llama_bytes_per_token(model, cfg.n_prompt - 1, cfg.n_gen)
    tok_s = cfg.n_gen / (dec_ms / 1e3)
    res = {"tok_s": round(tok_s, 1), "ms_per_token": round(dec_ms / cfg.n_gen, 4), "bytes_per_token": int(per_tok),
           "GB_s": round(per_tok * tok_s / 1e9, 1), "frac_of_peak": round(per_tok * tok_s / 1e9 / PEAK_HBM_GBS, 4),
           "roof_tok_s": round(PEAK_HBM_GBS * 1e9 / per_tok, 1), "greedy_tokens_match_reference": match,
           "shape": "SmolLM2-360M: hidden 960, 32 layers, 15/5 x 64, FFN 2560, vocab 49152, all Q8_0; "
                    "32-token prompt, 64 greedy tokens"}
    del drv, model
    L.draco_reset()
    return res


def moe_stack_configs3(lib, seed=3, use_graph=True):
    """the 48-layer Qwen3-30B-A3B-shaped MoE stack (attention 32 q /
    4 kv heads of 128, Q6_K; MoE FFN 128 experts, top 8, FFN 768, Q4_K experts,
    fp32 router) decoding at context 512: a 448-token prompt fed token by token
    through the graph-replayed decode step, then 64 greedy tokens (positions
    448..511) timed with HIP events.  Bytes per token = attention weights +
    the 8 routed experts' three matrices + the router, per layer, + the K/V rows
    read (mean over the decode positions) + the head and one embedding row."""
    import ctypes as ct
    from dracohip import models
    from dracohip.driver import LlamaDriver, hip_engine_lib
    cfg = models.QWEN3_MOE
    t0 = time.time()
    model = models.build_llama(cfg, seed)
    log(f"configs[3] model built in {time.time() - t0:.1f}s ({model.nbytes() / 1e9:.2f} GB)")
    L = lib.load()
    drv = LlamaDriver(model, hip_engine_lib())
    t0 = time.time()
    toks, _, (dec_ms, pre_ms) = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    log(f"configs[3] first run (upload + prompt + decode) {time.time() - t0:.1f}s")
    drv.reset()
    L.draco_state_push(ct.cast(drv.descs, ct.c_void_p), drv.NL)
    toks2, _, (dec_ms, pre_ms) = drv.generate_device(model.prompt(), cfg.n_gen, use_graph=use_graph)
    T = model.tensors
    H, E, F, KD = cfg.hidden, cfg.n_exp, cfg.exp_ff, cfg.n_kv * cfg.head_dim
    attn = sum(T[f"blk.0.{n}.weight"][0].nbytes for n in ("attn_q", "attn_k", "attn_v", "attn_output"))
    experts = sum(T[f"blk.0.{n}.weight"][0].nbytes // E for n in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"))
    router = E * H * 4
    # decode step i runs at tlen n_prompt - 1 + i and reads that many rows + its own
    rows = np.arange(cfg.n_prompt - 1, cfg.n_prompt - 1 + cfg.n_gen) + 1
    kv = 2 * KD * 4 * float(rows.mean())
    head = model.head()[0].nbytes
    emb_row = T["token_embd.weight"][0].nbytes // cfg.vocab
    per_tok = cfg.n_layer * (attn + cfg.n_used * experts + router + kv) + head + emb_row
    stack = cfg.n_layer * (attn + cfg.n_used * experts + router + kv)
    tok_s = cfg.n_gen / (dec_ms / 1e3)
    res = {"tok_s": round(tok_s, 1), "ms_per_token": round(dec_ms / cfg.n_gen, 4),
           "bytes_per_token": int(per_tok), "GB_s": round(per_tok * tok_s / 1e9, 1),
           "frac_of_peak": round(per_tok * tok_s / 1e9 / PEAK_HBM_GBS, 4),
           "stack_bytes_per_token_no_head": int(stack), "roof_tok_s": round(PEAK_HBM_GBS * 1e9 / per_tok, 1),
           "prompt_tokens": cfg.n_prompt, "prompt_ms_token_serial": round(pre_ms, 1),
           "greedy_tokens_repeat": toks == toks2,
           "shape": "48 layers: attention 32q/4kv x 128 Q6_K + MoE 128 experts top-8 FFN 768 Q4_K, fp32 router; "
                    "hidden 2048, vocab 151936 (untied Q6_K head), decode at positions 448..511"}
    del drv, model
    L.draco_reset()
    return res


def qwen_stack_configs4(lib, seed=4, use_graph=True):
    """the 48-layer qwen35 hybrid stack (36 GDN layers of 16 q/k
    and 32 V heads of 128, 12 full-attention layers of 16 q / 2 KV heads of
    256, 3:1 interleave, Q4_K projections, hidden 2048): a 4096-token prompt,
    all but its last token through the chunked prefill in 64-token chunks, then
    64 greedy decode steps (positions 4095..4158), graph-replayed.  Bytes per
    decode token = every layer's projection weights + the GDN state read and
    written + the beta / alpha rows + the full-attention K / V rows read (mean
    over the decode positions) + the head and one embedding row."""
    import ctypes as ct
    from dracohip import qwen35 as Q
    cfg = Q.QWEN35_GDN48
    t0 = time.time()
    stack = Q.build_stack(cfg, seed)
    log(f"configs[4] stack built in {time.time() - t0:.1f}s ({stack.nbytes() / 1e9:.2f} GB)")
    L = lib.load()
    drv = Q.QwenStackDriver(stack, Q.hip_ops(L), lib=L)
    old = L.draco_set_qwen_chunk(64)
    prompt = stack.prompt()
    t0 = time.time()
    toks, _, _ = drv.generate_device(prompt, cfg.n_gen, use_graph=use_graph)
    log(f"configs[4] first run (upload + prompt + decode) {time.time() - t0:.1f}s")
    drv.reset()
    toks2, _, (dec_ms, pre_ms) = drv.generate_device(prompt, cfg.n_gen, use_graph=use_graph)
    L.draco_set_qwen_chunk(old)
    gdn_w = full_w = 0
    for il, layer in enumerate(stack.layers):
        a = layer.arrays
        if isinstance(layer, Q.FullLayer):
            full_w += a["q"].nbytes + a["k"].nbytes + a["v"].nbytes + a["o"].nbytes
        else:
            gdn_w += a["qkv"].nbytes + a["gate"].nbytes + a["ssm_out"].nbytes
    n_gdn = sum(1 for layer in stack.layers if isinstance(layer, Q.GdnLayer))
    n_full = cfg.n_layer - n_gdn
    n_qkv = 2 * Q.NKH * Q.SV + cfg.n_vh * Q.SV
    gdn_state = n_gdn * (2 * cfg.n_vh * Q.SV * Q.SV * 4 + 2 * Q.H * cfg.n_vh * 4 + 2 * n_qkv * 3 * 4 + n_qkv * 16)
    rows = np.arange(cfg.n_prompt - 1, cfg.n_prompt - 1 + cfg.n_gen) + 1
    kv = n_full * 2 * Q.NKV_A * Q.HD_A * 4 * float(rows.mean())
    per_tok = gdn_w + full_w + gdn_state + kv + stack.head.nbytes + stack.emb.nbytes // cfg.vocab
    tok_s = cfg.n_gen / (dec_ms / 1e3)
    n_pre = len(prompt) - 1
    res = {"decode_tok_s": round(tok_s, 1), "ms_per_token": round(dec_ms / cfg.n_gen, 4),
           "bytes_per_token": int(per_tok), "GB_s": round(per_tok * tok_s / 1e9, 1),
           "frac_of_peak": round(per_tok * tok_s / 1e9 / PEAK_HBM_GBS, 4),
           "roof_tok_s": round(PEAK_HBM_GBS * 1e9 / per_tok, 1),
           "prefill_tokens": n_pre, "prefill_chunk": 64, "prefill_ms": round(pre_ms, 1),
           "prefill_tok_s": round(n_pre / (pre_ms / 1e3), 1), "greedy_tokens_repeat": toks == toks2,
           "shape": "48 layers 3:1 GDN (16 q/k + 32 V heads of 128) : full attention (16 q / 2 kv heads of 256), "
                    "Q4_K projections, hidden 2048, no FFN (the configuration's mixers), vocab 151936 untied Q6_K "
                    "head; 4095-token chunked prefill, decode at positions 4095..4158"}
    del drv, stack
    L.draco_reset()
    return res


PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16 MFMA


def prefill_gemm_configs2(lib, T=256, n_copies=4, iters=20):
    """configs[2] chunked prefill: one 256-token chunk through a Llama-1B layer's seven projections.

    fp32-equivalent TFLOP/s = 2*T*n_out*n_in / time.  The f16 MFMA work issued
    is 2x that for Q4_K (hi and lo halves of x; plus 1/8 for the min term on a
    K-padded 16-slot MFMA) and 4x for Q6_K (hi/lo x the two scale parts);
    `mfma_util` = issued f16 MFMA flops / (time * 2.5 PFLOP/s dense f16).
    """
    shapes = [("q", 5, 2048, 2048), ("k", 5, 512, 2048), ("v", 4, 512, 2048), ("o", 5, 2048, 2048),
              ("gate", 5, 8192, 2048), ("up", 5, 8192, 2048), ("down", 4, 2048, 8192)]
    rng = np.random.default_rng(2)
    res, tot_us, tot_flop, tot_i8 = {}, 0.0, 0.0, 0.0
    for name, code, n_out, n_in in shapes:
        W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
        o = np.zeros(4, np.float32)
        rc = lib.load().draco_bench_gemm(code, lib.pu8(W), n_out, n_in, T, n_copies, iters, lib.pf(o))
        if rc != 0:
            raise RuntimeError(lib.last_error())
        us = float(o[0])
        flop = 2.0 * T * n_out * n_in
        i8 = flop * (2.0 * 34.0 / 32.0 if code == 5 else 4.0)
        res[name] = {"us": round(us, 2), "us_kernel_only": round(float(o[1]), 2),
                     "tflops_fp32_equiv": round(flop / us / 1e6, 1)}
        tot_us += us
        tot_flop += flop
        tot_i8 += i8
    return {"tokens": T, "us_per_layer_chunk": round(tot_us, 1),
            "tflops_fp32_equiv": round(tot_flop / tot_us / 1e6, 1),
            "mfma_util": round(tot_i8 / tot_us / 1e6 / PEAK_F16_TFLOPS, 4),
            "prefill_tok_s_16_layers": round(T / (16 * tot_us * 1e-6), 1), "per_matrix": res}


def cpu_baseline_worker(args):
    """Child process: the reference engine decoding from context CTX_START."""
    from dracohip import models
    from dracohip.driver import EngineLib, LlamaDriver
    from oracle.oracle import REF_DIR
    import ctypes as ct
    cfg = models.LLAMA1B
    model = models.build_llama(cfg, 0)
    E = ct.CDLL(os.path.join(REF_DIR, "libref_engine.so"))
    E.m6_init_dl.argtypes = [ct.c_char_p] * 5
    sp = os.path.join(REF_DIR, "libref_scalar.so").encode()
    assert E.m6_init_dl(sp, sp, sp, sp, sp) == 0
    drv = LlamaDriver(model, EngineLib(E, name="ref"))
    kv = np.load(args.kv_file)
    for l in range(cfg.n_layer):
        drv.kc[l][:] = kv[f"k{l}"]
        drv.vc[l][:] = kv[f"v{l}"]
        drv.tl[l][0] = CTX_START
    tok = int(kv["next_token"])
    t0 = time.time()
    n = 0
    while n < args.cpu_tokens and (time.time() - t0) < args.cpu_seconds:
        drv.forward(tok, CTX_START + n)
        tok = int(np.argmax(drv.logits_of_x().astype(np.float64)))
        n += 1
    dt = time.time() - t0
    print(json.dumps({"tokens": n, "seconds": dt, "threads": int(os.environ.get("OMP_NUM_THREADS", "0"))}))


def cpu_gemv_worker(args):
    """Child process: the reference's AVX-512 Q4_K row kernel (m5_gemvn_q4k,
    src/m5/m5_batch8_k.c:80-114, compiled from source into oracle/_ref) on the
    configs[1] shapes at batch 1.  Its row loop ignores the row-block bounds
    it is handed (every OpenMP unit would recompute all rows), so the matrix
    is passed as 64-row slices, one slice per "expert" with x shared: each
    unit computes its own 64 rows once.  Weights rotate over copies totalling
    more than any host L3; median of 15 timed calls after 5 warm-ups."""
    import ctypes as ct
    from dracohip import lib
    from oracle.oracle import REF_DIR
    B = ct.CDLL(os.path.join(REF_DIR, "libref_batch8k.so"))
    fn = B.m5_gemvn_q4k
    fn.restype = ct.c_int
    fn.argtypes = [ct.c_void_p, ct.c_long, ct.c_void_p, ct.c_void_p, ct.c_long, ct.c_int, ct.c_int, ct.c_int,
                   ct.c_void_p]
    out = {}
    for n_out, n_in in ((14336, 4096), (4096, 14336)):
        rng = np.random.default_rng(1)
        W = lib.quantize(5, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
        copies = [W] + [W.copy() for _ in range(11)]  # 12 x 33 MB
        x = rng.standard_normal(n_in).astype(np.float32)
        y = np.zeros(n_out, np.float32)
        rows = 64
        idx = np.arange(n_out // rows, dtype=np.int32)
        per = rows * (n_in // 256) * 144
        times = []
        for i in range(20):
            w = copies[i % len(copies)]
            t0 = time.perf_counter()
            rc = fn(x.ctypes.data, 0, w.ctypes.data, idx.ctypes.data, per, rows, n_in, len(idx), y.ctypes.data)
            dt = time.perf_counter() - t0
            assert rc == 0
            if i >= 5:
                times.append(dt)
        t = float(np.median(times))
        out[f"{n_out}x{n_in}"] = {"us": round(t * 1e6, 1), "GB_s": round(W.nbytes / t / 1e9, 2)}
    print(json.dumps(out))


def cpu_host_info():
    """The host the CPU baseline ran on: core counts, the CPU's identification
    fields as /proc/cpuinfo gives them (the model-name string of a virtualised
    host can be as short as "AMD EPYC", so family / model / stepping and the
    vector extensions the reference's kernels use are recorded too), the
    sockets and the frequency governor."""
    info = {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        fields, sockets = {}, set()
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "physical id":
                    sockets.add(v)
                if k in ("model name", "vendor_id", "cpu family", "model", "stepping", "cpu MHz", "flags") \
                        and k not in fields:
                    fields[k] = v
        info["cpu_model"] = fields.get("model name")
        info["cpu_id"] = {k: fields.get(k) for k in ("vendor_id", "cpu family", "model", "stepping", "cpu MHz")}
        flags = set(fields.get("flags", "").split())
        info["cpu_vector_ext"] = sorted(x for x in flags if x.startswith(("avx512", "avx2", "fma", "f16c")))
        info["sockets"] = len(sockets) or None
    except OSError:
        pass
    for path in ("/sys/devices/system/cpu/cpu0/cpufreq/scaling_governor",):
        try:
            with open(path) as f:
                info["governor"] = f.read().strip()
        except OSError:
            info["governor"] = "unavailable"
    return info


def run_cpu_gemv(threads):
    env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="false")
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-gemv-worker"]
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        log("cpu gemv baseline failed:", r.stderr[-2000:])
        return None
    return json.loads(r.stdout.strip().splitlines()[-1])


def run_cpu_baseline(drv, cfg, first_token, threads, cpu_tokens, cpu_seconds):
    """Pull the GPU's KV at context CTX_START and time the reference engine from there."""
    import ctypes as ct
    from dracohip import lib
    lib.load().draco_state_pull(ct.cast(drv.descs, ct.c_void_p), drv.NL)
    n = CTX_START * cfg.n_kv * cfg.head_dim
    fd, path = tempfile.mkstemp(suffix=".npz", dir="/dev/shm" if os.path.isdir("/dev/shm") else None)
    os.close(fd)
    try:
        arrs = {f"k{l}": drv.kc[l].copy() for l in range(cfg.n_layer)}
        arrs.update({f"v{l}": drv.vc[l].copy() for l in range(cfg.n_layer)})
        for l in range(cfg.n_layer):
            arrs[f"k{l}"][n:] = 0
            arrs[f"v{l}"][n:] = 0
        np.savez(path, next_token=np.int64(first_token), **arrs)
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="false")
        cmd = [sys.executable, os.path.abspath(__file__), "--cpu-baseline-worker", "--kv-file", path,
               "--cpu-tokens", str(cpu_tokens), "--cpu-seconds", str(cpu_seconds)]
        r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            log("cpu baseline failed:", r.stderr[-2000:])
            return None
        res = json.loads(r.stdout.strip().splitlines()[-1])
    finally:
        os.unlink(path)
    return {"value": round(res["tokens"] / res["seconds"], 3), "unit": "tok/s", "cores": threads,
            "kind": "reference",
            "sample": f"{res['tokens']} greedy decode tokens of the same model from context {CTX_START} "
                      f"(KV taken from the GPU prefill), reference m6_engine.c + m5_kern_scalar.c "
                      f"(scalar kernels: the AVX-512 m5_kern*.so are not in the reference tree), "
                      f"{res['seconds']:.1f}s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-tokens", type=int, default=48)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--eager", action="store_true",
                    help="run the decode loop without HIP graphs (for profilers that cannot trace graphs)")
    ap.add_argument("--roofline-only", action="store_true", help="only the Q4_K GEMV roofline measurement")
    ap.add_argument("--no-roofline", action="store_true", help="skip the GEMV roofline measurement (profiling runs)")
    ap.add_argument("--no-stacks", action="store_true", help="skip the configs[0] / [3] / [4] decode legs")
    ap.add_argument("--no-serial-prefill", action="store_true",
                    help="skip the token-serial prompt run (the chunked prefill is the measured one)")
    ap.add_argument("--leg", choices=["configs0", "configs3", "configs4"],
                    help="run only this decode leg and print its record (profiling runs)")
    ap.add_argument("--cpu-baseline-worker", action="store_true")
    ap.add_argument("--cpu-gemv-worker", action="store_true")
    ap.add_argument("--kv-file")
    args = ap.parse_args()
    if args.cpu_baseline_worker:
        return cpu_baseline_worker(args)
    if args.cpu_gemv_worker:
        return cpu_gemv_worker(args)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on exactly one GPU (--gpus 1); multi-GPU runs are not part "
              "of it", file=sys.stderr)
        sys.exit(2)

    import ctypes as ct
    from dracohip import lib, models
    from dracohip.driver import LlamaDriver, hip_engine_lib

    if args.leg:
        fn = {"configs0": smol_decode_configs0, "configs3": moe_stack_configs3, "configs4": qwen_stack_configs4}
        res = fn[args.leg](lib, use_graph=not args.eager)
        log(f"{args.leg}: {res}")
        print(json.dumps({args.leg: res}), flush=True)
        return

    if args.roofline_only:
        roof = q4k_gemv_roofline(lib)
        log(f"Q4_K GEMV 14336x4096: {roof['us_per_launch']} us/launch, {roof['achieved']} GB/s; 4096x14336: "
            f"{roof['other_shape']['us_per_launch']} us/launch, {roof['other_shape']['achieved']} GB/s")
        q8 = q8k_gemv_configs1(lib)
        for k, v in q8.items():
            log(f"Q4_K x Q8_K GEMV {k}: {v['us_per_launch']} us, {v['GB_s']} GB/s")
        moe = moe_ffn_configs3(lib)
        log(f"MoE FFN configs[3]: {moe['us_per_ffn']} us, {moe['GB_s']} GB/s")
        shx = shexp_qwen35moe(lib)
        log(f"qwen35moe shared expert: {shx['us_per_call']} us, {shx['GB_s']} GB/s")
        gdn = gdn_scan_configs4(lib)
        log(f"GDN scan configs[4]: {gdn['us_per_token_prefill_64chunks']} us/token (64-token launches), "
            f"{gdn['us_per_decode_step']} us/decode step")
        pre = prefill_gemm_configs2(lib)
        log(f"prefill GEMM configs[2] (256-token chunk, one layer): {pre['us_per_layer_chunk']} us, "
            f"{pre['tflops_fp32_equiv']} TFLOP/s fp32-equiv, f16 MFMA util {pre['mfma_util']}")
        qw = qwen35_ops_configs4(lib)
        log(f"qwen35 ops configs[4]: GDN layer {qw['gdn_op']['us_per_token']} us/token, full attention "
            f"{qw['full_attn_op']['us_per_token']} us/token at 4096 cached rows")
        print(json.dumps({"roofline": roof, "configs1_q8k_gemv": q8, "configs3_moe_ffn": moe,
                          "configs4_gdn_scan": gdn, "configs4_layer_ops": qw,
                          "configs2_prefill_gemm": pre}), flush=True)
        return

    cfg = models.LLAMA1B
    t0 = time.time()
    model = models.build_llama(cfg, 0)
    prompt = model.prompt()
    log(f"model {cfg.name} built in {time.time() - t0:.1f}s ({model.nbytes() / 1e6:.1f} MB)")
    L = lib.load()
    drv = LlamaDriver(model, hip_engine_lib())

    def run(n_tok):
        drv.reset()
        L.draco_state_push(ct.cast(drv.descs, ct.c_void_p), drv.NL)
        return drv.generate_device(prompt, n_tok, use_graph=not args.eager)

    if args.warmup > 0:
        run(min(args.warmup, MAX_DECODE))
        log(f"warmup {args.warmup} decode steps done")
    left, ms, toks_first, pre_list = args.steps, 0.0, None, []
    while left > 0:
        k = min(left, MAX_DECODE)
        toks, hidden, (dec_ms, pre_ms) = run(k)
        if toks_first is None:
            toks_first = toks
        ms += dec_ms
        pre_list.append(pre_ms)
        left -= k
        log(f"timed {k} decode steps: {dec_ms:.2f} ms (prefill {pre_ms:.1f} ms)")
    tok_s = args.steps / (ms / 1e3)
    # the prompt (all but its last token, which the first decode step takes)
    # through the 256-token chunked prefill, and once token by token for scale
    n_pre = len(prompt) - 1
    chunk = L.draco_set_prefill_chunk(-1)
    serial_ms = None
    if not args.no_serial_prefill:
        L.draco_set_prefill_chunk(0)
        _, _, (_, serial_ms) = run(1)
        L.draco_set_prefill_chunk(chunk)
    pre_ms = float(np.median(pre_list))
    prefill = {"prompt_tokens": n_pre, "chunk": chunk, "ms": round(pre_ms, 3),
               "tok_s": round(n_pre / (pre_ms / 1e3), 1),
               "token_serial_ms": round(serial_ms, 3) if serial_ms else None,
               "token_serial_tok_s": round(n_pre / (serial_ms / 1e3), 1) if serial_ms else None}
    log(f"prefill {n_pre} tokens: chunked {pre_ms:.1f} ms, token-serial {serial_ms} ms")
    match = None
    gpath = os.path.join(ROOT, "tests", "golden", "llama1b.npz")
    if os.path.exists(gpath):
        g = np.load(gpath)
        n = min(len(toks_first), len(g["tokens"]))
        match = bool(list(g["tokens"][:n]) == toks_first[:n])
    log(f"decode {tok_s:.1f} tok/s; greedy tokens match reference: {match}")
    # the decode path against the HBM roof: algorithmic bytes of one token
    # (every weight once, one embedding row, the K / V rows read) x tok/s
    per_tok = llama_bytes_per_token(model, CTX_START - 1, min(args.steps, MAX_DECODE))
    decode_roof = {"bound": "hbm", "bytes_per_token": int(per_tok), "achieved_GB_s": round(per_tok * tok_s / 1e9, 1),
                   "peak_GB_s": PEAK_HBM_GBS, "frac": round(per_tok * tok_s / 1e9 / PEAK_HBM_GBS, 4),
                   "roof_tok_s": round(PEAK_HBM_GBS * 1e9 / per_tok, 1)}

    roof = q8 = moe = shx = gdn = pre = qw = None
    if not args.no_roofline:
        roof = q4k_gemv_roofline(lib)
        log(f"Q4_K GEMV 14336x4096: {roof['us_per_launch']} us/launch, {roof['achieved']} GB/s; 4096x14336: "
            f"{roof['other_shape']['us_per_launch']} us/launch, {roof['other_shape']['achieved']} GB/s")
        q8 = q8k_gemv_configs1(lib)
        for k, v in q8.items():
            log(f"Q4_K x Q8_K GEMV {k}: {v['us_per_launch']} us, {v['GB_s']} GB/s")
        moe = moe_ffn_configs3(lib)
        log(f"MoE FFN configs[3]: {moe['us_per_ffn']} us, {moe['GB_s']} GB/s")
        shx = shexp_qwen35moe(lib)
        log(f"qwen35moe shared expert: {shx['us_per_call']} us, {shx['GB_s']} GB/s")
        gdn = gdn_scan_configs4(lib)
        log(f"GDN scan configs[4]: {gdn['us_per_token_prefill_64chunks']} us/token (64-token launches), "
            f"{gdn['us_per_decode_step']} us/decode step")
        pre = prefill_gemm_configs2(lib)
        log(f"prefill GEMM configs[2] (256-token chunk, one layer): {pre['us_per_layer_chunk']} us, "
            f"{pre['tflops_fp32_equiv']} TFLOP/s fp32-equiv, f16 MFMA util {pre['mfma_util']}")
        qw = qwen35_ops_configs4(lib)
        log(f"qwen35 ops configs[4]: GDN layer {qw['gdn_op']['us_per_token']} us/token, full attention "
            f"{qw['full_attn_op']['us_per_token']} us/token at 4096 cached rows")

    cpu = None
    if not args.no_cpu_baseline:
        # all the cores this process may use (the GPU box grants 16), and one
        threads = args.cpu_threads or min(16, len(os.sched_getaffinity(0)) or 1)
        # first decode token after the prompt: feed it through the CPU engine from CTX_START
        run(1)
        cpu = run_cpu_baseline(drv, cfg, toks_first[0], threads, args.cpu_tokens, args.cpu_seconds)
        if cpu:
            log(f"cpu baseline {cpu['value']} tok/s on {threads} threads")
            one = run_cpu_baseline(drv, cfg, toks_first[0], 1, args.cpu_tokens, args.cpu_seconds / 2)
            if one:
                cpu["one_thread"] = {"value": one["value"], "unit": "tok/s", "sample": one["sample"]}
                log(f"cpu baseline {one['value']} tok/s on 1 thread")
            gemv = {f"threads_{t}": run_cpu_gemv(t) for t in (threads, 1)}
            cpu["gemv_q4k_avx512_bs1"] = gemv
            cpu["host"] = cpu_host_info()
            log(f"cpu AVX-512 Q4_K GEMV: {gemv}")

    moe_stack = qwen_stack = smol = None
    if not args.no_stacks:
        smol = smol_decode_configs0(lib, use_graph=not args.eager)
        log(f"configs[0] SmolLM2-360M decode: {smol['tok_s']} tok/s ({smol['frac_of_peak']} of peak), tokens match "
            f"reference: {smol['greedy_tokens_match_reference']}")
        moe_stack = moe_stack_configs3(lib, use_graph=not args.eager)
        log(f"configs[3] MoE stack: {moe_stack['tok_s']} tok/s, {moe_stack['GB_s']} GB/s "
            f"({moe_stack['frac_of_peak']} of peak)")
        qwen_stack = qwen_stack_configs4(lib, use_graph=not args.eager)
        log(f"configs[4] qwen35 stack: decode {qwen_stack['decode_tok_s']} tok/s ({qwen_stack['frac_of_peak']} of "
            f"peak), prefill {qwen_stack['prefill_tok_s']} tok/s")

    line = {
        "metric": "decode tok/s bs1 @ctx1024; Q4_K GEMV achieved HBM GB/s as % of peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32 activations x Q4_K/Q6_K weights",
        "data": "synthetic: random-init N(0,0.02) weights from seed 0, random prompt ids",
        "config": {"workload": "configs[2] llama-3.2-1b-shaped Q4_K_M decode, bs1, 960-token prompt, "
                               "positions 960..1023", "global_batch": 1, "seq_len": 1024,
                   "parallelism": "single GPU"},
        "greedy_tokens_match_reference": match,
        "decode_roofline": decode_roof,
        "configs0_decode": smol,
        "configs2_prefill": prefill,
        "roofline": roof,
        "configs1_q8k_gemv": q8,
        "configs3_moe_ffn": moe,
        "qwen35moe_shared_expert": shx,
        "configs4_gdn_scan": gdn,
        "configs4_layer_ops": qw,
        "configs2_prefill_gemm": pre,
        "configs3_moe_stack": moe_stack,
        "configs4_qwen_stack": qwen_stack,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
