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
