"""ctypes binding of the CPU checker libraries.

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product path never does.

  Oracle()      liboracle.so, this build's C restatement (draco_oracle.c)
  Ref(name)     oracle/_ref/libref_<name>.so, the reference's own C compiled
                from its sources (present only where oracle/Makefile 'ref' ran)
"""
import ctypes as ct
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")

f32p = ct.POINTER(ct.c_float)
u8p = ct.POINTER(ct.c_uint8)
i32p = ct.POINTER(ct.c_int)


def pf(a):
    return a.ctypes.data_as(f32p)


def pu8(a):
    return a.ctypes.data_as(u8p)


def pi32(a):
    return a.ctypes.data_as(i32p)


_SIGS = {
    "or_f16": (ct.c_float, [ct.c_uint16]),
    "or_rowbytes": (ct.c_size_t, [ct.c_int, ct.c_int]),
    "or_supported": (ct.c_int, [ct.c_int]),
    "or_gemv": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, f32p]),
    "or_gemv_range": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, f32p, ct.c_int, ct.c_int]),
    "or_dequant_row": (ct.c_int, [ct.c_int, u8p, ct.c_int, f32p]),
    "or_rms_norm": (None, [f32p, f32p, ct.c_int, ct.c_float, f32p]),
    "or_forward_token": (ct.c_int, [f32p, ct.c_int, ct.c_float, ct.c_int, ct.c_void_p, ct.c_int, f32p]),
    "or_head_op": (ct.c_int, [f32p, f32p, ct.c_int, ct.c_float, u8p, ct.c_int, ct.c_int, f32p, f32p]),
    "or_argmax": (ct.c_int, [f32p, ct.c_int]),
    "or_llama_attn_op": (None, [f32p, ct.c_void_p, ct.c_int, f32p]),
    "or_dense_op": (None, [f32p, ct.c_void_p, f32p]),
    "or_moe_ffn_op": (None, [f32p, ct.c_void_p, f32p]),
    "or_topk": (None, [f32p, ct.c_int, ct.c_int, i32p]),
    "or_moe_route": (None, [f32p, f32p, ct.c_int, ct.c_int, ct.c_int, f32p, i32p, f32p]),
    "or_granite_moe": (None, [f32p, ct.c_void_p, i32p, f32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int,
                              ct.c_int, f32p, f32p]),
    "or_granite_shexp": (None, [f32p, ct.c_void_p, i32p, f32p, f32p, f32p, f32p, ct.c_int, ct.c_int]),
    "or_gdn_scan": (None, [f32p, f32p, f32p, f32p, f32p, f32p, f32p, f32p, ct.c_int, ct.c_int,
                           ct.c_int, f32p, f32p]),
    "or_moe_tok": (None, [f32p, i32p, f32p, ct.c_void_p, i32p, ct.c_int, ct.c_int, ct.c_int,
                          ct.c_int, ct.c_int, ct.c_int, f32p]),
    "or_gdn_attn": (ct.c_int, [f32p, ct.c_void_p, f32p, f32p, f32p, f32p]),
    "or_full_attn": (ct.c_int, [f32p, ct.c_void_p, f32p, f32p, ct.c_int, ct.c_int, f32p, f32p, f32p, f32p]),
    "or_gemm": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "or_gemvn_q4k": (ct.c_int, [f32p, ct.c_long, u8p, i32p, ct.c_long, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "or_gemvn_q6k": (ct.c_int, [f32p, ct.c_long, u8p, i32p, ct.c_long, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "or_quantize_q8k": (None, [f32p, ct.c_int, u8p]),
    "or_q8k_block_isums": (None, [ct.c_int, u8p, u8p, i32p, i32p]),
    "or_gemv_q8k": (ct.c_int, [ct.c_int, u8p, u8p, ct.c_int, ct.c_int, f32p]),
    "or_gemm_q8k": (ct.c_int, [ct.c_int, u8p, u8p, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "or_set_threads": (None, [ct.c_int]),
    "or_get_threads": (ct.c_int, []),
}


class Oracle:
    def __init__(self, path=None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        self.lib = ct.CDLL(path)
        for n, (r, a) in _SIGS.items():
            f = getattr(self.lib, n)
            f.restype = r
            f.argtypes = a
        self.path = path
        # op function pointers usable inside descriptor arrays
        self.attn_op = ct.cast(self.lib.or_llama_attn_op, ct.c_void_p).value
        self.dense_op = ct.cast(self.lib.or_dense_op, ct.c_void_p).value
        self.moe_op = ct.cast(self.lib.or_moe_ffn_op, ct.c_void_p).value

    def gemv(self, code, x, W, n_out, n_in):
        y = np.zeros(n_out, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        rc = self.lib.or_gemv(code, pf(x), pu8(W), n_out, n_in, pf(y))
        assert rc == 0, rc
        return y

    def gemv_range(self, code, x, W, n_out, n_in, o0, o1, y=None):
        y = np.zeros(n_out, np.float32) if y is None else y
        rc = self.lib.or_gemv_range(code, pf(np.ascontiguousarray(x, np.float32)), pu8(W), n_out, n_in,
                                    pf(y), o0, o1)
        assert rc == 0, rc
        return y

    def dequant(self, code, W, n_out, n_in):
        rb = self.lib.or_rowbytes(code, n_in)
        out = np.zeros((n_out, n_in), np.float32)
        for r in range(n_out):
            rc = self.lib.or_dequant_row(code, pu8(W[r * rb:(r + 1) * rb]), n_in, pf(out[r]))
            assert rc == 0
        return out

    def quantize_q8k(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros((x.size // 256) * 292, np.uint8)
        self.lib.or_quantize_q8k(pf(x), x.size, pu8(out))
        return out

    def gemv_q8k(self, code, xq, W, n_out, n_in):
        y = np.zeros(n_out, np.float32)
        rc = self.lib.or_gemv_q8k(code, pu8(xq), pu8(W), n_out, n_in, pf(y))
        assert rc == 0, rc
        return y


def ref_available(name="scalar"):
    return os.path.exists(os.path.join(REF_DIR, f"libref_{name}.so"))


class Ref:
    """The reference's own compiled C (oracle/_ref)."""

    def __init__(self, name):
        path = os.path.join(REF_DIR, f"libref_{name}.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle ref` where the reference tree exists")
        self.lib = ct.CDLL(path)
        self.path = path
