"""ctypes binding of libdraco_hip.so (the HIP product library).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere on the product path.
"""
import ctypes as ct
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("DRACO_HIP_SO", os.path.join(PKG, "lib", "libdraco_hip.so"))

f32p = ct.POINTER(ct.c_float)
u8p = ct.POINTER(ct.c_uint8)
i32p = ct.POINTER(ct.c_int)

_LIB = None


def pf(a):
    return a.ctypes.data_as(f32p)


def pu8(a):
    return a.ctypes.data_as(u8p)


def pi32(a):
    return a.ctypes.data_as(i32p)


def vp(a):
    return ct.c_void_p(a.ctypes.data)


# name -> (restype, argtypes).  Mirrors include/draco_hip.h.
SIGNATURES = {
    # m5 kernel-library ABI (src/m5_kern_scalar.c:146-165)
    "m5_scalar_supported": (ct.c_int, [ct.c_int]),
    "m5_gemv": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, f32p]),
    "m5_gemv_range": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, f32p, ct.c_int, ct.c_int]),
    # m6 layer-engine ABI (src/m6_engine.c)
    "m6_rms_norm": (None, [f32p, f32p, ct.c_int, ct.c_float, f32p]),
    "m6_rowbytes": (ct.c_size_t, [ct.c_int, ct.c_int]),
    "m6_engine_version": (ct.c_char_p, []),
    "m6_init_dl": (ct.c_int, [ct.c_char_p] * 5),
    "m6_init_extra_dl": (ct.c_int, [ct.c_char_p]),
    "m6_init_iq3_dl": (ct.c_int, [ct.c_char_p]),
    "m6_forward_token": (ct.c_int, [f32p, ct.c_int, ct.c_float, ct.c_int, ct.c_void_p, ct.c_int, f32p]),
    "m6_head_op": (ct.c_int, [f32p, f32p, ct.c_int, ct.c_float, ct.c_void_p, ct.c_int, ct.c_int, f32p, f32p]),
    "m6_llama_attn_op": (None, [f32p, ct.c_void_p, ct.c_int, f32p]),
    "m6_dense_op": (None, [f32p, ct.c_void_p, f32p]),
    "m6_granite_shexp": (None, [f32p, ct.c_void_p, i32p, f32p, f32p, f32p, f32p, ct.c_int, ct.c_int]),
    "draco_bench_shexp": (ct.c_int, [f32p, ct.c_void_p, i32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "draco_state_pull": (ct.c_int, [ct.c_void_p, ct.c_int]),
    "draco_state_push": (ct.c_int, [ct.c_void_p, ct.c_int]),
    "draco_llama_generate": (ct.c_int, [ct.c_void_p, ct.c_int, ct.c_int, ct.c_float, f32p, ct.c_void_p,
                                        ct.c_int, ct.c_int, ct.c_void_p, ct.c_int, i32p, ct.c_int, ct.c_int,
                                        ct.c_int, i32p, f32p, f32p]),
    "draco_set_prefill_chunk": (ct.c_int, [ct.c_int]),
    "draco_set_attn_o_fusion": (ct.c_int, [ct.c_int]),
    "draco_set_moe_split": (ct.c_int, [ct.c_int]),
    "draco_set_attn_short": (ct.c_int, [ct.c_int]),
    "draco_set_gqa_waves": (ct.c_int, [ct.c_int]),
    "draco_set_seg_rows": (ct.c_int, [ct.c_int]),
    "draco_set_gdn_dec": (ct.c_int, [ct.c_int]),
    "draco_llama_prefill": (ct.c_int, [ct.c_void_p, ct.c_int, ct.c_int, ct.c_float, ct.c_void_p, ct.c_int, ct.c_int,
                                       i32p, ct.c_int, ct.c_int, f32p]),
    # qwen35 hybrid layers (src/m6_layer.c:189-518)
    "m6_gdn_attn": (None, [f32p, ct.c_void_p, f32p, f32p, f32p, f32p, f32p]),
    "m6_full_attn": (None, [f32p, ct.c_void_p, f32p, f32p, ct.c_int, ct.c_int, f32p, f32p, f32p, f32p,
                            f32p, f32p]),
    "draco_bench_qwen_op": (ct.c_int, [ct.c_int, ct.c_void_p, f32p, f32p, f32p, ct.c_int, ct.c_int, f32p]),
    "draco_array_pull": (ct.c_int, [ct.c_void_p, ct.c_size_t]),
    "draco_array_push": (ct.c_int, [ct.c_void_p, ct.c_size_t]),
    # qwen35 hybrid stack on the device (no reference counterpart as one call)
    "draco_qwen_forward": (ct.c_int, [f32p, ct.c_int, ct.c_int, ct.c_void_p, ct.c_int]),
    "draco_qwen_prefill": (ct.c_int, [ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p, ct.c_int, ct.c_int, i32p, ct.c_int,
                                      ct.c_int, f32p]),
    "draco_set_qwen_chunk": (ct.c_int, [ct.c_int]),
    "draco_set_gdn_split": (ct.c_int, [ct.c_int, ct.c_int]),
    "draco_qwen_generate": (ct.c_int, [ct.c_void_p, ct.c_int, ct.c_int, ct.c_float, f32p, ct.c_void_p, ct.c_int,
                                       ct.c_int, ct.c_void_p, ct.c_int, ct.c_int, i32p, ct.c_int, ct.c_int, ct.c_int,
                                       i32p, f32p, f32p]),
    "draco_qwen_state_pull": (ct.c_int, [ct.c_void_p, ct.c_int, ct.c_int]),
    "draco_qwen_state_push": (ct.c_int, [ct.c_void_p, ct.c_int, ct.c_int]),
    "draco_moe_ffn_op": (None, [f32p, ct.c_void_p, f32p]),
    # library utilities
    "draco_last_error": (ct.c_char_p, []),
    "draco_forget": (ct.c_int, [ct.c_void_p]),
    "draco_reset": (None, []),
    "draco_resident_bytes": (ct.c_size_t, []),
    "draco_version": (ct.c_char_p, []),
    "draco_bench_gemv": (ct.c_int, [ct.c_int, u8p, ct.c_int, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "draco_bench_launch": (ct.c_int, [ct.c_int, f32p]),
    "draco_dq_plan": (ct.c_int, [ct.c_int] * 7 + [i32p]),
    # MoE (src/m6_layer.c:771-802, src/m5/m5_batch8_k.c:80-183)
    "m6_granite_moe": (None, [f32p, ct.c_void_p, i32p, f32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int, ct.c_int,
                              f32p, f32p]),
    "m6_moe_tok": (None, [ct.c_void_p, ct.c_void_p, f32p, f32p, i32p, f32p, ct.c_void_p, i32p] + [ct.c_int] * 6
                   + [f32p, f32p, i32p]),
    "m5_gemvn_q4k": (ct.c_int, [f32p, ct.c_long, u8p, i32p, ct.c_long, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "m6_moe_batch4": (None, [f32p, ct.c_void_p, i32p, f32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int, f32p, f32p]),
    "m5_gemvn_q6k": (ct.c_int, [f32p, ct.c_long, u8p, i32p, ct.c_long, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "draco_bench_granite_moe": (ct.c_int, [f32p, ct.c_void_p, i32p, f32p, ct.c_int, ct.c_int, ct.c_int, ct.c_int,
                                           ct.c_int, ct.c_int, f32p]),
    # prefill GEMM (src/m5/m5_gemm_fused.c:231-241, src/m5/m5_gemm.c:249-272)
    "m5_gemm_auto": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "m5_gemm": (ct.c_int, [ct.c_int, f32p, u8p, ct.c_int, ct.c_int, ct.c_int, f32p, f32p]),
    "m5_dequant_row": (ct.c_int, [ct.c_int, u8p, ct.c_int, f32p]),
    **{f"m5_gemm_{f}": (None, [f32p, u8p, ct.c_int, ct.c_int, ct.c_int, f32p])
       for f in ("q80", "q6k", "q5k", "q4k", "iq4xs", "iq3s")},
    "draco_bench_gemm": (ct.c_int, [ct.c_int, u8p, ct.c_int, ct.c_int, ct.c_int, ct.c_int, ct.c_int, f32p]),
    # Gated-DeltaNet scan (src/m6_gdn_scan.c:18-93)
    "m6_gdn_scan": (None, [f32p] * 8 + [ct.c_int] * 3 + [f32p, f32p]),
    "draco_bench_gdn_scan": (ct.c_int, [f32p] * 8 + [ct.c_int] * 5 + [f32p]),
    # Q8_K activations (no reference counterpart)
    "draco_q8k_quantize": (ct.c_int, [f32p, ct.c_int, ct.c_int, u8p]),
    "draco_gemv_q8k": (ct.c_int, [ct.c_int, u8p, ct.c_int, u8p, ct.c_int, ct.c_int, f32p]),
    "draco_gemv_q8k_f32": (ct.c_int, [ct.c_int, f32p, ct.c_int, u8p, ct.c_int, ct.c_int, f32p]),
    "draco_q8k_isums": (ct.c_int, [ct.c_int, u8p, u8p, ct.c_int, ct.c_int, i32p, i32p]),
    "draco_bench_gemv_q8k": (ct.c_int, [ct.c_int, u8p, ct.c_int, ct.c_int, ct.c_int, ct.c_int, ct.c_int, f32p]),
    "draco_gemv_q8k_f32_noalloc": (ct.c_int, [ct.c_int, ct.c_void_p, ct.c_int, ct.c_void_p, ct.c_int, ct.c_int,
                                              ct.c_void_p, ct.c_void_p]),
    "draco_noalloc_capacity": (ct.c_size_t, []),
    "draco_quantize": (ct.c_int, [ct.c_int, f32p, ct.c_int, ct.c_int, u8p]),
    "draco_layout_query": (ct.c_size_t, [ct.c_int, ct.c_int, ct.c_int, ct.POINTER(ct.c_size_t)]),
    "draco_repack": (ct.c_int, [ct.c_int, u8p, ct.c_int, ct.c_int, u8p]),
    "draco_unpack": (ct.c_int, [ct.c_int, u8p, ct.c_int, ct.c_int, u8p]),
    "draco_rope_table": (None, [ct.c_int, ct.c_int, ct.c_float, f32p]),
    "draco_f16_to_f32": (ct.c_float, [ct.c_uint16]),
    "draco_f32_to_f16": (ct.c_uint16, [ct.c_float]),
}


def load():
    """Return the loaded library (cached).  Raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libdraco_hip.so not built at {LIB_PATH}: run __graft_entry__.build()")
    lib = ct.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def last_error():
    return load().draco_last_error().decode(errors="replace")


def check(rc, what="call"):
    if rc != 0:
        raise RuntimeError(f"{what} failed rc={rc}: {last_error()}")
    return rc


def quantize(code, x):
    """Encode a 2-D float32 array into GGUF rows of `code` (0 Q8_0, 4 Q6_K, 5 Q4_K)."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    n_rows, n_in = x.shape
    out = np.empty(n_rows * row_bytes(code, n_in), np.uint8)
    check(load().draco_quantize(code, pf(x), n_rows, n_in, pu8(out)), "draco_quantize")
    return out


def row_bytes(code, n_in):
    return {0: (n_in // 32) * 34, 3: (n_in // 256) * 176, 4: (n_in // 256) * 210,
            5: (n_in // 256) * 144, 7: n_in * 2, 9: n_in * 4}[code]


def gemv(code, x, W, n_out, n_in, o0=None, o1=None):
    """Host-pointer m5_gemv / m5_gemv_range through the C ABI; returns y."""
    lib = load()
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(n_out, np.float32)
    if o0 is None:
        rc = lib.m5_gemv(code, pf(x), pu8(W), n_out, n_in, pf(y))
    else:
        rc = lib.m5_gemv_range(code, pf(x), pu8(W), n_out, n_in, pf(y), o0, o1)
    check(rc, "m5_gemv")
    return y
