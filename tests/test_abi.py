"""The C-ABI library loads and exports every symbol include/*.h declares.

CPU only: loading the library does not touch the GPU, and no compute entry
point is called here.
"""
import ctypes as ct
import glob
import os
import re

from helpers import ROOT


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"typedef[^;]*;", "", src)  # function-pointer typedefs are not exports
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z][a-z0-9_]*)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_reference_entry_points():
    names = declared_symbols()
    for n in ("m5_gemv", "m5_gemv_range", "m5_scalar_supported"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from dracohip import lib
    L = lib.load()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(L, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from dracohip import lib
    declared = declared_symbols()
    assert set(lib.SIGNATURES) <= declared


# Every m5_* / m6_* symbol the reference's drivers and engine bind by name,
# with the restype / argtypes they set (file:line of the binding).  With
# M6_SO / the kernel-slot paths pointed at this library, each lookup must
# resolve.  m5_gemv13_segs (src/k2_engine.py:118, the IQ2_S segment kernel of
# the K2 driver) is not listed: that driver guards it with `except
# AttributeError` and IQ2_S is not carried here.
_f = ct.POINTER(ct.c_float)
_u8 = ct.POINTER(ct.c_uint8)
_i = ct.POINTER(ct.c_int)
_FUSED = [_f, _u8, ct.c_int, ct.c_int, ct.c_int, _f]
REFERENCE_BINDINGS = [
    ("src/smol_engine.py:66", "m6_init_dl", ct.c_int, [ct.c_char_p] * 5),
    ("src/smol_engine.py:67", "m6_init_extra_dl", ct.c_int, [ct.c_char_p]),
    ("src/smol_engine.py:73", "m6_rms_norm", None, [_f, _f, ct.c_int, ct.c_float, _f]),
    ("src/smol_engine.py:75", "m6_engine_version", ct.c_char_p, []),
    ("src/smol_engine.py:76", "m6_forward_token", ct.c_int, [_f, ct.c_int, ct.c_float, ct.c_int, ct.c_void_p,
                                                             ct.c_int, _f]),
    ("src/smol_engine.py:78", "m6_head_op", ct.c_int, [_f, _f, ct.c_int, ct.c_float, ct.c_void_p, ct.c_int,
                                                       ct.c_int, _f, _f]),
    # (the driver's argtypes list has one pointer too many and one too few
    # against the C signature, src/m6_layer.c:656-658; only the lookup at
    # import matters to it: it never calls the op)
    ("src/smol_engine.py:81", "m6_moe_batch4", None, [ct.c_void_p] * 5 + [ct.c_int] * 4 + [ct.c_void_p]),
    ("src/smol_engine.py:92", "m5_gemv", ct.c_int, [ct.c_int, _f, _u8, ct.c_int, ct.c_int, _f]),
    ("src/smol_engine.py:117", "m6_llama_attn_op", None, None),
    ("src/smol_engine.py:118", "m6_dense_op", None, None),
    ("src/m6_layer.c:130", "m5_gemv_range", ct.c_int, [ct.c_int, _f, _u8, ct.c_int, ct.c_int, _f, ct.c_int,
                                                        ct.c_int]),
    ("src/qwen35_engine.py:103", "m6_init_iq3_dl", ct.c_int, [ct.c_char_p]),
    ("src/qwen35_engine.py:108", "m6_gdn_attn", None, [_f, ct.c_void_p] + [_f] * 5),
    ("src/qwen35_engine.py:112", "m6_full_attn", None, [_f, ct.c_void_p, _f, _f, ct.c_int, ct.c_int] + [_f] * 6),
    ("src/qwen35_engine.py:118", "m6_granite_shexp", None, [_f, ct.POINTER(ct.c_uint64), _i, _f, _f, _f, _f,
                                                            ct.c_int, ct.c_int]),
    ("src/qwen35_engine.py:122", "m6_granite_moe", None, [_f, ct.POINTER(ct.c_uint64), _i, _f] + [ct.c_int] * 5
     + [_f, _f]),
    ("src/qwen35_prefill.py:66", "m5_gemm", ct.c_int, [ct.c_int, ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int,
                                                       ct.c_int, ct.c_void_p, ct.c_void_p]),
    ("src/qwen35_prefill.py:71", "m6_moe_tok", None, [ct.c_void_p] * 8 + [ct.c_int] * 6 + [ct.c_void_p] * 3),
    ("src/qwen35_prefill.py:73", "m5_dequant_row", None, None),
    ("src/qwen35_prefill.py:75", "m5_gemm_auto", ct.c_int, [ct.c_int] + [ct.c_void_p] * 2 + [ct.c_int] * 3
     + [ct.c_void_p]),
    ("src/qwen35_prefill.py:78", "m5_gemm_q80", None, _FUSED),
    ("src/qwen35_prefill.py:78", "m5_gemm_iq3s", None, _FUSED),
    ("src/qwen35_prefill.py:79", "m5_gemm_q5k", None, _FUSED),
    ("src/qwen35_prefill.py:79", "m5_gemm_q6k", None, _FUSED),
    ("src/qwen35_prefill.py:80", "m5_gemm_q4k", None, _FUSED),
    ("src/qwen35_prefill.py:80", "m5_gemm_iq4xs", None, _FUSED),
    ("src/qwen35_prefill.py:84", "m6_gdn_scan", None, [ct.c_void_p] * 8 + [ct.c_int] * 3 + [ct.c_void_p] * 2),
    ("src/k2_engine.py:101", "m5_gemvn_q4k", ct.c_int, [_f, ct.c_long, _u8, _i, ct.c_long, ct.c_int, ct.c_int,
                                                        ct.c_int, _f]),
    ("src/k2_engine.py:101", "m5_gemvn_q6k", ct.c_int, [_f, ct.c_long, _u8, _i, ct.c_long, ct.c_int, ct.c_int,
                                                        ct.c_int, _f]),
]


def test_reference_drivers_bind_unchanged():
    """A fresh handle on the library (as the reference's drivers open it)
    resolves every name they bind and takes their argtypes; the op pointers
    they take with ct.cast (src/smol_engine.py:117-118) are non-null."""
    from dracohip import lib
    L = ct.CDLL(lib.LIB_PATH)
    missing = []
    for where, name, res, args in REFERENCE_BINDINGS:
        if not hasattr(L, name):
            missing.append((name, where))
            continue
        fn = getattr(L, name)
        if args is not None:
            fn.restype = res
            fn.argtypes = args
        assert ct.cast(fn, ct.c_void_p).value, name
    assert not missing, missing
    declared = declared_symbols()
    assert {n for _, n, _, _ in REFERENCE_BINDINGS} <= declared
