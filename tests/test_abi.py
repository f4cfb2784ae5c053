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
