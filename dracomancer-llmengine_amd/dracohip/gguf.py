"""Read-only GGUF reader (mmap, zero-copy tensor views) and a GGUF writer.

The reader keeps the interface subset of the reference's `FastGGUF`
(src/gguf_fast.py:167-370): `FastGGUF(path)` (cached per (path, size, mtime)),
`.fields` (name -> `FastField` with `.contents()`), `.tensors` (`FastTensor`:
name, tensor_type (with `.name`), shape (ne[0] first), n_elements, n_bytes,
data_offset, `.data` zero-copy view, `.raw_bytes()`), `get_field`,
`get_tensor`, `tensor(name)`, `tensor_bytes(name)`, `close()`, and `load()`.
The reference takes its type tables from gguf-py (llama.cpp b10819), which
is not available here; the tables below are the GGUF file format's own
(value types 0..12, ggml type ids, block sizes), for the types the engine
and its tests touch.

The writer produces GGUF version 3 files (little endian, data aligned to
`general.alignment`, default 32): it is what turns the synthetic models into
on-disk models, so the load path from a file is exercised end to end.
"""
from __future__ import annotations

import enum
import mmap as _mmap
import os
import struct
import sys
from collections import OrderedDict

import numpy as np

__all__ = ["FastGGUF", "FastTensor", "FastField", "GGUFValueType", "GGMLQuantizationType", "load", "write_gguf",
           "M5_CODE", "GGML_OF_M5"]

GGUF_DEFAULT_ALIGNMENT = 32
GGML_MAX_DIMS = 4


class GGUFValueType(enum.IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


class GGMLQuantizationType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1_M = 29
    BF16 = 30


# (values per block, bytes per block)
GGML_QUANT_SIZES = {
    GGMLQuantizationType.F32: (1, 4), GGMLQuantizationType.F16: (1, 2), GGMLQuantizationType.BF16: (1, 2),
    GGMLQuantizationType.F64: (1, 8), GGMLQuantizationType.I8: (1, 1), GGMLQuantizationType.I16: (1, 2),
    GGMLQuantizationType.I32: (1, 4), GGMLQuantizationType.I64: (1, 8),
    GGMLQuantizationType.Q4_0: (32, 18), GGMLQuantizationType.Q4_1: (32, 20),
    GGMLQuantizationType.Q5_0: (32, 22), GGMLQuantizationType.Q5_1: (32, 24),
    GGMLQuantizationType.Q8_0: (32, 34), GGMLQuantizationType.Q8_1: (32, 36),
    GGMLQuantizationType.Q2_K: (256, 84), GGMLQuantizationType.Q3_K: (256, 110),
    GGMLQuantizationType.Q4_K: (256, 144), GGMLQuantizationType.Q5_K: (256, 176),
    GGMLQuantizationType.Q6_K: (256, 210), GGMLQuantizationType.Q8_K: (256, 292),
    GGMLQuantizationType.IQ4_NL: (32, 18), GGMLQuantizationType.IQ4_XS: (256, 136),
    GGMLQuantizationType.IQ3_S: (256, 110), GGMLQuantizationType.IQ2_S: (256, 82),
}

# ggml type name -> the engine's format code (src/smol_engine.py:46-47, plus F32 = 9)
M5_CODE = {"Q8_0": 0, "IQ4_NL": 1, "IQ3_S": 2, "Q5_K": 3, "Q6_K": 4, "Q4_K": 5, "IQ4_XS": 6, "F16": 7, "Q5_0": 8,
           "F32": 9}
GGML_OF_M5 = {c: GGMLQuantizationType[n] for n, c in M5_CODE.items()}

_SCALAR = {
    GGUFValueType.UINT8: ("B", np.uint8, 1), GGUFValueType.INT8: ("b", np.int8, 1),
    GGUFValueType.UINT16: ("H", np.uint16, 2), GGUFValueType.INT16: ("h", np.int16, 2),
    GGUFValueType.UINT32: ("I", np.uint32, 4), GGUFValueType.INT32: ("i", np.int32, 4),
    GGUFValueType.FLOAT32: ("f", np.float32, 4), GGUFValueType.BOOL: ("B", np.uint8, 1),
    GGUFValueType.UINT64: ("Q", np.uint64, 8), GGUFValueType.INT64: ("q", np.int64, 8),
    GGUFValueType.FLOAT64: ("d", np.float64, 8),
}
_ITEM = {
    GGMLQuantizationType.F16: np.float16, GGMLQuantizationType.F32: np.float32, GGMLQuantizationType.F64: np.float64,
    GGMLQuantizationType.I8: np.int8, GGMLQuantizationType.I16: np.int16, GGMLQuantizationType.I32: np.int32,
    GGMLQuantizationType.I64: np.int64,
}

_CACHE: dict = {}


class FastField:
    """One metadata key: `contents()` gives a str, a Python scalar, or a list
    (arrays of strings or of numbers), as the reference's reader does."""

    __slots__ = ("offset", "name", "value", "types")

    def __init__(self, offset, name, value, types):
        self.offset, self.name, self.value, self.types = offset, name, value, types

    def contents(self, index_or_slice=slice(None)):
        v = self.value
        if isinstance(v, list):
            return v[index_or_slice] if isinstance(index_or_slice, int) else list(v[index_or_slice])
        if isinstance(v, np.ndarray):
            return v.tolist()[index_or_slice]
        return v

    def __repr__(self):
        return f"FastField({self.name!r})"


class FastTensor:
    """A tensor of the file: `.data` is a read-only view of the mapping
    (quantized types as uint8 [rows, row bytes], float/int types in their
    dtype, numpy shape = reversed GGUF dims)."""

    __slots__ = ("name", "tensor_type", "shape", "n_elements", "n_bytes", "data_offset", "data", "_mm")

    def __init__(self, name, tensor_type, dims, mm, data_off_abs, n_elements, n_bytes):
        self.name = name
        self.tensor_type = tensor_type
        self.shape = dims
        self.n_elements = n_elements
        self.n_bytes = n_bytes
        self.data_offset = data_off_abs
        self._mm = mm
        np_dims = tuple(int(d) for d in reversed(dims.tolist()))
        item = _ITEM.get(tensor_type)
        if item is not None:
            self.data = np.frombuffer(mm, dtype=item, count=n_elements, offset=data_off_abs).reshape(np_dims)
        else:
            bs, ts = GGML_QUANT_SIZES[tensor_type]
            byte_shape = np_dims[:-1] + (np_dims[-1] // bs * ts,)
            self.data = np.frombuffer(mm, dtype=np.uint8, count=n_bytes, offset=data_off_abs).reshape(byte_shape)

    def raw_bytes(self):
        return memoryview(self._mm)[self.data_offset:self.data_offset + self.n_bytes]

    def __repr__(self):
        return f"FastTensor({self.name!r}, {self.tensor_type.name}, {tuple(self.shape.tolist())})"


class FastGGUF:
    """Read-only, zero-copy, cached per file (path, size, mtime)."""

    def __new__(cls, path, mode="r"):
        key = os.path.abspath(os.fspath(path))
        st = os.stat(key)
        sig = (st.st_size, st.st_mtime_ns)
        hit = _CACHE.get(key)
        if hit is not None and hit._sig == sig:
            return hit
        obj = super().__new__(cls)
        obj._key, obj._sig = key, sig
        _CACHE[key] = obj
        return obj

    def __init__(self, path, mode="r"):
        if getattr(self, "_ready", False):
            return
        if sys.byteorder != "little":
            raise RuntimeError("GGUF reader: little-endian hosts only")
        self.path = self._key
        self.fields: "OrderedDict[str, FastField]" = OrderedDict()
        self.tensors: list = []
        self._fd = os.open(self.path, os.O_RDONLY)
        try:
            self._mm = _mmap.mmap(self._fd, 0, access=_mmap.ACCESS_READ)
        except ValueError:
            os.close(self._fd)
            _CACHE.pop(self._key, None)
            raise ValueError(f"not a GGUF file (empty): {self.path}")
        self.data = np.frombuffer(self._mm, dtype=np.uint8)
        try:
            self._parse()
        except Exception:
            self.data = None
            self.tensors, self.fields = [], OrderedDict()
            try:
                self._mm.close()
            except BufferError:  # views held by the traceback: the mapping goes with them
                pass
            os.close(self._fd)
            _CACHE.pop(self._key, None)
            raise
        self._ready = True

    def _need(self, o, n):
        if o + n > len(self._mm):
            raise ValueError(f"GGUF file truncated at byte {o} (needs {n} more): {self.path}")

    def _u32(self, o):
        self._need(o, 4)
        return struct.unpack_from("<I", self._mm, o)[0]

    def _u64(self, o):
        self._need(o, 8)
        return struct.unpack_from("<Q", self._mm, o)[0]

    def _str(self, o):
        n = self._u64(o)
        self._need(o + 8, n)
        return o + 8 + n, self._mm[o + 8:o + 8 + n].decode("utf-8", "replace")

    def _value(self, o, t):
        t = GGUFValueType(t)
        if t == GGUFValueType.STRING:
            o, s = self._str(o)
            return o, s, [t]
        if t == GGUFValueType.ARRAY:
            it = GGUFValueType(self._u32(o))
            cnt = self._u64(o + 4)
            o += 12
            if it == GGUFValueType.STRING:
                vals = []
                for _ in range(cnt):
                    o, s = self._str(o)
                    vals.append(s)
                return o, vals, [t, it]
            if it == GGUFValueType.ARRAY:
                raise ValueError("nested GGUF arrays are not supported")
            _, dt, sz = _SCALAR[it]
            self._need(o, cnt * sz)
            return o + cnt * sz, np.frombuffer(self._mm, dtype=dt, count=cnt, offset=o), [t, it]
        fmt, _, sz = _SCALAR[t]
        self._need(o, sz)
        return o + sz, struct.unpack_from("<" + fmt, self._mm, o)[0], [t]

    def _parse(self):
        if len(self._mm) < 24 or self._mm[:4] != b"GGUF":
            raise ValueError(f"not a GGUF file: {self.path}")
        ver = self._u32(4)
        if ver not in (2, 3):
            raise ValueError(f"unsupported GGUF version {ver} (2 and 3 are read)")
        self.version = ver
        self.tensor_count, self.kv_count = self._u64(8), self._u64(16)
        o = 24
        for _ in range(self.kv_count):
            start = o
            o, k = self._str(o)
            rt = self._u32(o)
            o, v, chain = self._value(o + 4, rt)
            self.fields[k] = FastField(start, k, v, chain)
        infos = []
        for _ in range(self.tensor_count):
            o, name = self._str(o)
            nd = self._u32(o)
            o += 4
            if nd > GGML_MAX_DIMS:
                raise ValueError(f"tensor {name}: {nd} dimensions (at most {GGML_MAX_DIMS})")
            self._need(o, 8 * nd)
            dims = np.frombuffer(self._mm, dtype=np.uint64, count=nd, offset=o).copy()
            o += 8 * nd
            raw_type = self._u32(o)
            t_off = self._u64(o + 4)
            o += 12
            infos.append((name, dims, raw_type, t_off))
        al = self.fields.get("general.alignment")
        self.alignment = int(al.value) if al is not None else GGUF_DEFAULT_ALIGNMENT
        if self.alignment == 0 or (self.alignment & (self.alignment - 1)):
            raise ValueError(f"invalid alignment {self.alignment}")
        if o % self.alignment:
            o += self.alignment - o % self.alignment
        self.data_offset = o
        seen = set()
        for name, dims, raw_type, t_off in infos:
            if name in seen:
                raise ValueError(f"duplicate tensor name {name}")
            seen.add(name)
            gt = GGMLQuantizationType(raw_type)
            n_el = 1
            for d in dims.tolist():
                n_el *= int(d)
            bs, ts = GGML_QUANT_SIZES[gt]
            if dims.size and int(dims[0]) % bs:
                raise ValueError(f"tensor {name}: row of {int(dims[0])} values is not a whole number of blocks")
            n_bytes = n_el // bs * ts
            abs_off = o + t_off
            if abs_off + n_bytes > len(self._mm):
                raise ValueError(f"tensor {name}: data ({n_bytes} bytes at {abs_off}) past the end of the file")
            self.tensors.append(FastTensor(name, gt, dims, self._mm, abs_off, n_el, n_bytes))
        self._by_name = {t.name: t for t in self.tensors}

    def get_field(self, key):
        return self.fields.get(key)

    def get_tensor(self, idx):
        return self.tensors[idx]

    def tensor(self, name):
        return self._by_name.get(name)

    def tensor_bytes(self, name):
        return bytes(self.tensor(name).raw_bytes())

    def close(self):
        """Drop the cache entry and release the mapping.  Views taken from
        `.data` of this reader's tensors must be gone first."""
        _CACHE.pop(self._key, None)
        for t in self.tensors:
            t.data = None
            t._mm = None
        self.data = None
        self._mm.close()
        os.close(self._fd)


def load(path):
    r = FastGGUF(path)
    return r, {t.name: t for t in r.tensors}


# ------------------------------------------------------------------ writer --
def _pack_str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v):
    """(type, bytes) of a metadata value: str, bool, int (int32 / uint32 /
    int64 by range), float (float32), or a list of str / int / float."""
    if isinstance(v, str):
        return GGUFValueType.STRING, _pack_str(v)
    if isinstance(v, bool):
        return GGUFValueType.BOOL, struct.pack("<B", int(v))
    if isinstance(v, (int, np.integer)):
        v = int(v)
        if 0 <= v < 2 ** 32:
            return GGUFValueType.UINT32, struct.pack("<I", v)
        if -2 ** 31 <= v < 2 ** 31:
            return GGUFValueType.INT32, struct.pack("<i", v)
        return GGUFValueType.INT64, struct.pack("<q", v)
    if isinstance(v, (float, np.floating)):
        return GGUFValueType.FLOAT32, struct.pack("<f", float(v))
    if isinstance(v, (list, tuple)):
        if all(isinstance(x, str) for x in v):
            return GGUFValueType.ARRAY, struct.pack("<IQ", GGUFValueType.STRING, len(v)) + b"".join(_pack_str(x) for x in v)
        if all(isinstance(x, (int, np.integer)) and not isinstance(x, bool) for x in v):
            return GGUFValueType.ARRAY, struct.pack("<IQ", GGUFValueType.INT32, len(v)) + np.asarray(v, "<i4").tobytes()
        return GGUFValueType.ARRAY, struct.pack("<IQ", GGUFValueType.FLOAT32, len(v)) + np.asarray(v, "<f4").tobytes()
    raise TypeError(f"unsupported metadata value {v!r}")


def write_gguf(path, fields, tensors, alignment=GGUF_DEFAULT_ALIGNMENT):
    """Write a GGUF v3 file.  fields: {key: value} (see _pack_value);
    tensors: [(name, ggml type name or GGMLQuantizationType, dims with ne[0]
    first, bytes-like data)] in file order."""
    fields = dict(fields)
    if alignment != GGUF_DEFAULT_ALIGNMENT:
        fields["general.alignment"] = int(alignment)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(fields)))
    for k, v in fields.items():
        t, b = _pack_value(v)
        head += _pack_str(k) + struct.pack("<I", t) + b
    offs, off = [], 0
    for name, ttype, dims, data in tensors:
        gt = ttype if isinstance(ttype, GGMLQuantizationType) else GGMLQuantizationType[ttype]
        bs, ts = GGML_QUANT_SIZES[gt]
        n_el = int(np.prod([int(d) for d in dims]))
        nbytes = memoryview(data).nbytes
        if nbytes != n_el // bs * ts:
            raise ValueError(f"tensor {name}: {nbytes} bytes for {n_el} {gt.name} values")
        head += _pack_str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *[int(d) for d in dims])
        head += struct.pack("<IQ", int(gt), off)
        offs.append(off)
        off += nbytes
        off += (-off) % alignment
    head += b"\0" * ((-len(head)) % alignment)
    tmp = os.fspath(path) + ".tmp"
    with open(tmp, "wb") as f:
        f.write(head)
        pos = 0
        for (name, ttype, dims, data), o in zip(tensors, offs):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            f.write(memoryview(data).cast("B"))
            pos += memoryview(data).nbytes
        f.write(b"\0" * ((-pos) % alignment))
    os.replace(tmp, path)
