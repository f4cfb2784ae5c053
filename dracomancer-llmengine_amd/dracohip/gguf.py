"""Read-only GGUF reader (mmap, zero-copy tensor views) and a GGUF writer.

The reader keeps the public interface subset of the reference's `FastGGUF`
(src/gguf_fast.py:167-370), with its own parser (a bounds-checked cursor over
the mapping) and its own per-file reuse (a metaclass keyed by the file's
device, inode, size and mtime): `FastGGUF(path)` (one reader per unchanged file),
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

# metadata scalar types as little-endian numpy dtypes (BOOL is one byte)
_VT_DTYPE = {
    GGUFValueType.UINT8: np.dtype("<u1"), GGUFValueType.INT8: np.dtype("<i1"),
    GGUFValueType.UINT16: np.dtype("<u2"), GGUFValueType.INT16: np.dtype("<i2"),
    GGUFValueType.UINT32: np.dtype("<u4"), GGUFValueType.INT32: np.dtype("<i4"),
    GGUFValueType.FLOAT32: np.dtype("<f4"), GGUFValueType.BOOL: np.dtype("<u1"),
    GGUFValueType.UINT64: np.dtype("<u8"), GGUFValueType.INT64: np.dtype("<i8"),
    GGUFValueType.FLOAT64: np.dtype("<f8"),
}
# tensor types stored as plain numbers (everything else is block-quantized bytes)
_PLAIN_DTYPE = {
    GGMLQuantizationType.F16: np.float16, GGMLQuantizationType.F32: np.float32, GGMLQuantizationType.F64: np.float64,
    GGMLQuantizationType.I8: np.int8, GGMLQuantizationType.I16: np.int16, GGMLQuantizationType.I32: np.int32,
    GGMLQuantizationType.I64: np.int64,
}


class _Cursor:
    """Bounds-checked little-endian reads over the mapped file."""

    def __init__(self, buf, path):
        self.buf, self.path, self.pos = buf, path, 0

    def span(self, n):
        """Advance over n bytes and return their start offset."""
        at = self.pos
        if n < 0 or at + n > len(self.buf):
            raise ValueError(f"GGUF file truncated at byte {at} (needs {n} more): {self.path}")
        self.pos = at + n
        return at

    def number(self, dt):
        at = self.span(dt.itemsize)
        return np.frombuffer(self.buf, dtype=dt, count=1, offset=at)[0].item()

    def u32(self):
        return self.number(_VT_DTYPE[GGUFValueType.UINT32])

    def u64(self):
        return self.number(_VT_DTYPE[GGUFValueType.UINT64])

    def text(self):
        n = self.u64()
        at = self.span(n)
        return bytes(self.buf[at:at + n]).decode("utf-8", "replace")

    def value(self, vt):
        """One metadata value of type vt -> (python value or ndarray, type chain)."""
        vt = GGUFValueType(vt)
        if vt is GGUFValueType.STRING:
            return self.text(), [vt]
        if vt is not GGUFValueType.ARRAY:
            return self.number(_VT_DTYPE[vt]), [vt]
        et = GGUFValueType(self.u32())
        count = self.u64()
        if et is GGUFValueType.STRING:
            return [self.text() for _ in range(count)], [vt, et]
        if et is GGUFValueType.ARRAY:
            raise ValueError("nested GGUF arrays are not supported")
        dt = _VT_DTYPE[et]
        at = self.span(count * dt.itemsize)
        return np.frombuffer(self.buf, dtype=dt, count=count, offset=at), [vt, et]


class FastField:
    """One metadata key: `contents()` gives a str, a Python scalar, or a list
    (arrays of strings or of numbers), as the reference's reader does."""

    def __init__(self, offset, name, value, types):
        self.offset = offset
        self.name = name
        self.value = value
        self.types = types

    def contents(self, index_or_slice=slice(None)):
        v = self.value
        if isinstance(v, np.ndarray):
            v = v.tolist()
        if not isinstance(v, list):
            return v
        picked = v[index_or_slice]
        return picked if isinstance(index_or_slice, int) else list(picked)

    def __repr__(self):
        return f"FastField({self.name!r}, {[t.name for t in self.types]})"


class FastTensor:
    """A tensor of the file: `.data` is a read-only view of the mapping
    (quantized types as uint8 [rows, row bytes], float/int types in their
    dtype, numpy shape = reversed GGUF dims)."""

    def __init__(self, name, tensor_type, dims, mapping, offset, n_elements, n_bytes):
        self.name = name
        self.tensor_type = tensor_type
        self.shape = dims
        self.n_elements = n_elements
        self.n_bytes = n_bytes
        self.data_offset = offset
        self._mapping = mapping
        rows_first = tuple(int(d) for d in dims[::-1])
        plain = _PLAIN_DTYPE.get(tensor_type)
        if plain is not None:
            view = np.frombuffer(mapping, dtype=plain, count=n_elements, offset=offset)
            self.data = view.reshape(rows_first)
        else:
            per_block, block_bytes = GGML_QUANT_SIZES[tensor_type]
            row_bytes = rows_first[-1] // per_block * block_bytes
            view = np.frombuffer(mapping, dtype=np.uint8, count=n_bytes, offset=offset)
            self.data = view.reshape(rows_first[:-1] + (row_bytes,))

    def raw_bytes(self):
        return memoryview(self._mapping)[self.data_offset:self.data_offset + self.n_bytes]

    def __repr__(self):
        return f"FastTensor({self.name!r}, {self.tensor_type.name}, {tuple(self.shape.tolist())})"


class _OnePerFile(type):
    """Constructing a reader returns the open reader of the same file while
    the file is unchanged (same device/inode, size and modification time);
    otherwise a fresh one, which replaces it."""

    _open: dict = {}

    def __call__(cls, path, mode="r"):
        full = os.path.realpath(os.fspath(path))
        st = os.stat(full)
        ident = (st.st_dev, st.st_ino, st.st_size, st.st_mtime_ns)
        known = _OnePerFile._open.get(full)
        if known is not None and known._ident == ident:
            return known
        reader = super().__call__(full, mode)
        reader._ident = ident
        _OnePerFile._open[full] = reader
        return reader


class FastGGUF(metaclass=_OnePerFile):
    """Read-only, zero-copy GGUF reader; one open reader per unchanged file."""

    def __init__(self, path, mode="r"):
        if sys.byteorder != "little":
            raise RuntimeError("GGUF reader: little-endian hosts only")
        self.path = path
        self.fields: "OrderedDict[str, FastField]" = OrderedDict()
        self.tensors: list = []
        self._by_name: dict = {}
        with open(path, "rb") as f:
            try:
                self._map = _mmap.mmap(f.fileno(), 0, access=_mmap.ACCESS_READ)
            except ValueError:
                raise ValueError(f"not a GGUF file (empty): {path}") from None
        try:
            self._read_header()
        except Exception:
            self._release()
            raise
        self.data = np.frombuffer(self._map, dtype=np.uint8)

    def _read_header(self):
        cur = _Cursor(self._map, self.path)
        if len(self._map) < 24 or bytes(self._map[0:4]) != b"GGUF":
            raise ValueError(f"not a GGUF file: {self.path}")
        cur.span(4)
        self.version = cur.u32()
        if self.version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {self.version} (2 and 3 are read)")
        self.tensor_count = cur.u64()
        self.kv_count = cur.u64()
        for _ in range(self.kv_count):
            at = cur.pos
            key = cur.text()
            value, chain = cur.value(cur.u32())
            self.fields[key] = FastField(at, key, value, chain)
        directory = []
        for _ in range(self.tensor_count):
            name = cur.text()
            n_dims = cur.u32()
            if n_dims > GGML_MAX_DIMS:
                raise ValueError(f"tensor {name}: {n_dims} dimensions (at most {GGML_MAX_DIMS})")
            dims = np.array([cur.u64() for _ in range(n_dims)], np.uint64)
            ggml_type = GGMLQuantizationType(cur.u32())
            directory.append((name, dims, ggml_type, cur.u64()))
        align_field = self.fields.get("general.alignment")
        self.alignment = GGUF_DEFAULT_ALIGNMENT if align_field is None else int(align_field.contents())
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError(f"invalid alignment {self.alignment}")
        self.data_offset = -(-cur.pos // self.alignment) * self.alignment
        for name, dims, ggml_type, rel in directory:
            if name in self._by_name:
                raise ValueError(f"duplicate tensor name {name}")
            per_block, block_bytes = GGML_QUANT_SIZES[ggml_type]
            n_elements = int(np.prod(dims.astype(np.int64))) if dims.size else 1
            if dims.size and int(dims[0]) % per_block:
                raise ValueError(f"tensor {name}: row of {int(dims[0])} values is not a whole number of blocks")
            n_bytes = n_elements // per_block * block_bytes
            start = self.data_offset + rel
            if start + n_bytes > len(self._map):
                raise ValueError(f"tensor {name}: data ({n_bytes} bytes at {start}) past the end of the file")
            t = FastTensor(name, ggml_type, dims, self._map, start, n_elements, n_bytes)
            self.tensors.append(t)
            self._by_name[name] = t

    def _release(self):
        self.tensors, self._by_name, self.data = [], {}, None
        try:
            self._map.close()
        except BufferError:  # views still held elsewhere: the mapping goes with them
            pass

    def get_field(self, key):
        return self.fields.get(key)

    def get_tensor(self, idx):
        return self.tensors[idx]

    def tensor(self, name):
        return self._by_name.get(name)

    def tensor_bytes(self, name):
        return bytes(self._by_name[name].raw_bytes())

    def close(self):
        """Forget this reader and release the mapping.  Views taken from
        `.data` of its tensors must be gone first."""
        if _OnePerFile._open.get(self.path) is self:
            del _OnePerFile._open[self.path]
        for t in self.tensors:
            t.data = None
            t._mapping = None
        self._release()


def load(path):
    r = FastGGUF(path)
    return r, dict(r._by_name)


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
