"""GGUF files (dracohip/gguf.py): the reader keeps the interface subset of the
reference's FastGGUF (src/gguf_fast.py:167-370) and its checks (magic,
version, duplicate tensor names, data past the end); the writer turns the
synthetic models into files the reader maps back byte for byte.

gguf-py (the reference's source of type tables and of its own reader) is not
available here; the round trip pins the writer and the reader against each
other, and the fixed-layout test below pins the byte layout of a small file
written by hand from the GGUF format's field order.
"""
import os
import struct

import numpy as np
import pytest

from dracohip import gguf, models


def _tiny_model():
    return models.build_llama(models.TINY_K, 0)


def test_roundtrip_tiny_model(tmp_path):
    m = _tiny_model()
    p = tmp_path / "tiny.gguf"
    models.save_llama_gguf(m, p)
    m2 = models.load_llama_gguf(p)
    assert m2.digest() == m.digest()
    assert m2.cfg.hidden == m.cfg.hidden and m2.cfg.n_layer == m.cfg.n_layer
    assert (m2.cfg.n_head, m2.cfg.n_kv, m2.cfg.head_dim, m2.cfg.n_ff) == (m.cfg.n_head, m.cfg.n_kv, m.cfg.head_dim,
                                                                          m.cfg.n_ff)
    assert m2.cfg.vocab == m.cfg.vocab and m2.cfg.codes == m.cfg.codes and m2.cfg.tied == m.cfg.tied
    assert np.float32(m2.cfg.eps) == np.float32(m.cfg.eps) and m2.cfg.rope_base == m.cfg.rope_base
    assert list(m2.prompt()) == list(m.prompt())
    for name, (buf, code, n_out, n_in) in m.tensors.items():
        b2, c2, o2, i2 = m2.tensors[name]
        assert (c2, o2, i2) == (code, n_out, n_in)
        assert np.array_equal(b2, buf)
    for name, w in m.norms.items():
        assert np.array_equal(m2.norms[name], w)


def test_tensor_views_are_zero_copy_and_cached(tmp_path):
    m = _tiny_model()
    p = tmp_path / "tiny.gguf"
    models.save_llama_gguf(m, p)
    r = gguf.FastGGUF(p)
    assert gguf.FastGGUF(p) is r                       # cached per (path, size, mtime)
    t = r.tensor("blk.0.attn_q.weight")
    assert t.tensor_type.name == "Q4_K" and tuple(t.shape.tolist()) == (m.cfg.hidden, m.cfg.n_head * 64)
    assert np.shares_memory(t.data, r.data)           # a view of the mapping, no copy
    assert t.data.shape == (m.cfg.n_head * 64, m.cfg.hidden // 256 * 144)
    assert t.data_offset % r.alignment == 0
    assert bytes(t.raw_bytes()) == r.tensor_bytes(t.name) == m.tensors[t.name][0].tobytes()
    n = r.get_field("llama.attention.head_count")
    assert n.contents() == m.cfg.n_head and n.types == [gguf.GGUFValueType.UINT32]


def test_metadata_value_types(tmp_path):
    p = tmp_path / "meta.gguf"
    fields = {"a.str": "hello", "a.u32": 7, "a.i32": -3, "a.i64": -(2 ** 40), "a.f32": 0.5, "a.bool": True,
              "a.strs": ["x", "yz", ""], "a.ints": [1, -2, 3], "a.floats": [0.25, -1.5]}
    gguf.write_gguf(p, fields, [("t", "F32", (4,), np.arange(4, dtype=np.float32))])
    r = gguf.FastGGUF(p)
    got = {k: f.contents() for k, f in r.fields.items()}
    assert got["a.str"] == "hello" and got["a.u32"] == 7 and got["a.i32"] == -3 and got["a.i64"] == -(2 ** 40)
    assert got["a.f32"] == 0.5 and got["a.bool"] == 1
    assert got["a.strs"] == ["x", "yz", ""] and got["a.ints"] == [1, -2, 3] and got["a.floats"] == [0.25, -1.5]
    assert r.fields["a.strs"].types == [gguf.GGUFValueType.ARRAY, gguf.GGUFValueType.STRING]
    assert np.array_equal(r.tensor("t").data, np.arange(4, dtype=np.float32))


def test_hand_built_layout(tmp_path):
    """A one-key, one-tensor file laid out by hand from the format's field
    order: magic, version, tensor count, kv count, key, value type, value,
    tensor name, n_dims, dims, type, offset, padding to 32, data."""
    def s(x):
        return struct.pack("<Q", len(x)) + x
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 1)
    head += s(b"general.architecture") + struct.pack("<I", 8) + s(b"llama")
    head += s(b"w") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", 8, 0)   # Q8_0, 2 rows
    head += b"\0" * ((-len(head)) % 32)
    data = bytes(range(68))
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + data)
    r = gguf.FastGGUF(p)
    assert r.version == 3 and r.get_field("general.architecture").contents() == "llama"
    t = r.tensor("w")
    assert t.tensor_type == gguf.GGMLQuantizationType.Q8_0 and t.n_bytes == 68 and t.data_offset == len(head)
    assert t.data.shape == (2, 34) and bytes(t.raw_bytes()) == data
    # the writer produces the same bytes for the same content
    q = tmp_path / "written.gguf"
    gguf.write_gguf(q, {"general.architecture": "llama"}, [("w", "Q8_0", (32, 2), data)])
    assert q.read_bytes() == head + data + b"\0" * ((-len(data)) % 32)


@pytest.mark.parametrize("case", ["magic", "version", "dup", "past_end", "truncated"])
def test_rejects_bad_files(tmp_path, case):
    p = tmp_path / f"{case}.gguf"
    good = tmp_path / "good.gguf"
    gguf.write_gguf(good, {"k": 1}, [("a", "F32", (8,), np.zeros(8, np.float32)),
                                     ("b", "F32", (8,), np.ones(8, np.float32))])
    b = bytearray(good.read_bytes())
    if case == "magic":
        b[:4] = b"GGUG"
    elif case == "version":
        b[4:8] = struct.pack("<I", 9)
    elif case == "dup":
        i = b.index(b"\x01\x00\x00\x00\x00\x00\x00\x00b")   # the second tensor's name "b" -> "a"
        b[i + 8] = ord("a")
    elif case == "past_end":
        b = b[:-40]
    elif case == "truncated":
        b = b[:30]
    p.write_bytes(bytes(b))
    with pytest.raises(ValueError):
        gguf.FastGGUF(p)
