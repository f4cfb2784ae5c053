"""numpy row decoders for the driver's embedding lookup.

The reference driver dequantizes one embedding row on the host: Q8_0 inline
in numpy (src/smol_engine.py:180-185), other formats through gguf-py's
dequantize (src/smol_engine.py:187).  These decoders compute the same fp32
values with the same operation order ((d*sc)*q for Q6_K, d*sc*q - dmin*m for
Q4_K, q*d for Q8_0); tests/test_oracle_pins.py checks them bit-for-bit
against the oracle's row decoder.  The device-resident decode loop does the same lookup on
the GPU (embed kernel) and never calls this module.
"""
import numpy as np


def _f16(b):
    return b.copy().view(np.float16).astype(np.float32)


def dequant_q8_0(row):
    blk = row.reshape(-1, 34)
    d = _f16(blk[:, :2])
    q = blk[:, 2:].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)


def _kscales(s):
    s = s.astype(np.uint8)
    sc = np.empty((s.shape[0], 8), np.uint8)
    mn = np.empty((s.shape[0], 8), np.uint8)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc.astype(np.float32), mn.astype(np.float32)


def dequant_q4_k(row):
    blk = row.reshape(-1, 144)
    d = _f16(blk[:, 0:2])
    dmin = _f16(blk[:, 2:4])
    sc, mn = _kscales(blk[:, 4:16])
    qs = blk[:, 16:].reshape(-1, 4, 32)
    q = np.empty((blk.shape[0], 8, 32), np.float32)
    q[:, 0::2, :] = qs & 0xF
    q[:, 1::2, :] = qs >> 4
    dsc = (d * sc)[:, :, None]
    dm = (dmin * mn)[:, :, None]
    return (dsc * q - dm).reshape(-1)


def dequant_q5_k(row):
    """(q*d)*sc - dmin*m, q = nibble | fifth bit << 4, the order of the
    reference's row decoder (src/m5/m5_gemm.c:212-231)."""
    blk = row.reshape(-1, 176)
    nb = blk.shape[0]
    d = _f16(blk[:, 0:2])
    dmin = _f16(blk[:, 2:4])
    sc, mn = _kscales(blk[:, 4:16])
    qh = blk[:, 16:48]
    qs = blk[:, 48:].reshape(nb, 4, 32)
    q = np.empty((nb, 8, 32), np.int32)
    q[:, 0::2, :] = qs & 0xF
    q[:, 1::2, :] = qs >> 4
    for j in range(8):
        q[:, j, :] |= ((qh >> j) & 1).astype(np.int32) << 4
    qd = q.astype(np.float32) * d[:, :, None]
    return (qd * sc[:, :, None] - (dmin * mn)[:, :, None]).reshape(-1)


def dequant_q6_k(row):
    blk = row.reshape(-1, 210)
    nb = blk.shape[0]
    ql = blk[:, :128].reshape(nb, 2, 64)
    qh = blk[:, 128:192].reshape(nb, 2, 32)
    sc = blk[:, 192:208].copy().view(np.int8).astype(np.float32)
    d = _f16(blk[:, 208:210])
    q = np.empty((nb, 2, 4, 32), np.int32)
    q[:, :, 0] = (ql[:, :, :32] & 0xF) | (((qh >> 0) & 3) << 4)
    q[:, :, 1] = (ql[:, :, 32:] & 0xF) | (((qh >> 2) & 3) << 4)
    q[:, :, 2] = (ql[:, :, :32] >> 4) | (((qh >> 4) & 3) << 4)
    q[:, :, 3] = (ql[:, :, 32:] >> 4) | (((qh >> 6) & 3) << 4)
    qf = (q.reshape(nb, 256) - 32).astype(np.float32)
    dsc = (d * sc)  # [nb, 16]
    return (np.repeat(dsc, 16, axis=1) * qf).reshape(-1)


def dequant_row(code, row):
    if code == 0:
        return dequant_q8_0(row)
    if code == 5:
        return dequant_q4_k(row)
    if code == 4:
        return dequant_q6_k(row)
    if code == 3:
        return dequant_q5_k(row)
    if code == 9:
        return row.copy().view(np.float32)
    if code == 7:
        return row.copy().view(np.float16).astype(np.float32)
    raise ValueError(f"no row decoder for format code {code}")
