"""Private device layout: the repack is a bijection and puts every byte where
the GEMV kernels' lanes read it.

CPU only (draco_repack / draco_unpack are host functions).  The expected
positions are restated here in numpy from the layout's definition (rows in
tiles of 16, item (tile, super-block), lane l = j + 16*g), independently of
the C offset helpers.
"""
import numpy as np
import pytest

Q4T_ITEM, Q6T_ITEM, Q5T_ITEM = 2304, 3360, 2816


def _layout(lib, code, n_out, n_in, rng):
    x = rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02)
    W = lib.quantize(code, x)
    L = lib.load()
    nbytes = L.draco_layout_query(code, n_out, n_in, None)
    assert nbytes > 0
    dev = np.zeros(nbytes, np.uint8)
    assert L.draco_repack(code, lib.pu8(W), n_out, n_in, lib.pu8(dev)) == 0
    return W, dev


@pytest.mark.parametrize("code", [0, 3, 4, 5])
@pytest.mark.parametrize("n_out,n_in", [(1, 256), (17, 512), (48, 768), (100, 256), (33, 2048)])
def test_repack_roundtrip(code, n_out, n_in):
    from dracohip import lib
    W, dev = _layout(lib, code, n_out, n_in, np.random.default_rng(n_out * 7 + n_in))
    back = np.zeros_like(W)
    assert lib.load().draco_unpack(code, lib.pu8(dev), n_out, n_in, lib.pu8(back)) == 0
    assert np.array_equal(back, W)


@pytest.mark.parametrize("n_out,n_in", [(16, 256), (37, 768)])
def test_q4k_tile_positions(n_out, n_in):
    from dracohip import lib
    W, dev = _layout(lib, 5, n_out, n_in, np.random.default_rng(5))
    nb = n_in // 256
    blocks = W.reshape(n_out, nb, 144)
    ntiles = (n_out + 15) // 16
    items = dev[: ntiles * nb * Q4T_ITEM].reshape(ntiles, nb, Q4T_ITEM)
    for r in range(n_out):
        t, j = divmod(r, 16)
        for b in range(nb):
            blk, it = blocks[r, b], items[t, b]
            assert np.array_equal(it[2048 + 16 * j: 2048 + 16 * j + 16], blk[:16])
            for g in range(4):
                l = j + 16 * g
                for half in range(2):  # qs bytes 64*half + (g>>1)*32 + (g&1)*16 + e, stored ^ 0x80
                    src = blk[16 + 64 * half + (g >> 1) * 32 + (g & 1) * 16:][:16]
                    got = it[1024 * half + 16 * l: 1024 * half + 16 * l + 16]
                    assert np.array_equal(got, src ^ 0x80)
    # rows past n_out in the last tile are zero
    if n_out % 16:
        for j in range(n_out % 16, 16):
            it = items[ntiles - 1]
            assert not it[:, 2048 + 16 * j: 2048 + 16 * j + 16].any()


@pytest.mark.parametrize("n_out,n_in", [(16, 256), (37, 768)])
def test_q5k_tile_positions(n_out, n_in):
    """Q5_K items: the Q4_K positions for qs (not XORed) and the header,
    then qh[16 c + e] of row j at 2304 + 16 (j + 16 c)."""
    from dracohip import lib
    W, dev = _layout(lib, 3, n_out, n_in, np.random.default_rng(3))
    nb = n_in // 256
    blocks = W.reshape(n_out, nb, 176)
    ntiles = (n_out + 15) // 16
    items = dev[: ntiles * nb * Q5T_ITEM].reshape(ntiles, nb, Q5T_ITEM)
    for r in range(n_out):
        t, j = divmod(r, 16)
        for b in range(nb):
            blk, it = blocks[r, b], items[t, b]
            assert np.array_equal(it[2048 + 16 * j: 2048 + 16 * j + 16], blk[:16])
            for c in range(2):
                assert np.array_equal(it[2304 + 16 * (j + 16 * c): 2320 + 16 * (j + 16 * c)], blk[16 + 16 * c:][:16])
            for g in range(4):
                l = j + 16 * g
                for half in range(2):
                    src = blk[48 + 64 * half + (g >> 1) * 32 + (g & 1) * 16:][:16]
                    assert np.array_equal(it[1024 * half + 16 * l: 1024 * half + 16 * l + 16], src)


def test_q5k_encoder_error_bound():
    """The Q5_K encoder's values decode (numpy, the reference's row decoder
    order) to within one quantization step of the input: per sub-block the
    step is d*sc, and the offset dmin*m is within d*sc of -min(x) by
    construction, so |w - x| <= 1.5 d sc + dmin / 2."""
    from dracohip import lib, gguf_np
    rng = np.random.default_rng(55)
    x = rng.standard_normal((8, 512), dtype=np.float32) * np.float32(0.02)
    W = lib.quantize(3, x)
    rb = len(W) // 8
    for r in range(8):
        w = gguf_np.dequant_row(3, W[r * rb:(r + 1) * rb])
        blk = W[r * rb:(r + 1) * rb].reshape(-1, 176)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
        dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
        step = np.repeat(d * 63, 256) * 1.5 + np.repeat(dmin, 256) * 0.5
        assert np.all(np.abs(w - x[r]) <= step + 1e-7)
        assert np.abs(w - x[r]).max() < 0.01 * np.abs(x[r]).max() * 10


@pytest.mark.parametrize("n_out,n_in", [(16, 256), (21, 512)])
def test_q6k_tile_positions(n_out, n_in):
    from dracohip import lib
    W, dev = _layout(lib, 4, n_out, n_in, np.random.default_rng(6))
    nb = n_in // 256
    blocks = W.reshape(n_out, nb, 210)
    ntiles = (n_out + 15) // 16
    items = dev[: ntiles * nb * Q6T_ITEM].reshape(ntiles, nb, Q6T_ITEM)
    for r in range(n_out):
        t, j = divmod(r, 16)
        for b in range(nb):
            blk, it = blocks[r, b], items[t, b]
            ql, qh, sc, d = blk[:128], blk[128:192], blk[192:208], blk[208:210]
            assert np.array_equal(it[3328 + 2 * j: 3330 + 2 * j], d)
            for g in range(4):
                l, g2, c = j + 16 * g, g >> 1, g & 1
                assert np.array_equal(it[16 * l: 16 * l + 16], ql[64 * g2 + 16 * c:][:16])
                assert np.array_equal(it[1024 + 16 * l: 1040 + 16 * l], ql[64 * g2 + 32 + 16 * c:][:16])
                assert np.array_equal(it[2048 + 16 * l: 2064 + 16 * l], qh[32 * g2 + 16 * c:][:16])
                want_sc = np.array([sc[8 * g2 + c + 2 * rr] for rr in range(4)], np.uint8)
                assert np.array_equal(it[3072 + 4 * l: 3076 + 4 * l], want_sc)


def test_layout_rejects_bad_shapes():
    from dracohip import lib
    L = lib.load()
    assert L.draco_layout_query(5, 16, 100, None) == 0   # n_in not a multiple of 256
    assert L.draco_layout_query(2, 16, 256, None) == 0   # IQ3_S is not served
    assert L.draco_layout_query(4, 0, 256, None) == 0
