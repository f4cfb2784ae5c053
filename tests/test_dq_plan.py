"""Launch planning of the Q4_K / Q6_K segment GEMV (k_dq), on the CPU.

draco_dq_plan is the host function that picks a launch's waves per block,
grid and variant.  For every row width from 1 to 64 super-blocks, several
tile counts and every variant (plain, SwiGLU pair, row dots, split-K with
and without the GNORM prologue), this test replays the kernel's index
arithmetic in Python and checks, for each shape the planner accepts:
- every super-block an item multiplies was digitised by the prologue of the
  same block (and, in the instances without a block barrier after the
  prologue, by the same wave);
- the items of a tile (split-K: of a tile half) cover its super-blocks
  exactly once;
- the row-dot loads cover the row.
A shape that breaks one of these multiplies LDS that was never written: the
4-wave split-K instance on rows of 24 super-blocks did, before the planner
refused it.  No GPU is touched.
"""
import ctypes as ct

import numpy as np
import pytest

CUS = 256
TILE_COUNTS = (1, 3, 16, 128, 129, 300, 512, 2000)


def plan(L, n_in, tiles, dual=0, ksplit=0, do_norm=0, gd_n=0):
    out = (ct.c_int * 6)()
    rc = L.draco_dq_plan(n_in, tiles, dual, ksplit, do_norm, gd_n, CUS, out)
    return rc, list(out)


def replay(n_in, tiles, shape, barrier):
    """The kernel's prologue and item loops (k_dq in csrc/gemv.hip) for one
    launch shape; returns a list of violations.  Blocks differ only in which
    split-K half their prologue digitises and tiles only in which half they
    multiply, so each (prologue, tile half) pair that occurs is replayed once."""
    nw, grid, ipt1, ks, gd, xp = shape
    nb, n4, NT = n_in // 256, n_in // 4, 64 * nw
    total = 2 * tiles if ks else tiles
    bad = []
    ipt = 1 if ipt1 else ((nb // 2) // nw if ks else -(-nb // nw))
    kown = ks and grid == total  # one tile per block: the block digitises its half only

    def owners(kq_lo, kq_n):
        owner = np.full(n4, -1, np.int64)  # wave that digitised each float4
        for q in range(xp):
            if kq_lo <= q < kq_lo + kq_n:
                i4 = np.arange(NT) + q * NT
                ok = i4 < n4
                owner[i4[ok]] = np.arange(NT)[ok] // 64
        return owner.reshape(nb, 64)

    halves = (0, 1) if ks else (0,)
    if kown:
        kq_n = (nb // 2) // nw
        cases = [(owners(h * kq_n, kq_n), h) for h in halves]
    else:
        o = owners(0, xp)
        cases = [(o, h) for h in halves]
    for sb_owner, h in cases:
        first, span = (h * (nb // 2), nb // 2) if ks else (0, nb)
        seen = []
        for w in range(nw):
            for k in range(ipt):
                b = w + first + k * nw
                if b >= nb:
                    continue  # padding item
                seen.append(b)
                o = sb_owner[b]
                if (o < 0).any():
                    bad.append(f"half {h} wave {w}: super-block {b} not digitised")
                elif not barrier and (o != w).any():
                    bad.append(f"half {h} wave {w}: super-block {b} digitised by another wave")
        if sorted(seen) != list(range(first, first + span)):
            bad.append(f"half {h}: items cover {sorted(set(seen))[:4]}.. not [{first}, {first + span})")
    if gd and n4 > 2 * NT:
        bad.append("row-dot loads cover less than the row")
    return bad


VARIANTS = [  # (name, dual, ksplit, do_norm, gd_n, barrier after the prologue)
    ("plain", 0, 0, 0, 0, False),
    ("plain+rms", 0, 0, 1, 0, True),
    ("plain+pres", 0, 0, 3, 0, True),
    ("gnorm", 0, 0, 2, 0, False),
    ("swiglu+rms", 1, 0, 1, 0, True),
    ("swiglu+pres8", 1, 0, 4, 0, True),
    ("rowdots", 0, 0, 1, 16, True),
    ("splitk", 0, 2, 0, 0, False),
    ("splitk+gnorm", 0, 2, 2, 0, False),
]


@pytest.mark.parametrize("variant", VARIANTS, ids=[v[0] for v in VARIANTS])
def test_every_accepted_shape_covers_its_items(variant):
    from dracohip import lib
    L = lib.load()
    name, dual, ksplit, do_norm, gd_n, barrier = variant
    accepted = 0
    for nb in range(1, 65):
        n_in = 256 * nb
        for tiles in TILE_COUNTS:
            rc, shape = plan(L, n_in, tiles, dual, ksplit, do_norm, gd_n)
            if rc:
                continue
            accepted += 1
            assert shape[5] >= 1 and shape[0] in (4, 8, 16) and 1 <= shape[1]
            bad = replay(n_in, tiles, shape, barrier)
            assert not bad, (name, nb, tiles, shape, bad[:3])
    assert accepted > 0, name


def test_split_k_widths():
    """Split-K serves rows of 8, 16 and 32 super-blocks (the configs' o and
    down projections) and refuses 24: neither instance's prologue covers a
    24-block row's second half (4 waves hold 16 super-blocks of x)."""
    from dracohip import lib
    L = lib.load()
    assert L.draco_dq_plan(2048, 128, 0, 2, 0, 0, CUS, None) == 0
    got = {nb: plan(L, 256 * nb, 128, 0, 2, 0)[1][0] for nb in (8, 16, 32)}
    assert got == {8: 4, 16: 8, 32: 8}
    assert plan(L, 256 * 24, 128, 0, 2, 0)[0] == -1
    assert plan(L, 256 * 8, 128, 0, 2, 2)[0] == -1  # GNORM split-K is 8-wave only
    for nb in list(range(1, 8)) + [9, 10, 12, 20, 24, 28, 33, 40, 64]:
        assert plan(L, 256 * nb, 128, 0, 2, 0)[0] == -1, nb


def test_replay_flags_the_uncovered_split_k_shape():
    """The replay is a real check: the shape the launcher used to take for
    24-block split-K rows (4 waves, one tile per block) is flagged, as is a
    plain 4-wave launch on 32-block rows."""
    assert replay(6144, 128, [4, 256, 0, 1, 0, 4], False)
    assert replay(8192, 512, [4, 200, 0, 0, 0, 4], True)
