"""Per-wave timeline of the roofline GEMV launch (profiling tool).

Usage (repository root):
    python3 dracomancer-llmengine_amd/build.py --timeline   # lib/libdraco_hip_timeline.so (CPU side)
    python3 dracomancer-llmengine_amd/timeline.py           # on the GPU

The timeline build (-DDRACO_TIMELINE) has every wave of the roofline launch
(k_dq<8, 1, false, false, 0, 0, ...>: W 14336 x 4096 Q4_K, fp32 x, 512 blocks
of 8 waves, the `roofline` kernel of bench.py) store s_memrealtime stamps
(100 MHz, 10 ns) at its start, when its slice of x is digitised in LDS, after
each of its first four items (items 1 and 3 end a tile, with the tile's
reduction and store) and at its end.  This script replays the same graph as
bench.py's roofline block (draco_bench_gemv, 10 rotating weight copies, 200
launches), reads the stamps of the last launch and prints each phase's
distribution over the 4096 waves.  The stamps cost ~0.5 us per launch, so
the graph-timed figure printed here is above the product build's.
"""
import ctypes as ct
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
os.environ["DRACO_HIP_SO"] = os.path.join(HERE, "lib", "libdraco_hip_timeline.so")
sys.path.insert(0, HERE)

import numpy as np  # noqa: E402

from dracohip import lib  # noqa: E402

N_OUT, N_IN, BLOCKS, WAVES = 14336, 4096, 512, 8


def pct(v):
    return (f"min {v.min():5.2f}  p10 {np.percentile(v, 10):5.2f}  median {np.median(v):5.2f}  "
            f"p90 {np.percentile(v, 90):5.2f}  max {v.max():5.2f}")


def main():
    if not os.path.exists(os.environ["DRACO_HIP_SO"]):
        sys.exit("timeline build missing: run `python3 dracomancer-llmengine_amd/build.py --timeline` first")
    L = lib.load()
    read = L.draco_timeline_read
    read.argtypes, read.restype = [ct.c_void_p], ct.c_int
    rng = np.random.default_rng(1)
    W = lib.quantize(5, rng.standard_normal((N_OUT, N_IN), dtype=np.float32) * np.float32(0.02))
    buf = np.zeros(1024 * 16 * 8, np.uint64)
    for rep in range(3):
        out = np.zeros(8, np.float32)
        if L.draco_timeline_clear() or L.draco_bench_gemv(5, lib.pu8(W), N_OUT, N_IN, 10, 200, lib.pf(out)):
            sys.exit(lib.last_error())
        print(f"replay {rep}: {out[4]:.3f} us per launch (graph-timed, stamps included)")
    if read(buf.ctypes.data):
        sys.exit("timeline read failed")
    t = buf.reshape(1024 * 16, 8)[:BLOCKS * WAVES].astype(np.int64)
    if (t[:, 6] == 0).any():
        sys.exit("missing stamps: is this the timeline build?")
    rel = (t[:, :7] - t[:, 0].min()) * 0.01  # 100 MHz ticks -> us from the launch's first wave start
    xcc = t[:, 7]
    tiles = (N_OUT // 16 + BLOCKS - 1 - np.arange(BLOCKS)) // BLOCKS  # 896 tiles: 2 per block for blocks < 384
    two = np.repeat(tiles == 2, WAVES)
    print(f"last launch: {len(rel)} waves, first start -> last end {rel[:, 6].max():.2f} us")
    print("stamps (us from the first wave start):")
    rows = [("wave start", rel[:, 0]), ("x digitised in LDS", rel[:, 1]), ("item 0 done", rel[:, 2]),
            ("tile 1 done (item 1)", rel[:, 3]), ("item 2 done (2-tile blocks)", rel[two, 4]),
            ("tile 2 done (2-tile blocks)", rel[two, 5]), ("wave end", rel[:, 6])]
    for name, v in rows:
        print(f"  {name:>28}: {pct(v)}")
    print("phases (us per wave):")
    rows = [("x wait + digits", rel[:, 1] - rel[:, 0]), ("item 0 after x", rel[:, 2] - rel[:, 1]),
            ("item 1 + tile reduction", rel[:, 3] - rel[:, 2]), ("tile 2 (2-tile blocks)", rel[two, 5] - rel[two, 3])]
    for name, v in rows:
        print(f"  {name:>28}: {pct(v)}")
    print("by XCC (waves, median start, median end, last end):")
    for x in sorted(set(xcc.tolist())):
        s = xcc == x
        print(f"  xcc {x}: {s.sum():4d}  {np.median(rel[s, 0]):.2f}  {np.median(rel[s, 6]):.2f}  {rel[s, 6].max():.2f}")


if __name__ == "__main__":
    main()
