"""Per-block timeline of the single-token layer kernel (k_decode_layer) from its trace build.

Build the trace library first (`make -C silentotithrandousha_amd trace-lib`: the library with
-DMOE_TRACE_TIMELINE, where thread 0 of every block stores the 100 MHz realtime counter at
numbered points, and the block's XCC_ID / CU into slot 7), then run from the repository root:

    python3 silentotithrandousha_amd/probes/decode_timeline.py [n_experts]

Runs 24 eager single-token forwards of n_experts-expert GPT-OSS-shaped layers (hidden 2880,
top-4; 4 resident layers, distinct tokens) and prints, over the last 20 launches (medians), the
phase durations of the gate_up and down blocks, when the phases end (us from the first block's
start), which blocks share a CU, and the gate_up end time by the number of weight tiles its CU
streams. Stamps (decode_layer.hip, MOE_TRACE): gate_up blocks 0 start, 1 x split in LDS,
2 routing known, 3 tiles computed, 5 after the block barrier, 6 h stores acknowledged, 4 flag
stored; down blocks 0 start, 1 routing known, 2 all flags seen, 3 h copy issued, 5 sweep done,
4 output stored; router blocks (wavefront 0) 0 start, 1 logit computed (its stores follow).
Development tool: not used by the library, the tests or the benchmark.
"""
import ctypes
import os
import sys
from collections import defaultdict

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import silentotithrandousha_amd._ffi as F  # noqa: E402

F.LIB_PATH = os.path.join(ROOT, "silentotithrandousha_amd", "probes", "libmxfp4moe_trace.so")

from silentotithrandousha_amd import GpuMoeDispatcher  # noqa: E402
from silentotithrandousha_amd import synthetic as syn  # noqa: E402

H = I = 2880
N_CU = 256  # the geometry below assumes the full part (layer_geometry, layer_extra_tile)


def geometry(E):
    """layer_geometry (decode_layer.hip) for the 20B / 120B shapes on N_CU compute units."""
    n_rt, n_dn, tps = (E + 3) // 4, H // 16, 2 * I // 16
    tiles = 4 * tps
    n_gu = min((tiles + 3) // 4, max((tiles + 4) // 5, 2 * N_CU - n_rt - n_dn))
    return n_rt, n_gu, n_dn, tiles - 4 * n_gu


def extra_tile(b, n_rt, n_gu, n_dn, X):
    """layer_extra_tile (decode_layer.hip): whether gate_up block b streams an extra tile."""
    G, N, R, i = n_rt + n_gu + n_dn, N_CU, n_rt, n_rt + b
    if G <= N or G > 2 * N or R >= N:
        return (b + 1) * X // n_gu > b * X // n_gu
    rank = 0
    for lo, hi in ((G - N, N + R), (R + n_gu - N, G - N), (R - N, min(R + n_gu - N, G - N)), (N + R, N + R + n_gu)):
        lo, hi = max(lo, R), min(hi, R + n_gu)
        if lo <= i < hi:
            return rank + i - lo < X
        rank += max(0, hi - lo)
    return False


def main():
    E = int(sys.argv[1]) if len(sys.argv) > 1 else 32
    n_rt, n_gu, n_dn, X = geometry(E)
    nb = n_rt + n_gu + n_dn
    d = GpuMoeDispatcher(H, I, 7.0)
    for li in range(4):
        d.preload_layer(li, syn.make_layer(H, I, E, seed=100 + li))
    read = F.lib().moe_trace_read
    read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    read.restype = ctypes.c_int
    launches = []
    for it in range(24):
        d.layer_forward(it % 4, syn.hidden(1, H, seed=200 + it), 4)
        buf = np.zeros(nb * 16, dtype=np.int64)
        assert read(buf.ctypes.data, nb) == 0
        launches.append(buf.reshape(nb, 16))
    d.close()
    print(f"E={E}: {n_rt} router, {n_gu} gate_up ({X} with an extra tile), {n_dn} down blocks")
    ph, ends, by_load, pair = defaultdict(list), defaultdict(list), defaultdict(list), []
    gu, dn = range(n_rt, n_rt + n_gu), range(n_rt + n_gu, nb)
    for blk in launches[4:]:
        t0 = blk[n_rt:, 0].min()
        us = (blk - t0) / 100.0
        for name, (a, b_) in {"gate_up: x split": (0, 1), "gate_up: routing": (1, 2), "gate_up: tiles": (2, 3),
                              "gate_up: barrier": (3, 5), "gate_up: h stores acknowledged": (5, 6),
                              "gate_up: flag": (6, 4)}.items():
            ph[name].append(np.median([us[i, b_] - us[i, a] for i in gu]))
        for name, (a, b_) in {"down: routing": (0, 1), "down: flag wait": (1, 2), "down: copy + sweep": (3, 5),
                              "down: combine": (5, 4)}.items():
            ph[name].append(np.median([us[i, b_] - us[i, a] for i in dn]))
        rt = range(0, n_rt)
        ph["router: x, weights and logit"].append(np.median([us[i, 1] - us[i, 0] for i in rt]))
        ends["router blocks start (min)"].append(us[list(rt), 0].min())
        ends["router logits computed (max)"].append(us[list(rt), 1].max())
        ends["routing known (gate_up, p50)"].append(np.median(us[list(gu), 2]))
        ends["gate_up flags stored (max)"].append(us[list(gu), 4].max())
        ends["down: all flags seen (p50)"].append(np.median(us[list(dn), 2]))
        ends["end (down blocks, max)"].append(us[list(dn), 4].max())
        cu = defaultdict(list)
        for i in range(nb):
            cu[int(blk[i, 7])].append(i)
        pair.append(np.mean([len(v) == 2 and v[1] - v[0] == N_CU for v in cu.values()]))
        for members in cu.values():
            tiles = sum((4 + extra_tile(i - n_rt, n_rt, n_gu, n_dn, X)) if i in gu else (4 if i in dn else 0)
                        for i in members)
            gus = [us[i, 4] for i in members if i in gu]
            if gus:
                by_load[tiles].append(max(gus))
    print("phase durations (us, median over blocks and launches):")
    for k, v in ph.items():
        print(f"  {k:34s} {np.median(v):6.2f}")
    print("times from the first block's start (us, median over launches):")
    for k, v in ends.items():
        print(f"  {k:34s} {np.median(v):6.2f}")
    print(f"blocks i and i + {N_CU} on one CU: {100 * np.mean(pair):.0f} % of the CUs")
    print("gate_up end by the tiles its CU streams (CUs per launch, median end us):")
    for t in sorted(by_load):
        print(f"  {t:2d} tiles: {len(by_load[t]) / len(launches[4:]):5.0f} CUs, {np.median(by_load[t]):6.2f}")


if __name__ == "__main__":
    main()
