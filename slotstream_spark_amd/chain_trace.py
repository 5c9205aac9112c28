"""Phase trace of the chained verify kernel (ssmoe_moe_verify_chain) through ssmoe_set_trace.

    python -m slotstream_spark_amd.chain_trace [T] [layers]

Builds a chain of `layers` (default 16) config-1 MoE layers (H 2048, 512 experts top-10, I 512, shared 512,
affine-4bit gs64, Zipf 1.1 routing bias) with seeded synthetic weights, times the step graph (HIP events, median of
5 x 40 steps), then runs one eager launch with the trace on and prints, for the last two layers, the median and maximum
time of each stamp over the workgroups that own output rows ("tile") and the others ("free"), in us from the first
start of the layer before the last. The stamps are kept in LDS by the kernel and written at its exit.
"""
from __future__ import annotations

import sys

import numpy as np
import torch

from . import _lib
from .engine.step import MoEWeights, MTPStepGraph
from .memory.slot_pool import SlotPool
from .memory.synth import LayerWeights, normal_bf16, zipf_bias

# (slot, name) of the per-layer row and of its extra row (the kernel's SS_TRACE(k) and SS_TRACE(16 + k))
MAIN = [(0, "layer start"), (5, "stream polled"), (1, "x staged"), (2, "A signalled"), (3, "tail done"),
        (4, "unique"), (7, "items done"), (13, "shared rows"), (8, "items seen"), (9, "h staged"), (10, "down done"),
        (12, "combine start"), (15, "shx seen"), (6, "stream stored"), (11, "layer end")]
EXTRA = [(2, "poll start"), (1, "first poll back"), (4, "dense done"), (8, "logits in"), (9, "probs"),
         (10, "topk done"), (5, "item loads issued"), (6, "item loads landed"), (14, "item dots"), (7, "first item"), (3, "combine summed"), (0, "stream acked"),
         (11, "down expert 1"), (12, "down expert 2"), (13, "down expert 3")]


def run(T: int = 2, nl: int = 16) -> str:
    H, I, E, K = 2048, 512, 512, 10
    pool = SlotPool(nl, E, H, I)
    pool.fill_random(1729)
    pool.place_permuted(1732)
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(E, 1.1, 1731 + l))
          for l, w in enumerate([LayerWeights(H, E, 512, seed=1729 + l) for l in range(nl)])]
    xs = normal_bf16((8, T, H), 1.0, 5)
    sg = MTPStepGraph(pool, mw, None, depth=T - 1, top_k=K, single_launch=True)
    for i in range(4):
        sg.step(xs[i % 8])
    torch.cuda.synchronize()
    per_layer = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(40):
            sg.step(xs[i % 8])
        e1.record()
        torch.cuda.synchronize()
        per_layer.append(e0.elapsed_time(e1) * 1000 / 40 / nl)
    per_layer.sort()
    out = [f"T={T}: {per_layer[2]:.2f} us per layer (step graph; median of 5 x 40 steps, min {per_layer[0]:.2f})"]
    buf = torch.zeros(1024 * 16, dtype=torch.int64, device="cuda")
    _lib.check(_lib.lib().ssmoe_set_trace(buf.data_ptr(), buf.numel()))
    try:
        sg.x_in.copy_(xs[3])
        sg.run_eager()
        torch.cuda.synchronize()
    finally:
        _lib.check(_lib.lib().ssmoe_set_trace(None, 0))
    tr = buf.view(1024, 16).cpu().numpy().astype(np.float64)
    prev, last = tr[512:768], tr[:256]
    t0 = prev[:, 0][prev[:, 0] > 0].min()
    tiles = H // 16
    for lay, rows, ex in (("L-2", prev, tr[768:1024]), ("L-1", last, tr[256:512])):
        for table, names in ((rows, MAIN), (ex, EXTRA)):
            for k, nm in names:
                cells = []
                for grp, sl in (("tile", slice(0, tiles)), ("free", slice(tiles, 256))):
                    v = table[sl, k]
                    v = v[v > 0]
                    if v.size:
                        v = (v - t0) / 100.0  # s_memrealtime runs at 100 MHz
                        cells.append(f"{grp} p50 {np.median(v):6.2f} max {v.max():6.2f}")
                if cells:
                    out.append(f"{lay} {nm:>15s}: " + " | ".join(cells))
        out.append(f"{lay} stream poll iterations p50 {np.median(rows[:, 14]):.0f} max {rows[:, 14].max():.0f}")
    return "\n".join(out)


if __name__ == "__main__":
    print(run(int(sys.argv[1]) if len(sys.argv) > 1 else 2, int(sys.argv[2]) if len(sys.argv) > 2 else 16))
