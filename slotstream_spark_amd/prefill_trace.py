"""Per-block timeline of the prefill grouped GEMM pair (prefill_gemm_kernel) through ssmoe_set_trace.

    python -m slotstream_spark_amd.prefill_trace

Builds one config-3 prefill layer (2048 bf16 tokens, H 2048, 512 experts top-10, I 512, shared 512, affine-4bit gs64,
Zipf 1.1 routing bias) with seeded synthetic weights, runs it three times untraced, then once with the trace on, and
prints for each GEMM: blocks and span, block durations by valid-row class, the number of blocks running at 5 % steps
of the span, busy time per CU and the end of each XCD's last block. Each block stamps its start and end
(s_memrealtime, 100 MHz), its expert and valid rows, and its HW_ID / XCC_ID registers.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .engine.prefill import MoEPrefillLayer
from .memory.slot_pool import SlotPool
from .memory.synth import LayerWeights, normal_bf16, zipf_bias


def run() -> str:
    H, I, E, K, TP = 2048, 512, 512, 10, 2048
    pool = SlotPool(1, E, H, I)
    pool.fill_random(1729)
    pool.place_permuted(1732)
    w = LayerWeights(H, E, 512, seed=1729)
    layer = MoEPrefillLayer(pool, 0, w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, top_k=K,
                            router_bias=zipf_bias(E, 1.1, 1731), max_tokens=TP)
    xp = normal_bf16((TP, H), 1.0, 1733, "cuda")
    for _ in range(3):
        layer(xp)
    torch.cuda.synchronize()
    buf = torch.zeros(16384, dtype=torch.int64, device="cuda")
    _lib.check(_lib.lib().ssmoe_set_trace(buf.data_ptr(), buf.numel()))
    try:
        layer(xp)
        torch.cuda.synchronize()
    finally:
        _lib.check(_lib.lib().ssmoe_set_trace(None, 0))
    tr = buf.cpu().numpy().view(np.uint64)
    out = []
    for name, off in (("gate/up", 0), ("down", 8192)):
        t = tr[off:off + 8192].reshape(-1, 4)
        t = t[t[:, 0] > 0]
        if not len(t):
            out.append(f"{name}: no blocks")
            continue
        t0 = t[:, 0].min()
        st = (t[:, 0] - t0).astype(np.float64) / 100.0
        en = (t[:, 1] - t0).astype(np.float64) / 100.0
        dur = en - st
        nv = (t[:, 2] & np.uint64(0xFFFFFFFF)).astype(np.int64)
        xcc = ((t[:, 3] >> np.uint64(32)) & np.uint64(0xF)).astype(np.int64)
        hw = (t[:, 3] & np.uint64(0xFFFFFFFF)).astype(np.int64)
        cu = (hw >> 8) & 0xF
        se = (hw >> 13) & 0x7
        out.append(f"{name}: {len(t)} blocks, span {en.max():.1f} us")
        for lo, hi in ((1, 32), (33, 64), (65, 96), (97, 128)):
            m = (nv >= lo) & (nv <= hi)
            if m.any():
                out.append(f"  valid rows {lo:3d}-{hi:3d}: {m.sum():5d} blocks, us p50 {np.median(dur[m]):6.1f} "
                           f"min {dur[m].min():6.1f} max {dur[m].max():6.1f}; start p50 {np.median(st[m]):6.1f}")
        grid = np.linspace(0, en.max(), 21)
        out.append("  blocks running at 5 % steps: " + str([int(((st <= x) & (en > x)).sum()) for x in grid]))
        key = xcc * 1000 + se * 100 + cu
        _, inv = np.unique(key, return_inverse=True)
        busy = np.bincount(inv, weights=dur)
        out.append(f"  CUs {busy.size}; busy us per CU p50 {np.median(busy):.1f} min {busy.min():.1f} "
                   f"max {busy.max():.1f}")
        out.append("  last block end per XCD (us): " +
                   " ".join(f"{en[xcc == x].max():.1f}" for x in range(8) if (xcc == x).any()))
    return "\n".join(out)


if __name__ == "__main__":
    print(run())
