"""Phase trace of the one-launch p/q acceptance round (ssmoe_accept_pq) through ssmoe_set_trace.

    python -m slotstream_spark_amd.accept_trace [D] [V] [bonus]

Runs BASELINE config 2's round (depth D = 3, vocab V = 151,936, temperature 0.7) on seeded synthetic logits with
drafts drawn from q, times 200 rounds in one HIP graph (HIP events; the greedy round on the same target rows
likewise), then runs one eager round with the trace on and
prints, for every stamp, the median and maximum over the workgroups that wrote it, in us from the first workgroup
start. Stamps 0-6 are per workgroup; 8-11 come from the waves that hold a chunk of the sampled row. With bonus = 1 the
draft rows equal the target rows, so every draft is accepted and the bonus row is sampled.
"""
from __future__ import annotations

import sys

import numpy as np
import torch

from . import _lib
from .engine.accept import Acceptor, UniformStream
from .memory.synth import verify_logits

NAMES = [(0, "start"), (12, "logits loaded"), (13, "target chunk part"), (1, "chunk parts stored"), (2, "all chunk parts seen"), (3, "parts staged"),
         (4, "row statistics"), (5, "decision"), (8, "sampled values stored"), (9, "all sampled totals seen"),
         (10, "chunk of the sample found"), (11, "round written"), (6, "workgroup done")]


def run(D: int = 3, V: int = 151936, bonus: int = 0, temp: float = 0.7) -> str:
    acc = Acceptor(D, V)
    tgt, drf = verify_logits(D, V, 4242)
    if bonus:
        drf = tgt[:D].contiguous()
    u = torch.from_numpy(UniformStream(7).peek(D + 1)).cuda()
    drafts = acc.draw_drafts_async(drf, u[:D].contiguous(), temp)
    for _ in range(20):
        acc.pq_async(tgt, drf, drafts, u, temp)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(200):
                acc.pq_async(tgt, drf, drafts, u, temp)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(5):
        with torch.cuda.stream(s):
            e0.record(s)
            g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1000 / 200)
    times.sort()
    out = [f"D={D} V={V}: {times[2]:.2f} us per round (graph of 200 rounds; median of 5, min {times[0]:.2f})"]
    gg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(gg, stream=s):
            for _ in range(200):
                acc.greedy_async(tgt, drafts)
    gt = []
    for _ in range(5):
        with torch.cuda.stream(s):
            e0.record(s)
            gg.replay()
            e1.record(s)
        torch.cuda.synchronize()
        gt.append(e0.elapsed_time(e1) * 1000 / 200)
    gt.sort()
    out.append(f"greedy round: {gt[2]:.2f} us (graph of 200 rounds; median of 5, min {gt[0]:.2f})")
    buf = torch.zeros(1024 * 16, dtype=torch.int64, device="cuda")
    _lib.check(_lib.lib().ssmoe_set_trace(buf.data_ptr(), buf.numel()))
    try:
        acc.pq_async(tgt, drf, drafts, u, temp)
        torch.cuda.synchronize()
    finally:
        _lib.check(_lib.lib().ssmoe_set_trace(None, 0))
    res = acc.out.cpu().numpy()
    nch = (V + 1023) // 1024
    grid = ((D + 1) * nch + 3) // 4
    st = buf.cpu().numpy().reshape(1024, 16)[:grid].astype(np.float64)
    t0 = st[:, 0][st[:, 0] > 0].min()
    out.append(f"{grid} workgroups; round: accepted {res[0]}, emitted {res[1]}, tokens {res[4:4 + res[1]].tolist()}")
    for k, name in NAMES:
        v = st[:, k]
        v = (v[v > 0] - t0) / 100.0  # s_memrealtime: 100 MHz
        if v.size:
            out.append(f"{name:>26s}: p50 {np.median(v):6.2f} max {v.max():6.2f} us ({v.size} workgroups)")
    return "\n".join(out)


if __name__ == "__main__":
    args = [int(a) for a in sys.argv[1:]]
    print(run(*args))
