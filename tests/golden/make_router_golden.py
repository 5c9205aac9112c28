"""Writes router_ref.npz: the reference CPU router (model/reference_torch.py:121-124: bf16 F.linear, fp32 softmax,
torch.topk) on 64 seeded config-1-shaped inputs (H 2048, E 512, top-10; T = 2 for even seeds, 4 for odd ones), with
and without the Zipf(1.1) routing bias of BASELINE config 1 (added in fp32 to the bf16 logits, as the bench does).

Only torch is called: the reference's router is these three torch calls, so no reference module is imported. The
fixtures record which torch build and CPU produced them, because the fp32 accumulation order of torch's CPU bf16
GEMM belongs to the library and to the instruction set it dispatches to.

Usage: python -m tests.golden.make_router_golden
"""
from __future__ import annotations

import json
import platform
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SEEDS = list(range(100, 164))
H, E, K = 2048, 512, 10


def inputs(seed: int):
    """(x bf16 bits [T, H], router_w bf16 bits [E, H], Zipf bias fp32 [E]) of one case."""
    from tests.golden import gen

    T = 2 if seed % 2 == 0 else 4
    rng = np.random.default_rng([seed, 1])
    x = gen._bf16(rng, (T, H), 1.0)
    rw = gen._bf16(rng, (E, H), 0.02)
    r = np.arange(1, E + 1, dtype=np.float64)
    logp = -1.1 * np.log(r) - np.log((r ** -1.1).sum())
    bias = np.empty(E, np.float64)
    bias[np.random.default_rng([seed, 3]).permutation(E)] = logp
    return x, rw, bias.astype(np.float32)


def main() -> None:
    import torch
    import torch.nn.functional as F

    arrays, meta = {}, []
    for seed in SEEDS:
        x, rw, bias = inputs(seed)
        xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
        wt = torch.from_numpy(rw.view(np.int16)).view(torch.bfloat16)
        logits = F.linear(xt, wt)
        probs = F.softmax(logits, dtype=torch.float, dim=-1)
        tv, ids = torch.topk(probs, K, dim=-1)
        probs_b = F.softmax(logits.float() + torch.from_numpy(bias), dtype=torch.float, dim=-1)
        tv_b, ids_b = torch.topk(probs_b, K, dim=-1)
        key = f"s{seed}"
        arrays[key + "_logits"] = logits.view(torch.int16).numpy().view(np.uint16)
        arrays[key + "_ids"] = ids.to(torch.int32).numpy()
        arrays[key + "_topv"] = tv.numpy()
        arrays[key + "_ids_bias"] = ids_b.to(torch.int32).numpy()
        arrays[key + "_topv_bias"] = tv_b.numpy()
        meta.append(dict(seed=seed, T=int(x.shape[0])))
    arrays["meta"] = np.frombuffer(json.dumps(dict(
        cases=meta, H=H, E=E, K=K, torch=torch.__version__, numpy=np.__version__, cpu=platform.processor() or
        platform.machine(), source="model/reference_torch.py:121-124 (F.linear bf16, softmax fp32, torch.topk)")
    ).encode(), dtype=np.uint8)
    np.savez_compressed(HERE / "router_ref.npz", **arrays)


if __name__ == "__main__":
    main()
