"""Writes moe_align_ref.npz from the reference's own torch moe_align (kernels/moe_align.py:17-48), run on the CPU in
the build container only; the fixtures, not the reference, travel.

Cases: uniform and Zipf-skewed expert lists, -1 entries (rows outside the current group), entries >= num_local,
block_m 4 / 64 / 128, the config-3 shape (20,480 rows over 512 experts, Zipf 1.1, block 128), and R = 1.

Usage: python -m tests.golden.make_align_golden /root/reference
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
CASES = [  # (name, R, num_local, block_m, kind, seed)
    ("tiny", 20, 4, 4, "uniform_neg", 1), ("r1", 1, 3, 64, "uniform", 2), ("mid", 1000, 64, 64, "zipf", 3),
    ("oob", 300, 8, 128, "oob", 4), ("cfg3", 20480, 512, 128, "zipf", 5), ("skew64", 4096, 32, 64, "zipf_neg", 6),
]


def experts(R, nl, kind, seed):
    rng = np.random.default_rng(seed)
    if kind.startswith("zipf"):
        p = np.arange(1, nl + 1, dtype=np.float64) ** -1.1
        p = p[rng.permutation(nl)]
        le = rng.choice(nl, size=R, p=p / p.sum())
    else:
        le = rng.integers(0, nl, size=R)
    if kind.endswith("neg"):
        le[rng.random(R) < 0.2] = -1
    if kind == "oob":
        le[rng.random(R) < 0.15] = nl + 3
        le[rng.random(R) < 0.1] = -1
    return le.astype(np.int32)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from slotstream_spark.kernels.moe_align import moe_align

    arrays = {}
    for name, R, nl, bm, kind, seed in CASES:
        le = experts(R, nl, kind, seed)
        s, b, n = moe_align(torch.from_numpy(le), nl, bm)
        arrays[name + "_le"] = le
        arrays[name + "_meta"] = np.array([R, nl, bm], np.int64)
        arrays[name + "_sorted"], arrays[name + "_block"] = s.numpy(), b.numpy()
        arrays[name + "_num"] = n.numpy()
    np.savez_compressed(HERE / "moe_align_ref.npz", **arrays)
    print("wrote", HERE / "moe_align_ref.npz")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
