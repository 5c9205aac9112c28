"""Writes mtp_ref.npz from the reference's own torch CPU functions (run in the build container only; the fixtures, not
the reference, travel):

  rmsnorm          model/reference_torch.py:30-38 rmsnorm, full width and per group of H (the two uses of the MTP
                   head: pre_fc_norm_* in fuse, engine/mtp.py:189-190, and hc_norm in hc_mix, model/layers.py:192)
  gated_residual   model/reference_torch.py:174-183 RefModel.gated_residual, the CPU-backend twin of Segments.hc_mix
                   (model/layers.py:190-198), with and without the injection

on small seeded bf16 inputs (hc 4, H 128, low rank 48, 3 rows). engine/mtp.py itself imports tomllib, which this
image's Python 3.10 lacks, so fuse and the head step are pinned by closed forms instead (tests/test_mtp_oracle.py).

Usage: python -m tests.golden.make_mtp_golden /root/reference
"""
from __future__ import annotations

import json
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np

HERE = Path(__file__).resolve().parent
HC, H, LOW, S, EPS = 4, 128, 48, 3, 1e-6


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from slotstream_spark.model import reference_torch as R

    g = torch.Generator().manual_seed(2026)

    def rnd(shape, std, mean=0.0):
        return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)

    n = HC * H
    arrays = {}
    # Branch scales differ so a per-group and a full-width norm disagree.
    scale = torch.tensor([0.5, 1.0, 2.0, 4.0]).repeat_interleave(H)
    x = (torch.randn(S, n, generator=g) * scale).to(torch.bfloat16)
    w = rnd((n,), 0.1, 1.0)
    arrays["norm_x"], arrays["norm_w"] = _bits(x), _bits(w)
    arrays["norm_full"] = _bits(R.rmsnorm(x, w, EPS))
    arrays["norm_group"] = _bits(R.rmsnorm(x, w, EPS, group=H))

    P = {"p.hc_norm.weight": rnd((n,), 0.1, 1.0), "p.input_mix_weight_down.weight": rnd((LOW, n), n ** -0.5),
         "p.input_mix_weight_up.weight": rnd((n, LOW), 2 * LOW ** -0.5),
         "p.block_inject_weight.weight": rnd((HC, n), n ** -0.5)}
    hyp = (torch.randn(S, n, generator=g) * scale).to(torch.bfloat16)
    fake = SimpleNamespace(w=lambda name: P[name], eps=EPS, hc=HC, H=H)
    mixed, inj = R.RefModel.gated_residual(fake, "p", hyp)
    mixed_ni, none = R.RefModel.gated_residual(fake, "p", hyp, inject=False)
    assert none is None
    arrays["hc_hyp"] = _bits(hyp)
    for k, v in P.items():
        arrays["hc_" + k.split(".")[1]] = _bits(v)
    arrays["hc_mixed"], arrays["hc_inj"], arrays["hc_mixed_noinject"] = _bits(mixed), _bits(inj), _bits(mixed_ni)
    meta = {"torch": torch.__version__, "hc": HC, "H": H, "low": LOW, "S": S, "eps": EPS,
            "source": "slotstream_spark/model/reference_torch.py rmsnorm, RefModel.gated_residual"}
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), np.uint8)
    np.savez_compressed(HERE / "mtp_ref.npz", **arrays)
    print("wrote", HERE / "mtp_ref.npz", {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
