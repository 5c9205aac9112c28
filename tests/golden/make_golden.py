"""Writes the golden fixtures from the reference's own CPU functions (run in the build container only; the
fixtures, not the reference, travel).

  moe_ref_cases.npz  model/reference_torch.py:118-134 (moe_ref) on config-0 and config-1-shaped layers (no bias:
                     the reference router has none): router logits of the F.linear call moe_ref makes, its top-k
                     ids, and its output y (bf16 bits). Inputs are regenerated from tests/golden/gen.py.
  sampler_ref.json   engine/sampler.py Sampler.next draws over make_logits(vocab, 99) for a grid of parameters.

Pins what only the reference's torch/numpy calls define: the bf16 rounding of F.linear's router logits, torch.topk
tie order, and numpy's float32 exp / pairwise sum inside the sampler. Fixture metadata records the library
versions, since the reference pins torch 2.13 and this container has another.

Usage: python -m tests.golden.make_golden /root/reference
"""
from __future__ import annotations

import itertools
import json
import random
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
CASES = [  # (seed, T, H, E, K, I, Is)
    (0, 2, 2048, 64, 4, 512, 512), (1, 2, 2048, 64, 4, 512, 512), (2, 2, 2048, 64, 4, 512, 512),
    (3, 4, 2048, 64, 4, 512, 512), (4, 2, 2048, 512, 10, 512, 512), (5, 2, 2048, 512, 10, 512, 512),
]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from slotstream_spark.engine import sampler as ref_sampler
    from slotstream_spark.model.reference_torch import moe_ref

    from oracle import oracle as orc
    from tests.golden import gen

    torch.manual_seed(0)
    arrays, meta = {}, []
    for (seed, T, H, E, K, I, Is) in CASES:
        xs = gen.layer_inputs(seed, T, H, E, Is)
        x, rw, sg, su, sd, sgg = (torch.from_numpy(a.view(np.int16)).view(torch.bfloat16) for a in xs)
        cache = {}

        def expert(layer, e, seed=seed, H=H, I=I, cache=cache):
            if e not in cache:
                g, u, d = orc.expert_dense(gen.record(seed, e, H, I), H, I, np.float32)
                cache[e] = (torch.from_numpy(g), torch.from_numpy(u), torch.from_numpy(d))
            return cache[e]

        y, ti = moe_ref(x, rw, K, expert, 0, sg, su, sd, sgg)
        logits = torch.nn.functional.linear(x, rw)  # the call moe_ref makes first
        probs = torch.softmax(logits, dtype=torch.float, dim=-1)
        key = f"s{seed}"
        arrays[key + "_logits"] = logits.view(torch.int16).numpy().view(np.uint16)
        arrays[key + "_probs"] = probs.numpy()
        arrays[key + "_ids"] = ti.to(torch.int32).numpy()
        arrays[key + "_y"] = y.view(torch.int16).numpy().view(np.uint16)
        meta.append(dict(seed=seed, T=T, H=H, E=E, K=K, I=I, Is=Is))
    arrays["meta"] = np.frombuffer(json.dumps(dict(
        cases=meta, torch=torch.__version__, numpy=np.__version__,
        source="model/reference_torch.py:118-134 moe_ref")).encode(), dtype=np.uint8)
    np.savez_compressed(HERE / "moe_ref_cases.npz", **arrays)

    grid = list(itertools.product((0.0, 0.6, 0.8, 1.2), (1.0, 0.95, 0.5), (0, 1, 40), (0.0, 0.05),
                                  (0.0, 1.5), (True, False), (256, 4096, 151936), (7, 0, 12345)))
    cases = random.Random(2718).sample(grid, 48)
    out = []
    for (t, tp, tk, mp, pp, acc, vocab, seed) in cases:
        p = ref_sampler.SampleParams(temperature=t, top_p=tp, top_k=tk, min_p=mp, presence_penalty=pp)
        logits = ref_sampler.make_logits(vocab, 99)
        s, generated, toks = ref_sampler.Sampler(seed), set(), []
        for _ in range(16):
            tok = s.next(logits, p, generated)
            toks.append(tok)
            if acc:
                generated.add(tok)
        out.append(dict(temperature=t, top_p=tp, top_k=tk, min_p=mp, presence_penalty=pp, accumulate=acc,
                        vocab=vocab, seed=seed, tokens=toks))
    (HERE / "sampler_ref.json").write_text(json.dumps(dict(
        source="engine/sampler.py Sampler.next over make_logits(vocab, 99)", numpy=np.__version__,
        cases=out), indent=0))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
