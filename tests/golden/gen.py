"""Deterministic inputs of the golden cases (numpy PCG64, stable across numpy versions), shared by make_golden.py
and the tests that replay the fixtures. Distributions follow BASELINE config 0: activations bf16 N(0, 1); router
and shared-expert weights bf16 N(0, 0.02); expert records with uniform nibbles, s = bf16(|N(0, 0.02)|), b = -8 s."""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc


def _bf16(rng, shape, std):
    return orc.f32_to_bf16(rng.normal(0.0, std, shape).astype(np.float32))


def layer_inputs(seed: int, T: int, H: int, E: int, Is: int):
    """(x, router_w, sh_gate, sh_up, sh_down, sh_g) as bf16 bits (uint16)."""
    rng = np.random.default_rng([seed, 1])
    x = _bf16(rng, (T, H), 1.0)
    router_w = _bf16(rng, (E, H), 0.02)
    sh_gate = _bf16(rng, (Is, H), 0.02)
    sh_up = _bf16(rng, (Is, H), 0.02)
    sh_down = _bf16(rng, (H, Is), 0.02)
    sh_g = _bf16(rng, (1, H), 0.02)
    return x, router_w, sh_gate, sh_up, sh_down, sh_g


def record(seed: int, e: int, H: int, I: int) -> np.ndarray:
    """uint8 record of expert e in the reference piece layout."""
    rng = np.random.default_rng([seed, 2, e])
    offs, total = orc.record_offsets(H, I)
    rec = rng.integers(0, 256, total, dtype=np.uint8)
    for (_, s, b) in orc.unpack_record(rec, H, I):
        sv = orc.f32_to_bf16(np.abs(rng.normal(0.0, 0.02, s.shape)).astype(np.float32))
        s[...] = sv
        b[...] = orc.f32_to_bf16(-8.0 * orc.bf16_to_f32(sv))
    return rec
