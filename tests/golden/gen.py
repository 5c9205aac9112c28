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


_M64 = (1 << 64) - 1


def _splitmix(v: int) -> int:
    v = (v + 0x9E3779B97F4A7C15) & _M64
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & _M64
    return v ^ (v >> 31)


def sampler_logits(vocab: int, seed: int) -> np.ndarray:
    """The logits the sampler fixtures were drawn over: the reference helper make_logits (engine/sampler.py:27-32),
    uniform in [-4, 4) from the splitmix64 stream, float32 arithmetic."""
    st, out = seed, np.empty(vocab, np.float32)
    for i in range(vocab):
        st = _splitmix(st)
        out[i] = np.float32(st >> 40) / np.float32(1 << 24) * np.float32(8.0) - np.float32(4.0)
    return out


def sampler_uniform(state: int):
    """(next state, u) of the sampler's stream (engine/sampler.py:101-102)."""
    state = _splitmix((state + 1) & _M64)
    return state, np.float32((state >> 11) / float(1 << 53))


def replay_sampler_case(case, logits, draw):
    """Replays one fixture case: draw(logits, generated, params..., u) -> token, with the fixture's seed, penalty
    and accumulation; returns the 16 tokens."""
    state = case["seed"] if case["seed"] != 0 else 0xDEADBEEF
    gen, toks = set(), []
    for _ in range(len(case["tokens"])):
        u = np.float32(0.0)
        if case["temperature"] > 0:
            state, u = sampler_uniform(state)
        tok = draw(logits, gen if case["presence_penalty"] != 0 else (), case["temperature"], case["top_p"],
                   case["top_k"], case["min_p"], case["presence_penalty"], u)
        toks.append(tok)
        if case["accumulate"]:
            gen.add(tok)
    return toks
