"""Seeded synthetic inputs of the BASELINE configurations (random-init weights; there is no checkpoint).

Distributions: activations bf16 N(0, 1); router gate bf16 N(0, 0.02) [E, H]; shared
expert gate/up [Is, H], down [H, Is] and shared_expert_gate [1, H] bf16 N(0, 0.02); expert records as in
SlotPool.fill_random. Routing skew: Zipf(s) popularity over a seeded permutation of the experts, realised as an
fp32 bias ln p_rank(e) added to the router logits. Verify logits: target N(0, 3) fp32, draft = rho * target +
sqrt(1 - rho^2) * N(0, 3).
"""
from __future__ import annotations

import math

import torch


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=torch.device(device)).manual_seed(seed)


def normal_bf16(shape, std: float, seed: int, device="cuda") -> torch.Tensor:
    g = _gen(seed, device)
    return (torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)


def zipf_bias(experts: int, s: float = 1.1, seed: int = 1731, device="cuda") -> torch.Tensor:
    """bias[e] = ln p_rank(e), p_r proportional to r^-s (r = 1..E) over a seeded permutation of the experts."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(experts, generator=g)
    r = torch.arange(1, experts + 1, dtype=torch.float64)
    logp = -s * torch.log(r) - math.log(float((r ** -s).sum()))
    bias = torch.empty(experts, dtype=torch.float64)
    bias[perm] = logp
    return bias.to(torch.float32).to(device)


def affine4(rows: int, cols: int, seed: int, scale: float = 0.02 / 4.6, device="cuda"):
    """A synthetic affine 4-bit (gs 64) weight [rows, cols] in the layout of the reference checkpoint's quantized
    linears (model/weights.py:84-92): q uniform in 0..15 (random words), s = bf16(|N(0, scale)|), b = bf16(-8 s),
    so w = s (q - 8) has about the spread of N(0, 4.6 scale)."""
    from ..kernels.gemv_affine import AffineWeight

    g = _gen(seed, device)
    q = torch.randint(-2**31, 2**31 - 1, (rows, cols // 8), generator=g, device=device, dtype=torch.int32)
    s = (torch.randn((rows, cols // 64), generator=g, device=device) * scale).abs().to(torch.bfloat16)
    return AffineWeight(q, s, (-8 * s.float()).to(torch.bfloat16), 4, 64, rows, cols)


class LayerWeights:
    """Router and shared-expert weights of one synthetic MoE layer; `shared_q4` makes the shared expert's gate, up
    and down projections affine 4-bit AffineWeights (the router and the shared_expert_gate row stay bf16, dense in
    the reference checkpoint)."""

    def __init__(self, hidden: int, experts: int, shared_inter: int, seed: int, device="cuda", shared_q4=False):
        self.router_w = normal_bf16((experts, hidden), 0.02, seed * 8 + 1, device)
        if shared_q4:
            self.sh_gate = affine4(shared_inter, hidden, seed * 8 + 2, device=device)
            self.sh_up = affine4(shared_inter, hidden, seed * 8 + 3, device=device)
            self.sh_down = affine4(hidden, shared_inter, seed * 8 + 4, device=device)
        else:
            self.sh_gate = normal_bf16((shared_inter, hidden), 0.02, seed * 8 + 2, device)
            self.sh_up = normal_bf16((shared_inter, hidden), 0.02, seed * 8 + 3, device)
            self.sh_down = normal_bf16((hidden, shared_inter), 0.02, seed * 8 + 4, device)
        self.sh_g = normal_bf16((1, hidden), 0.02, seed * 8 + 5, device)

    def nbytes(self) -> int:
        def nb(t):
            return t.q.numel() * 4 + t.s.numel() * 4 if hasattr(t, "q") else t.numel() * 2
        return sum(nb(t) for t in (self.router_w, self.sh_gate, self.sh_up, self.sh_down, self.sh_g))


def verify_logits(depth: int, vocab: int, seed: int, rho: float = 0.8, std: float = 3.0, device="cuda"):
    """(target fp32 [depth+1, vocab], draft fp32 [depth, vocab]) with draft rows correlated rho to the target."""
    g = _gen(seed, device)
    z = torch.randn((depth + 1, vocab), generator=g, device=device) * std
    n = torch.randn((depth, vocab), generator=g, device=device) * std
    return z, rho * z[:depth] + math.sqrt(1.0 - rho * rho) * n


def head_weights(hidden: int, hc: int, lowrank: int, vocab: int, seed: int, device="cuda"):
    """Random-init dense weights of the MTP head (engine.mtp.HeadWeights): embedding table N(0, 1) [vocab, H]; norm
    weights 1 + N(0, 0.1); every projection N(0, 1 / fan_in), so activations keep unit scale through the step."""
    from ..engine.mtp import HeadWeights, HyperConnection

    n = hc * hidden
    k = iter(range(seed * 32, seed * 32 + 32))

    def norm_w(size):
        return (normal_bf16((size,), 0.1, next(k), device).float() + 1).to(torch.bfloat16)

    def proj(rows, cols):
        return normal_bf16((rows, cols), cols ** -0.5, next(k), device)

    def hcw(inject):
        return HyperConnection(norm_w(n), proj(lowrank, n), proj(n, lowrank), proj(hc, n) if inject else None)

    return HeadWeights(embed=normal_bf16((vocab, hidden), 1.0, next(k), device),
                       pre_fc_norm_embedding=norm_w(hidden), fc_embedding=proj(hidden, hidden),
                       pre_fc_norm_hidden=norm_w(n), fc_hidden=proj(hidden, hidden), mlp_hc=hcw(True),
                       mixer_hc=hcw(False))
