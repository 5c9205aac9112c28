"""Helpers shared by the GPU parity tests (not collected: no test_ prefix)."""
import numpy as np
import torch

from oracle import oracle as O
from slotstream_spark_amd.memory.slot_pool import SlotPool


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 numpy bits (host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def make_pool(experts, hidden, inter, seed, layers=1, permute=True, device="cuda"):
    pool = SlotPool(layers, experts, hidden, inter, device=device)
    pool.fill_random(seed)
    if permute:
        pool.place_permuted(seed + 1)
    else:
        for layer in range(layers):
            pool.assign(layer, list(range(layer * experts, (layer + 1) * experts)))
    return pool


class DenseCache:
    """fp64 dequantized experts of a pool layer, read back from the device records on demand."""

    def __init__(self, pool, layer=0):
        self.pool, self.layer = pool, layer
        self.map = pool.map.cpu().numpy()
        self.cache = {}

    def record(self, e):
        slot = int(self.map[self.layer * self.pool.experts + e])
        return self.pool.record(slot).cpu().numpy()

    def __call__(self, e):
        if e not in self.cache:
            self.cache[e] = O.expert_dense(self.record(e), self.pool.hidden, self.pool.inter, np.float64)
        return self.cache[e]


def rand_ids(r, k, experts, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(experts, generator=g)[:k] for _ in range(r)]).to(torch.int32)


def rand_weights(r, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.softmax(torch.randn(r, k, generator=g), dim=-1)


def rand_x(r, h, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(r, h, generator=g).to(dtype)
