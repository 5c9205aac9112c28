"""Expert slot pool resident in HBM, with the reference's table ABI.

The reference keeps expert records in host-memory slots and hands the kernels two device-visible tables:
`map` int32 [layers * E] (expert of a layer -> slot, -1 = not resident) and `slot_ptr` int64 [n_slots]
(slot -> record base address) (slotio/include/slotio/pool.hpp:39-92, runtime/pool.py:89-100). On MI355X every
expert of every layer fits in the 288 GB of HBM, so the pool here is one device allocation of n_slots records
(each a multiple of 256 bytes, so every piece stays 16-byte aligned for 128-bit loads) and both tables live in HBM.
Records keep the reference piece layout (gate.w gate.s gate.b up.w up.s up.b down.w down.s down.b;
docs/model-and-repack.md:39-53): an MLX weight row is contiguous, which is what the kernels' 16-byte-per-lane
loads need, so no repacking is required.
"""
from __future__ import annotations

import torch

from .. import _lib


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


class SlotPool:
    def __init__(self, layers: int, experts: int, hidden: int, inter: int, n_slots: int | None = None,
                 device: str | torch.device = "cuda"):
        self.layers, self.experts, self.hidden, self.inter = layers, experts, hidden, inter
        self.offsets, self.record_bytes = _lib.record_layout(hidden, inter)
        self.stride = _align(self.record_bytes)
        self.n_slots = layers * experts if n_slots is None else n_slots
        self.device = torch.device(device)
        self.storage = torch.empty(self.n_slots * self.stride, dtype=torch.uint8, device=self.device)
        base = self.storage.data_ptr()
        self.slot_ptr = torch.tensor([base + s * self.stride for s in range(self.n_slots)], dtype=torch.int64,
                                     device=self.device)
        self.map = torch.full((layers * experts,), -1, dtype=torch.int32, device=self.device)

    # Reference ExpertPool property names (runtime/pool.py:89-100).
    @property
    def map_tensor(self) -> torch.Tensor:
        return self.map

    @property
    def slot_ptr_tensor(self) -> torch.Tensor:
        return self.slot_ptr

    def slots(self) -> torch.Tensor:
        """[n_slots, stride] uint8 view of the pool."""
        return self.storage.view(self.n_slots, self.stride)

    def record(self, slot: int) -> torch.Tensor:
        return self.slots()[slot, : self.record_bytes]

    def assign(self, layer: int, slot_of_expert) -> None:
        """map[layer * E + e] = slot_of_expert[e] for the E experts of one layer."""
        s = torch.as_tensor(slot_of_expert, dtype=torch.int32, device=self.device)
        if s.numel() != self.experts:
            raise ValueError(f"need {self.experts} slots, got {s.numel()}")
        self.map[layer * self.experts:(layer + 1) * self.experts] = s

    def place_permuted(self, seed: int) -> None:
        """Every layer's experts in a seeded random permutation of its own block of slots."""
        g = torch.Generator().manual_seed(seed)
        for layer in range(self.layers):
            perm = torch.randperm(self.experts, generator=g).to(torch.int32) + layer * self.experts
            self.assign(layer, perm)

    def write_record(self, slot: int, record: torch.Tensor) -> None:
        if record.dtype != torch.uint8 or record.numel() != self.record_bytes:
            raise ValueError(f"record must be uint8 [{self.record_bytes}]")
        self.record(slot).copy_(record.reshape(-1))

    def fill_random(self, seed: int, slots: slice | None = None) -> None:
        """Synthetic MLX-style affine 4-bit records: q uniform in 0..15 (uniform random bytes), s = bf16(|N(0,
        0.02)|), b = bf16(-8 s) (exact), generated on the pool's device."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        view = self.slots()[slots if slots is not None else slice(None)]
        o = self.offsets
        H, I = self.hidden, self.inter
        w_gu, sb_gu = I * H // 2, I * (H // 64) * 2
        w_d, sb_d = H * I // 2, H * (I // 64) * 2
        for ow, os_, ob, wsz, ssz in ((o[0], o[1], o[2], w_gu, sb_gu), (o[3], o[4], o[5], w_gu, sb_gu),
                                      (o[6], o[7], o[8], w_d, sb_d)):
            view[:, ow: ow + wsz].random_(0, 256, generator=g)
            n = ssz // 2
            s = (torch.randn((view.shape[0], n), generator=g, device=self.device).abs_() * 0.02).to(torch.bfloat16)
            view[:, os_: os_ + ssz].view(torch.bfloat16).copy_(s)
            view[:, ob: ob + ssz].view(torch.bfloat16).copy_(s * -8)


def pack_record(gate, up, down, hidden: int, inter: int) -> torch.Tensor:
    """One record from three (q int32 [N, K/8], s bf16 [N, K/64], b bf16 [N, K/64]) pieces (gate/up [I, H],
    down [H, I]) -> uint8 [record_bytes] on the pieces' device (tools/repack_experts.py piece order)."""
    offs, total = _lib.record_layout(hidden, inter)
    dev = gate[0].device
    rec = torch.zeros(total, dtype=torch.uint8, device=dev)
    for p, piece in enumerate((gate, up, down)):
        for t, off in zip(piece, offs[3 * p: 3 * p + 3]):
            raw = t.contiguous().view(torch.uint8).reshape(-1)
            rec[off: off + raw.numel()] = raw
    return rec
