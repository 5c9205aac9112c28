"""Test infrastructure (not product code): a plain-Python restatement of the reference slot pool's bookkeeping, the
checker for the native pool (ssmoe_pool_*). Only tests/ may import it.

Follows slotio/src/clock.cpp (Clock::victim, Pins::pin, Pins::retire_below), slotio/src/ensure.cpp
(Ensurer::ensure steps 1-9) and slotio/src/pool.cpp:194-233 (resize_slots, publish / unmap). Records are not
modelled: the model tracks map, owners, reference bits, the hand and the pins, and says which slot every request
gets or which error it raises. Pinned by hand-derived sequences in tests/test_pool_model.py.
"""
from __future__ import annotations


class Exhausted(Exception):
    pass


class PoolModel:
    def __init__(self, layers: int, experts: int, max_slots: int):
        self.layers, self.experts, self.max_slots = layers, experts, max_slots
        self.slots = 0
        self.map = [-1] * (layers * experts)
        self.owner = [-1] * max_slots
        self.ref = [0] * max_slots
        self.hand = 0
        self.pin_gen = [-1] * max_slots
        self.pin_count = 0

    # Pins (clock.cpp: Pins::pin keeps the larger generation)
    def _pin(self, s: int, gen: int) -> None:
        if self.pin_gen[s] < 0:
            self.pin_count += 1
        self.pin_gen[s] = max(self.pin_gen[s], gen)

    def retire_below(self, progress: int) -> None:
        for s in range(self.max_slots):
            if self.pin_gen[s] >= 0 and self.pin_gen[s] < progress:
                self.pin_gen[s] = -1
                self.pin_count -= 1

    # Clock::victim: skip pinned, clear a set reference bit and move on, else take the slot; 3 * slots steps at most
    def _victim(self) -> int:
        for _ in range(3 * self.slots):
            s = self.hand
            self.hand = (self.hand + 1) % self.slots
            if self.pin_gen[s] >= 0:
                continue
            if self.ref[s]:
                self.ref[s] = 0
                continue
            return s
        raise Exhausted("CLOCK found no victim")

    def resize(self, n: int) -> None:
        for s in range(n, self.slots):
            if self.owner[s] >= 0:
                self.map[self.owner[s]] = -1
                self.owner[s] = -1
            self.ref[s] = 0
            if self.pin_gen[s] >= 0:
                self.pin_gen[s] = -1
                self.pin_count -= 1
        if n < self.slots and self.hand >= n:
            self.hand = 0
        self.slots = n

    def ensure(self, layer: int, experts, gen: int, fail_read: bool = False) -> list[int]:
        """Ensurer::ensure. fail_read models a read error after the victims were chosen (step 8)."""
        uniq = []
        for e in experts:
            if e not in uniq:
                uniq.append(e)
        slot = [self.map[layer * self.experts + e] for e in uniq]
        miss = [i for i, s in enumerate(slot) if s < 0]
        unpinned_hits = sum(1 for s in slot if s >= 0 and self.pin_gen[s] < 0)
        if len(miss) > self.slots - self.pin_count - unpinned_hits:
            raise Exhausted("capacity")
        snap = (list(self.pin_gen), self.pin_count)
        for s in slot:
            if s >= 0:
                self._pin(s, gen)
                self.ref[s] = 1
        victims = []
        try:
            for _ in miss:
                v = self._victim()
                self._pin(v, gen)
                victims.append(v)
        except Exhausted:
            self.pin_gen, self.pin_count = snap
            raise
        for v in victims:
            if self.owner[v] >= 0:
                self.map[self.owner[v]] = -1
                self.owner[v] = -1
            self.ref[v] = 0
        if fail_read:
            self.pin_gen, self.pin_count = snap
            raise IOError("read failed")
        for i, v in zip(miss, victims):
            idx = layer * self.experts + uniq[i]
            self.owner[v] = idx
            self.map[idx] = v
            self.ref[v] = 1
            slot[i] = v
        return [slot[uniq.index(e)] for e in experts]
