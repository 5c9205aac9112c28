"""Rollback of a verify round (drop-in for slotstream_spark/engine/rollback.py:1-41 and the StepRecord of
kernels/gdn_step_record.py:19-56).

A round runs `rows` tokens (the pending one and the drafts) through the verify pass. The tokens kept are the first
`keep`: the per-row state the pass recorded comes back from the record, and the position and the token list are
cut to the checkpoint plus `keep`. `Checkpoint`, `checkpoint` and `rollback` keep the reference's fields, checks and
error messages.

StepRecord is the reference's ring, generalised to whatever per-row state a stack carries between rounds: for each
named live tensor of the sequence state it holds `rows` snapshots, the pass writes snapshot i after row i, and
`restore(st, keep)` copies snapshot keep - 1 back. The MoE path's stack has no recurrent GDN, conv or PLE state
(those are outside it), so its record is empty and a rollback is position and token bookkeeping; a stack with state
registers it here. `restore_async` takes `keep` as a device int32 (the n_emit of a greedy round's result vector)
and restores with the row-gather kernel, so a captured round can roll back without reading the decision.

`Checkpoint`, `checkpoint()` and `rollback()` follow fortil/slotstream-spark engine/rollback.py:15-41 (fields, body,
checks and error strings: the drop-in contract). That file, itself a port of slotstream's Generate.swift and
Model.swift (MIT, Copyright (c) 2026 Carlos Galarza), is under the MIT License:

    Copyright (c) 2026 William Penagos

    Permission is hereby granted, free of charge, to any person obtaining a copy of this software and associated
    documentation files (the "Software"), to deal in the Software without restriction, including without limitation
    the rights to use, copy, modify, merge, publish, distribute, sublicense, and/or sell copies of the Software, and
    to permit persons to whom the Software is furnished to do so, subject to the following conditions: The above
    copyright notice and this permission notice shall be included in all copies or substantial portions of the
    Software. THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR IMPLIED, INCLUDING BUT NOT
    LIMITED TO THE WARRANTIES OF MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT
    SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION
    OF CONTRACT, TORT OR OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER
    DEALINGS IN THE SOFTWARE.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class Checkpoint:
    pos: int
    ntokens: int


@dataclass
class SeqState:
    """What a sequence carries between rounds: position, token list, named per-sequence state tensors (recorded by
    StepRecord) and attention caches (none on the MoE path; each would have `pos` and `last`)."""
    pos: int = 0
    tokens: list = field(default_factory=list)
    state: dict = field(default_factory=dict)
    attn: dict = field(default_factory=dict)


def checkpoint(model) -> Checkpoint:
    st = model.st
    return Checkpoint(int(st.pos), len(st.tokens))


def rollback(model, record, ck: Checkpoint, keep: int, rows: int = 3) -> None:
    """Keep the first `keep` (1..rows) rows of the round that started at `ck`; releases the round's record."""
    if not 1 <= keep <= rows:
        raise ValueError(f"keep must be in 1..{rows}, got {keep}")
    st = model.st
    if st.pos != ck.pos + rows:
        raise RuntimeError(f"rollback: state at {st.pos}, expected the checkpoint {ck.pos} + {rows} rows")
    if keep == rows:
        record.release()
    else:
        record.restore(st, keep)
    st.pos = ck.pos + keep
    del st.tokens[ck.ntokens + keep:]
    for c in st.attn.values():
        c.pos = st.pos
        c.last = None


class StepRecord:
    """The ring bound to the state tensors of one SeqState: ring[name] [rows, *shape]. `outstanding` counts rounds
    whose record has not been consumed (restored from or released)."""

    def __init__(self, st: SeqState, rows: int = 3):
        self.rows = rows
        self.ring = {name: torch.zeros((rows, *t.shape), dtype=t.dtype, device=t.device) for name, t in st.state.items()}
        self.outstanding = 0
        self.rounds = 0

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.ring.values())

    def begin(self) -> None:
        """A verify round is about to run (the pass writes the ring)."""
        self.outstanding += 1
        self.rounds += 1

    def release(self) -> None:
        if self.outstanding <= 0:
            raise RuntimeError("StepRecord.release without a matching begin")
        self.outstanding -= 1

    def restore(self, st: SeqState, keep: int) -> None:
        """State after the first `keep` rows of the round (1 <= keep <= rows) -> st, then release the round."""
        if not 1 <= keep <= self.rows:
            raise ValueError(f"keep must be in 1..{self.rows}, got {keep}")
        for name, ring in self.ring.items():
            st.state[name].copy_(ring[keep - 1])
        self.release()

    def restore_async(self, st: SeqState, keep: torch.Tensor) -> None:
        """restore() with `keep` an int32 device scalar (1..rows), read by the gather kernel: no host synchronisation,
        capturable. A keep outside 1..rows zeroes the state and raises SSMOE_ERR_TOKEN in the device status."""
        from ..kernels.head_ops import gather_rows

        for name, ring in self.ring.items():
            dst = st.state[name]
            gather_rows(ring, keep.view(1), idx_add=-1, out=dst.view(1, *dst.shape))
        self.release()
