"""Acceptance of an MTP verify round on the device: greedy argmax-match and p/q rejection sampling.

Greedy follows the acceptance loop of _mtp_decode (slotstream_spark/engine/generate.py:208-229) at temperature 0
(Sampler.next -> np.argmax, engine/sampler.py:83-84): row i's token is the first maximum of its logits; the round
accepts drafts while they equal those tokens and emits tokens 0..good; a row holding a non-finite logit stops the
round before it (generate.py:210-212). `sampled` is the same loop with the full reference sampler (temperature,
top-k, top-p, min-p, presence penalty over the tokens seen so far). p/q is Leviathan et al. 2023, Alg. 1, which the
reference does not have. Alg. 1 preserves the target distribution only when each draft token x_i is drawn from the
q_i it divides by: `draw_drafts_async` draws x_i ~ softmax(draft_i / temperature) on the device (ssmoe_sample_rows)
and `pq_round` is the whole proposal + acceptance step. The reference's greedy drafts (engine/mtp.py:265-277) are
the temperature-0 proposal, valid for the greedy round only.

The uniforms come from the reference sampler's splitmix64 stream (engine/sampler.py:20-24, 101-102), drawn on the
host: decision i consumes uniforms[i], the final sample the next one; `n_uniform` reports how many were used, so
the stream advances exactly as a sequential host implementation would.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .. import _lib

FLAG_NONFINITE, FLAG_BAD_DRAFT, FLAG_RESIDUAL_EMPTY, FLAG_FALLBACK = 1, 2, 4, 8

_M64 = (1 << 64) - 1


def _splitmix(v: int) -> int:
    v = (v + 0x9E3779B97F4A7C15) & _M64
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & _M64
    return v ^ (v >> 31)


class UniformStream:
    """The sampler's generator (Sampler.__init__/next, engine/sampler.py:73-74, 101-102): state advances by
    splitmix(state + 1) per draw and u = float32((state >> 11) / 2^53)."""

    def __init__(self, seed: int = 0):
        self.state = seed if seed != 0 else 0xDEADBEEF

    def peek(self, n: int) -> np.ndarray:
        st, out = self.state, np.empty(n, np.float32)
        for i in range(n):
            st = _splitmix((st + 1) & _M64)
            out[i] = np.float32((st >> 11) / float(1 << 53))
        return out

    def advance(self, n: int) -> None:
        for _ in range(n):
            self.state = _splitmix((self.state + 1) & _M64)


@dataclass
class AcceptResult:
    n_accept: int
    n_emit: int
    n_uniform: int
    flags: int
    tokens: list = field(default_factory=list)

    @staticmethod
    def from_out(out) -> "AcceptResult":
        o = [int(v) for v in out]
        return AcceptResult(o[0], o[1], o[2], o[3], o[4: 4 + o[1]])


class Acceptor:
    """Device acceptance for depth D over a V-token vocabulary (workspace and output owned here)."""

    def __init__(self, depth: int, vocab: int, device="cuda"):
        self.depth, self.vocab = depth, vocab
        nb = _lib.lib().ssmoe_accept_workspace_bytes(depth, vocab)
        self.work = torch.zeros(int(nb), dtype=torch.uint8, device=device)  # header zero before the first call
        self.out = torch.empty(depth + 5, dtype=torch.int32, device=device)
        self._swork = None
        self._dwork = None

    def _check(self, target, draft=None):
        d, v = self.depth, self.vocab
        if target.dtype != torch.float32 or tuple(target.shape) != (d + 1, v) or not target.is_contiguous():
            raise ValueError(f"target must be contiguous fp32 [{d + 1}, {v}]")
        if draft is not None and (draft.dtype != torch.float32 or tuple(draft.shape) != (d, v)
                                  or not draft.is_contiguous()):
            raise ValueError(f"draft must be contiguous fp32 [{d}, {v}]")

    def greedy_async(self, target: torch.Tensor, drafts: torch.Tensor) -> torch.Tensor:
        """Launch only; returns the device output int32 [D+5] (n_accept, n_emit, n_uniform, flags, tokens)."""
        self._check(target)
        if drafts.dtype != torch.int32 or drafts.numel() != self.depth:
            raise ValueError(f"drafts must be int32 [{self.depth}]")
        _lib.check(_lib.lib().ssmoe_accept_greedy(target.data_ptr(), drafts.data_ptr(), self.depth, self.vocab,
                                                  self.work.data_ptr(), self.work.numel(), self.out.data_ptr(),
                                                  _lib.stream_of(target)))
        return self.out

    def pq_async(self, target, draft, drafts, uniforms, temperature: float) -> torch.Tensor:
        self._check(target, draft)
        if drafts.dtype != torch.int32 or drafts.numel() != self.depth:
            raise ValueError(f"drafts must be int32 [{self.depth}]")
        if uniforms.dtype != torch.float32 or uniforms.numel() != self.depth + 1:
            raise ValueError(f"uniforms must be fp32 [{self.depth + 1}]")
        if not temperature > 0:
            raise ValueError("temperature must be > 0")
        _lib.check(_lib.lib().ssmoe_accept_pq(target.data_ptr(), draft.data_ptr(), drafts.data_ptr(),
                                              uniforms.data_ptr(), self.depth, self.vocab, float(temperature),
                                              self.work.data_ptr(), self.work.numel(), self.out.data_ptr(),
                                              _lib.stream_of(target)))
        return self.out

    def draw_drafts_async(self, draft, uniforms, temperature: float, out=None) -> torch.Tensor:
        """x_i ~ softmax(draft[i] / temperature) for the D draft rows with uniforms[i] (fp32 [D] on the device) ->
        int32 [D] on the device: the proposal of the p/q round (ssmoe_sample_rows: the p/q round's softmax in one
        launch; the draw is exact in distribution, its bits are or_draw_rows', not the reference sampler's)."""
        d, v = self.depth, self.vocab
        if draft.dtype != torch.float32 or tuple(draft.shape) != (d, v) or not draft.is_contiguous():
            raise ValueError(f"draft must be contiguous fp32 [{d}, {v}]")
        if uniforms.dtype != torch.float32 or uniforms.numel() < d or not uniforms.is_contiguous():
            raise ValueError(f"uniforms must be contiguous fp32 [{d}]")
        if not temperature > 0:
            raise ValueError("temperature must be > 0")
        out = torch.empty(d, dtype=torch.int32, device=draft.device) if out is None else out
        if out.dtype != torch.int32 or out.numel() != d or not out.is_contiguous():
            raise ValueError(f"out must be contiguous int32 [{d}]")
        if d == 0:
            return out
        if self._dwork is None:
            nb = int(_lib.lib().ssmoe_sample_rows_workspace_bytes(d, v))
            self._dwork = torch.zeros(nb, dtype=torch.uint8, device=draft.device)  # zero before the first call
        _lib.check(_lib.lib().ssmoe_sample_rows(draft.data_ptr(), d, v, float(temperature), uniforms.data_ptr(),
                                                self._dwork.data_ptr(), self._dwork.numel(), out.data_ptr(),
                                                _lib.stream_of(draft)))
        return out

    def pq_round(self, target, draft, stream: UniformStream, temperature: float):
        """One speculative-sampling round (Leviathan et al. 2023, Alg. 1) as a drafter and verifier run it: the D
        drafts are drawn from q_i = softmax(draft_i / temperature) with the stream's next D uniforms (the draft
        phase), then the p/q round consumes its uniforms from the stream -> (drafts int32 [D] on the device,
        AcceptResult)."""
        d = self.depth
        ud = torch.from_numpy(stream.peek(d)).to(target.device)
        stream.advance(d)
        drafts = self.draw_drafts_async(draft, ud, temperature)
        return drafts, self.pq(target, draft, drafts, stream, temperature)

    def sampled_async(self, target, drafts, params, seen=(), uniforms=None) -> torch.Tensor:
        """Launch the sampled round; returns the device output int32 [D+5]. `params` is a SampleParams (sanitized
        here), `seen` the tokens generated before the round, `uniforms` fp32 [D+1] on the device."""
        self._check(target)
        if drafts.dtype != torch.int32 or drafts.numel() != self.depth:
            raise ValueError(f"drafts must be int32 [{self.depth}]")
        if uniforms is None or uniforms.dtype != torch.float32 or uniforms.numel() != self.depth + 1:
            raise ValueError(f"uniforms must be fp32 [{self.depth + 1}]")
        p = params.sanitized()
        if self._swork is None:
            nb = int(_lib.lib().ssmoe_accept_sampled_workspace_bytes(self.depth, self.vocab))
            self._swork = torch.empty(nb, dtype=torch.uint8, device=target.device)
        s = sorted(set(int(t) for t in seen)) if p.presence_penalty != 0 else []
        st = torch.tensor(s, dtype=torch.int32, device=target.device) if s else None
        _lib.check(_lib.lib().ssmoe_accept_sampled(
            target.data_ptr(), drafts.data_ptr(), self.depth, self.vocab, _lib.ptr(st), len(s), float(p.temperature),
            float(p.top_p), int(p.top_k), float(p.min_p), float(p.presence_penalty), uniforms.data_ptr(),
            self._swork.data_ptr(), self._swork.numel(), self.out.data_ptr(), _lib.stream_of(target)))
        return self.out

    def sampled(self, target, drafts, params, seen, stream: UniformStream) -> AcceptResult:
        """One sampled round with the sampler's stream: consumes one uniform per draw at temperature > 0, as
        Sampler.next does, and adds the emitted tokens to `seen` when it is a set (generate.py:214)."""
        u = torch.from_numpy(stream.peek(self.depth + 1)).to(target.device)
        res = AcceptResult.from_out(self.sampled_async(target, drafts, params, seen, u).cpu())
        stream.advance(res.n_uniform)
        if isinstance(seen, set):
            seen.update(res.tokens)
        return res

    def greedy(self, target, drafts) -> AcceptResult:
        return AcceptResult.from_out(self.greedy_async(target, drafts).cpu())

    def pq(self, target, draft, drafts, stream: UniformStream, temperature: float) -> AcceptResult:
        u = torch.from_numpy(stream.peek(self.depth + 1)).to(target.device)
        res = AcceptResult.from_out(self.pq_async(target, draft, drafts, u, temperature).cpu())
        stream.advance(res.n_uniform)
        return res


@dataclass
class RoundStats:
    """The statistics _mtp_decode returns (engine/generate.py:164-165, 221-230)."""
    rounds: int = 0
    drafted: int = 0
    accepted: int = 0
    attempts_by_depth: list = field(default_factory=list)
    accepted_by_depth: list = field(default_factory=list)
    emitted_by_round: list = field(default_factory=list)

    def add(self, depth: int, res: AcceptResult) -> None:
        if len(self.attempts_by_depth) < depth:
            self.attempts_by_depth += [0] * (depth - len(self.attempts_by_depth))
            self.accepted_by_depth += [0] * (depth - len(self.accepted_by_depth))
        self.rounds += 1
        self.drafted += depth
        self.accepted += res.n_accept
        attempted = min(depth, res.n_accept + 1) if res.n_emit > res.n_accept else res.n_accept
        for i in range(attempted):
            self.attempts_by_depth[i] += 1
        for i in range(res.n_accept):
            self.accepted_by_depth[i] += 1
        self.emitted_by_round.append(res.n_emit)

    @property
    def acceptance_length(self) -> float:
        return sum(self.emitted_by_round) / max(1, self.rounds)
