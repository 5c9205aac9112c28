"""The reference token sampler on the device (drop-in for slotstream_spark/engine/sampler.py).

`SampleParams` and `Sampler` keep the reference's names, fields, defaults and clamping (sampler.py:35-108); the draw
runs in libssmoe (`ssmoe_sample`) on a device row of fp32 logits. The generator is the reference's splitmix64 stream
on the host (`UniformStream`): a draw at temperature > 0 consumes exactly one uniform, a greedy draw none, as in
Sampler.next. The float32 steps are the reference's; the order of each sum and the exp are the library's, so a draw
can differ from numpy's only where the uniform falls within rounding of a CDF step.

`SampleParams` and its `sanitized()` clamps follow fortil/slotstream-spark engine/sampler.py:14-64 field for field
(the public parameter type of the drop-in). That file, itself a port of slotstream's sampler (MIT, Copyright (c)
2026 Carlos Galarza), is under the MIT License:

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

import math
from dataclasses import dataclass, field

import torch

from .. import _lib
from .accept import UniformStream

MAX_TOKEN_CEILING = 32_768


@dataclass
class SampleParams:
    temperature: float = 0.8
    top_p: float = 0.95
    top_k: int = 40
    min_p: float = 0.0
    presence_penalty: float = 0.0
    max_tokens: int = 512
    stop: list = field(default_factory=list)

    def sanitized(self) -> "SampleParams":
        """Clamp every knob into the range the sampler is defined on (sampler.py:45-64)."""
        p = SampleParams(self.temperature, self.top_p, self.top_k, self.min_p, self.presence_penalty,
                         self.max_tokens, list(self.stop))
        if not math.isfinite(p.temperature):
            p.temperature = 0.0
        p.temperature = max(0.0, p.temperature)
        if not math.isfinite(p.top_p) or p.top_p <= 0 or p.top_p > 1:
            p.top_p = 1.0
        if not math.isfinite(p.min_p):
            p.min_p = 0.0
        p.min_p = min(max(0.0, p.min_p), 1.0)
        if not math.isfinite(p.presence_penalty):
            p.presence_penalty = 0.0
        p.top_k = max(0, int(p.top_k))
        if p.max_tokens <= 0:
            p.max_tokens = MAX_TOKEN_CEILING
        p.max_tokens = min(p.max_tokens, MAX_TOKEN_CEILING)
        p.stop = [s for s in p.stop if s]
        return p


class Sampler:
    """Sampler(seed).next(logits, params, generated) -> token, with logits a device fp32 [V] tensor."""

    def __init__(self, seed: int = 0):
        self.stream = UniformStream(seed)
        self._work = None
        self._out = None
        self._u = None

    @property
    def state(self) -> int:
        return self.stream.state

    def _buffers(self, logits: torch.Tensor):
        v = logits.numel()
        nb = int(_lib.lib().ssmoe_sample_workspace_bytes(v))
        if nb < 0:
            raise ValueError(f"vocabulary of {v} tokens is outside [1, 1048576]")
        if self._work is None or self._work.numel() < nb or self._work.device != logits.device:
            self._work = torch.empty(nb, dtype=torch.uint8, device=logits.device)
            self._out = torch.empty(2, dtype=torch.int32, device=logits.device)
            self._u = torch.empty(1, dtype=torch.float32, device=logits.device)

    def next_async(self, logits: torch.Tensor, p: SampleParams, generated=()) -> torch.Tensor:
        """Launch one draw; returns the device int32 [2] (token, flags). Advances the stream as Sampler.next."""
        if logits.dtype != torch.float32 or logits.dim() != 1 or not logits.is_contiguous() or not logits.is_cuda:
            raise ValueError("logits must be a contiguous fp32 [V] GPU tensor")
        p = p.sanitized()
        self._buffers(logits)
        gen = sorted(set(int(t) for t in generated)) if p.presence_penalty != 0 else []
        g = torch.tensor(gen, dtype=torch.int32, device=logits.device) if gen else None
        if p.temperature > 0:
            self._u.fill_(float(self.stream.peek(1)[0]))
            self.stream.advance(1)
        else:
            self._u.zero_()
        _lib.check(_lib.lib().ssmoe_sample(
            logits.data_ptr(), logits.numel(), _lib.ptr(g), len(gen), float(p.temperature), float(p.top_p),
            int(p.top_k), float(p.min_p), float(p.presence_penalty), self._u.data_ptr(), self._work.data_ptr(),
            self._work.numel(), self._out.data_ptr(), _lib.stream_of(logits)))
        return self._out

    def next(self, logits: torch.Tensor, p: SampleParams, generated=()) -> int:
        return int(self.next_async(logits, p, generated)[0].item())
