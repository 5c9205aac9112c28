"""Dense GEMV over MLX affine 4-bit weights on the device (drop-in for slotstream_spark/kernels/gemv_affine.py).

`AffineWeight` keeps the reference's fields and validation (gemv_affine.py:29-47); `gemv(x, w, out, ws, cfg)` keeps
its signature and errors (:214-262) and runs `ssmoe_gemv_affine4` for bits=4, gs=64 (the model's format, e.g. the
lm_head 248,320 x 2560): fp32 accumulation of exact bf16 products, one fixed order per output element, and row r of
the result depends on x row r alone, so an R-row call equals R one-row calls bit for bit (kernels/tuning.py:1-10).
`LMHeadGreedy` fuses the lm_head with the greedy round after it (engine/generate.py:208-229), `LMHeadPQ` with the
p/q round (the GEMV forms the logits' chunk maxima, so the round reads the logits once), and `LMHeadArgmax` gives the
draft head's token (engine/mtp.py:275).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib
from ..engine.accept import AcceptResult

SUPPORTED_K = (1024, 2048, 2560, 4096)


@dataclass
class AffineWeight:
    q: torch.Tensor   # int32 [n, k*bits/32]
    s: torch.Tensor   # bf16 [n, k/gs]
    b: torch.Tensor   # bf16 [n, k/gs]
    bits: int
    gs: int
    n: int
    k: int

    def __post_init__(self):
        if self.bits not in (4, 8) or self.gs not in (32, 64):
            raise ValueError(f"unsupported bits={self.bits} gs={self.gs}")
        if self.k % self.gs:
            raise ValueError(f"k={self.k} not a multiple of gs={self.gs}")
        if tuple(self.q.shape) != (self.n, self.k * self.bits // 32) or self.q.dtype != torch.int32:
            raise ValueError(f"q must be int32 {(self.n, self.k * self.bits // 32)}, got {tuple(self.q.shape)} "
                             f"{self.q.dtype}")
        for t in (self.s, self.b):
            if tuple(t.shape) != (self.n, self.k // self.gs) or t.dtype != torch.bfloat16:
                raise ValueError("scales and biases must be bf16 [n, k/gs]")


def _device_weight(w: AffineWeight) -> None:
    if w.bits != 4 or w.gs != 64:
        raise NotImplementedError(f"this build runs affine GEMVs with bits=4, gs=64 (got bits={w.bits}, gs={w.gs})")
    if w.k not in SUPPORTED_K:
        raise NotImplementedError(f"K={w.k}: this build's GEMV kernels take K in {SUPPORTED_K}")
    for t in (w.q, w.s, w.b):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("weights must be contiguous GPU tensors")


def _check_x(x: torch.Tensor, w: AffineWeight) -> None:
    if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float32) or not x.is_contiguous():
        raise ValueError("x must be a contiguous 2-D bf16 or fp32 tensor")
    if x.shape[1] != w.k:
        raise ValueError(f"x has K={x.shape[1]}, weight has K={w.k}")
    if not x.is_cuda:
        raise ValueError("x must be a GPU tensor")


def gemv(x: torch.Tensor, w, out: torch.Tensor | None = None, ws: torch.Tensor | None = None,
         cfg: dict | None = None) -> torch.Tensor:
    """x [R, K] bf16|fp32 -> [R, N] fp32. `ws` and `cfg` are accepted for the reference's signature; the kernel
    needs no workspace and its tiling is fixed by the shape."""
    if not isinstance(w, AffineWeight):
        raise TypeError("w must be AffineWeight (bf16 dense projections: kernels.router.lin_bf16)")
    _check_x(x, w)
    _device_weight(w)
    r = x.shape[0]
    if out is None:
        out = torch.empty((r, w.n), dtype=torch.float32, device=x.device)
    elif tuple(out.shape) != (r, w.n) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"out must be contiguous fp32 {(r, w.n)}")
    _lib.check(_lib.lib().ssmoe_gemv_affine4(x.data_ptr(), 1 if x.dtype == torch.float32 else 0, r, w.k,
                                             w.q.data_ptr(), w.s.data_ptr(), w.b.data_ptr(), w.n, out.data_ptr(),
                                             _lib.stream_of(x)))
    return out


class LMHeadGreedy:
    """The lm_head over the D+1 verify rows fused with the greedy round: per 16-row vocabulary tile one argmax key
    per row, then the round (out int32 [D+5] as Acceptor.greedy). Workspace owned here."""

    def __init__(self, w: AffineWeight, depth: int, device="cuda"):
        _device_weight(w)
        self.w, self.depth = w, depth
        nb = int(_lib.lib().ssmoe_lm_head_greedy_workspace_bytes(depth, w.n))
        if nb < 0:
            raise ValueError(f"depth must be in [0, 60], got {depth}")
        self.work = torch.zeros(nb, dtype=torch.uint8, device=device)  # zero before the first call (calls leave it so)
        self.out = torch.empty(depth + 5, dtype=torch.int32, device=device)

    def run_async(self, x: torch.Tensor, drafts: torch.Tensor, logits: torch.Tensor | None = None) -> torch.Tensor:
        _check_x(x, self.w)
        if x.shape[0] != self.depth + 1:
            raise ValueError(f"x must hold {self.depth + 1} rows")
        if drafts.dtype != torch.int32 or drafts.numel() != self.depth:
            raise ValueError(f"drafts must be int32 [{self.depth}]")
        if logits is not None and (tuple(logits.shape) != (self.depth + 1, self.w.n) or logits.dtype != torch.float32
                                   or not logits.is_contiguous()):
            raise ValueError(f"logits must be contiguous fp32 {(self.depth + 1, self.w.n)}")
        _lib.check(_lib.lib().ssmoe_lm_head_greedy(
            x.data_ptr(), 1 if x.dtype == torch.float32 else 0, self.depth, self.w.k, self.w.q.data_ptr(),
            self.w.s.data_ptr(), self.w.b.data_ptr(), self.w.n, drafts.data_ptr(), self.work.data_ptr(),
            self.work.numel(), _lib.ptr(logits), self.out.data_ptr(), _lib.stream_of(x)))
        return self.out

    def __call__(self, x, drafts, logits=None) -> AcceptResult:
        return AcceptResult.from_out(self.run_async(x, drafts, logits).cpu())


class LMHeadArgmax:
    """torch.argmax of the lm_head logits per row, the draft token of MTPHead.draft (engine/mtp.py:275): with
    `round_bf16` the argmax ranks the logits rounded to bf16, as lin returns them for a bf16 x; ties to the first
    index, NaN as the maximum. The ids stay on the device. Workspace owned here, for up to `max_rows` rows."""

    def __init__(self, w: AffineWeight, max_rows: int = 1, round_bf16: bool = True, device="cuda"):
        _device_weight(w)
        self.w, self.max_rows, self.round_bf16 = w, max_rows, round_bf16
        nb = int(_lib.lib().ssmoe_lm_head_argmax_workspace_bytes(max_rows, w.n))
        if nb < 0:
            raise ValueError(f"max_rows must be in [1, 64], got {max_rows}")
        self.work = torch.zeros(nb, dtype=torch.uint8, device=device)  # zero before the first call (calls leave it so)

    def __call__(self, x: torch.Tensor, ids: torch.Tensor | None = None,
                 logits: torch.Tensor | None = None) -> torch.Tensor:
        _check_x(x, self.w)
        r = x.shape[0]
        if not 1 <= r <= self.max_rows:
            raise ValueError(f"x must hold 1..{self.max_rows} rows, got {r}")
        ids = torch.empty(r, dtype=torch.int32, device=x.device) if ids is None else ids
        if ids.dtype != torch.int32 or ids.numel() != r or not ids.is_contiguous():
            raise ValueError(f"ids must be contiguous int32 [{r}]")
        if logits is not None and (tuple(logits.shape) != (r, self.w.n) or logits.dtype != torch.float32
                                   or not logits.is_contiguous()):
            raise ValueError(f"logits must be contiguous fp32 {(r, self.w.n)}")
        _lib.check(_lib.lib().ssmoe_lm_head_argmax(
            x.data_ptr(), 1 if x.dtype == torch.float32 else 0, r, self.w.k, self.w.q.data_ptr(), self.w.s.data_ptr(),
            self.w.b.data_ptr(), self.w.n, 1 if self.round_bf16 else 0, self.work.data_ptr(), self.work.numel(),
            _lib.ptr(logits), ids.data_ptr(), _lib.stream_of(x)))
        return ids


class LMHeadPQ:
    """The lm_head over the D+1 verify rows with the p/q round behind it (ssmoe_lm_head_pq): the GEMV writes the
    logits (lin's values) and their chunk maxima, and the round reads the logits once, for the sums; the same result
    as Acceptor.pq on those logits, bit for bit. Workspace, logits [D+1, V] and out [D+5] owned here."""

    def __init__(self, w: AffineWeight, depth: int, temperature: float, device="cuda"):
        _device_weight(w)
        if not temperature > 0:
            raise ValueError("temperature must be > 0")
        self.w, self.depth, self.temperature = w, depth, float(temperature)
        nb = int(_lib.lib().ssmoe_lm_head_pq_workspace_bytes(depth, w.n))
        if nb < 0:
            raise ValueError(f"depth must be in [0, 3], got {depth}")
        self.work = torch.zeros(nb, dtype=torch.uint8, device=device)  # the round's counters start at zero
        self.logits = torch.empty((depth + 1, w.n), dtype=torch.float32, device=device)
        self.out = torch.empty(depth + 5, dtype=torch.int32, device=device)

    def run_async(self, x: torch.Tensor, draft: torch.Tensor, drafts: torch.Tensor,
                  uniforms: torch.Tensor) -> torch.Tensor:
        _check_x(x, self.w)
        D, V = self.depth, self.w.n
        if x.shape[0] != D + 1:
            raise ValueError(f"x must hold {D + 1} rows")
        if draft.dtype != torch.float32 or tuple(draft.shape) != (D, V) or not draft.is_contiguous():
            raise ValueError(f"draft must be contiguous fp32 {(D, V)}")
        if drafts.dtype != torch.int32 or drafts.numel() != D:
            raise ValueError(f"drafts must be int32 [{D}]")
        if uniforms.dtype != torch.float32 or uniforms.numel() != D + 1:
            raise ValueError(f"uniforms must be fp32 [{D + 1}]")
        _lib.check(_lib.lib().ssmoe_lm_head_pq(
            x.data_ptr(), 1 if x.dtype == torch.float32 else 0, D, self.w.k, self.w.q.data_ptr(), self.w.s.data_ptr(),
            self.w.b.data_ptr(), V, draft.data_ptr(), drafts.data_ptr(), uniforms.data_ptr(), self.temperature,
            self.work.data_ptr(), self.work.numel(), self.logits.data_ptr(), self.out.data_ptr(), _lib.stream_of(x)))
        return self.out

    def __call__(self, x, draft, drafts, stream) -> AcceptResult:
        """With the uniforms of a UniformStream (peeked, then advanced by the number the round used)."""
        u = torch.from_numpy(stream.peek(self.depth + 1)).to(x.device)
        res = AcceptResult.from_out(self.run_async(x, draft, drafts, u).cpu())
        stream.advance(res.n_uniform)
        return res
