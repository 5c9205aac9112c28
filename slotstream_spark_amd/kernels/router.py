"""Router of one MoE layer and the bf16 dense projection, on gfx950.

route() is the routing half of Segments.seg_router (slotstream_spark/model/layers.py:336-348) and of
reference_torch.moe_ref (:121-124): logits = bf16(x Wg^T), softmax in fp32, stable top-k (ties to the lower index),
renormalised weights. An optional fp32 routing bias (not in the reference; BASELINE uses it to skew expert
popularity) is added to the bf16 logits before the softmax.

The logits are an fp32 dot in a fixed order (lane l of a 64-lane wave accumulates elements 512j + 8l .. +7 with
fused multiply-adds, then an xor-butterfly sum) rounded once to bf16; the softmax uses the library's own exp
(Cody-Waite + degree-7 polynomial) and fixed reduction trees. The CPU restatement replays exactly these
operations, so router ids and weights are bit-identical to it.
"""
from __future__ import annotations

import torch

from .. import _lib


def lin_bf16(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x bf16 [T, H] @ w bf16 [N, H]^T -> bf16 [T, N] (lin() for bf16 weights, model/layers.py:62-76)."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("x and w must be bf16 2-D tensors")
    if x.shape[1] != w.shape[1] or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("x [T, H] and w [N, H] must be contiguous with the same H")
    t, n = x.shape[0], w.shape[0]
    if out is None:
        out = torch.empty((t, n), dtype=torch.bfloat16, device=x.device)
    if tuple(out.shape) != (t, n) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError(f"out must be contiguous bf16 [{t}, {n}]")
    _lib.check(_lib.lib().ssmoe_dense_gemv_bf16(x.data_ptr(), w.data_ptr(), out.data_ptr(), t, x.shape[1], n,
                                                _lib.stream_of(x)))
    return out


def gemm_bf16(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x bf16 [M, K] @ w bf16 [N, K]^T -> bf16 [M, N] on the MFMA GEMM (ssmoe_dense_gemm): lin over a prompt chunk
    (model/layers.py:62-76 inside prefill_gemm()). K a multiple of 256, N a multiple of 8."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("x and w must be bf16 2-D tensors")
    if x.shape[1] != w.shape[1] or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("x [M, K] and w [N, K] must be contiguous with the same K")
    m, n = x.shape[0], w.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    if tuple(out.shape) != (m, n) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError(f"out must be contiguous bf16 [{m}, {n}]")
    _lib.check(_lib.lib().ssmoe_dense_gemm(x.data_ptr(), x.shape[1], w.data_ptr(), w.shape[1], out.data_ptr(), n, m, n,
                                           x.shape[1], _lib.stream_of(x)))
    return out


def route(x: torch.Tensor, router_w: torch.Tensor, k: int, bias: torch.Tensor | None = None, *,
          logits: torch.Tensor | None = None, probs: torch.Tensor | None = None,
          ids: torch.Tensor | None = None, weights: torch.Tensor | None = None):
    """x bf16 [T, H] · router_w bf16 [E, H] -> (ids int32 [T, k], weights fp32 [T, k]).
    `logits` (bf16 [T, E]) and `probs` (fp32 [T, E]) receive the intermediates when given."""
    if x.dtype != torch.bfloat16 or router_w.dtype != torch.bfloat16 or x.dim() != 2 or router_w.dim() != 2:
        raise ValueError("x and router_w must be bf16 2-D tensors")
    if x.shape[1] != router_w.shape[1] or not x.is_contiguous() or not router_w.is_contiguous():
        raise ValueError("x [T, H] and router_w [E, H] must be contiguous with the same H")
    t, e = x.shape[0], router_w.shape[0]
    dev = x.device
    if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (e,) or not bias.is_contiguous()):
        raise ValueError(f"bias must be contiguous fp32 [{e}]")
    if logits is None:
        logits = torch.empty((t, e), dtype=torch.bfloat16, device=dev)
    if ids is None:
        ids = torch.empty((t, k), dtype=torch.int32, device=dev)
    if weights is None:
        weights = torch.empty((t, k), dtype=torch.float32, device=dev)
    for buf, shape, dt in ((logits, (t, e), torch.bfloat16), (ids, (t, k), torch.int32),
                           (weights, (t, k), torch.float32)):
        if tuple(buf.shape) != shape or buf.dtype != dt or not buf.is_contiguous():
            raise ValueError(f"buffer must be contiguous {dt} {shape}")
    if probs is not None and (tuple(probs.shape) != (t, e) or probs.dtype != torch.float32):
        raise ValueError(f"probs must be contiguous fp32 [{t}, {e}]")
    _lib.check(_lib.lib().ssmoe_router(x.data_ptr(), router_w.data_ptr(), _lib.ptr(bias), logits.data_ptr(),
                                       _lib.ptr(probs), ids.data_ptr(), weights.data_ptr(), t, x.shape[1], e, int(k),
                                       _lib.stream_of(x)))
    return ids, weights
