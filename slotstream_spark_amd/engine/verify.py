"""One routed-MoE layer of the MTP verify step, fused on the device.

Mirrors the MoE segment of the reference verify graph, GraphSet._moe + Segments.seg_router
(slotstream_spark/runtime/graphs.py:160-178, model/layers.py:336-348): router logits, softmax, stable top-k and
renormalisation, the routed experts (moe_decode), the shared expert gated by sigmoid(shared_expert_gate x), and
y = routed.to(bf16) + shared, with the reference's bf16 rounding of every shared-expert projection. The whole layer
is one persistent launch per block of up to 4 tokens on the caller's stream (csrc/ss_verify.hip) with no host
sync, so a step over many layers can be captured in one HIP graph.
"""
from __future__ import annotations

import torch

from .. import _lib
from ..memory.slot_pool import SlotPool


class MoEVerifyLayer:
    def __init__(self, pool: SlotPool, layer: int, router_w, sh_gate, sh_up, sh_down, sh_g, top_k: int = 10,
                 router_bias: torch.Tensor | None = None, max_tokens: int = 4):
        self.pool, self.layer, self.top_k = pool, layer, top_k
        self.router_w, self.sh_gate, self.sh_up, self.sh_down, self.sh_g = router_w, sh_gate, sh_up, sh_down, sh_g
        self.router_bias = router_bias
        self.hidden, self.inter = pool.hidden, pool.inter
        self.experts = router_w.shape[0]
        self.shared_inter = sh_gate.shape[0]
        if router_w.shape != (self.experts, self.hidden) or sh_down.shape != (self.hidden, self.shared_inter):
            raise ValueError("router_w must be [E, H] and sh_down [H, Is]")
        if sh_up.shape != sh_gate.shape or tuple(sh_g.shape) != (1, self.hidden):
            raise ValueError("sh_up must match sh_gate [Is, H] and sh_g must be [1, H]")
        for t in (router_w, sh_gate, sh_up, sh_down, sh_g):
            if t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError("router and shared-expert weights must be contiguous bf16")
        if self.experts != pool.experts:
            raise ValueError(f"router has {self.experts} experts, the pool {pool.experts}")
        self.max_tokens = max_tokens
        nb = _lib.lib().ssmoe_verify_workspace_bytes(max_tokens, self.hidden, self.inter, self.shared_inter, top_k,
                                                      self.experts)
        self.workspace = torch.zeros(int(nb), dtype=torch.uint8, device=pool.device)  # counters start at zero

    def __call__(self, x: torch.Tensor, y: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                 weights: torch.Tensor | None = None, routed: torch.Tensor | None = None):
        """x bf16 [T, H] -> (y bf16 [T, H], ids int32 [T, K], weights fp32 [T, K]); `routed` (fp32 [T, H]) receives
        the routed sum before the shared expert when given."""
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.hidden or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous bf16 [T, {self.hidden}] tensor")
        t = x.shape[0]
        if t > self.max_tokens:
            raise ValueError(f"at most {self.max_tokens} tokens per call, got {t}")
        dev = x.device
        y = torch.empty((t, self.hidden), dtype=torch.bfloat16, device=dev) if y is None else y
        ids = torch.empty((t, self.top_k), dtype=torch.int32, device=dev) if ids is None else ids
        weights = torch.empty((t, self.top_k), dtype=torch.float32, device=dev) if weights is None else weights
        if routed is not None and (tuple(routed.shape) != (t, self.hidden) or routed.dtype != torch.float32):
            raise ValueError(f"routed must be fp32 [{t}, {self.hidden}]")
        L = _lib.lib()
        _lib.check(L.ssmoe_moe_verify_layer(
            x.data_ptr(), self.router_w.data_ptr(), _lib.ptr(self.router_bias), self.sh_gate.data_ptr(),
            self.sh_up.data_ptr(), self.sh_down.data_ptr(), self.sh_g.data_ptr(), self.layer,
            self.pool.map.data_ptr(), self.pool.map.numel(), self.pool.slot_ptr.data_ptr(), self.pool.slot_ptr.numel(),
            self.workspace.data_ptr(), self.workspace.numel(), ids.data_ptr(), weights.data_ptr(), y.data_ptr(),
            _lib.ptr(routed), t, self.hidden, self.inter, self.shared_inter, self.top_k, self.experts,
            _lib.stream_of(x)))
        return y, ids, weights

    def chain(self, stream: torch.Tensor, y: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
              stream_out: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
              routed: torch.Tensor | None = None):
        """The layer on bf16(rmsnorm(stream) * norm_weight), writing y and, when given, stream_out = bf16(stream + y):
        one launch per layer of a chain (ssmoe_moe_verify_layer_chain), the same values as residual_rmsnorm followed
        by __call__."""
        t = stream.shape[0]
        for name, b in (("stream", stream), ("y", y), ("stream_out", stream_out)):
            if b is not None and (b.dtype != torch.bfloat16 or tuple(b.shape) != (t, self.hidden)
                                  or not b.is_contiguous() or not b.is_cuda):
                raise ValueError(f"{name} must be a contiguous bf16 [T, {self.hidden}] GPU tensor")
        if t > self.max_tokens:
            raise ValueError(f"at most {self.max_tokens} tokens per call, got {t}")
        if tuple(ids.shape) != (t, self.top_k) or ids.dtype != torch.int32 or not ids.is_contiguous():
            raise ValueError(f"ids must be contiguous int32 [{t}, {self.top_k}]")
        if tuple(weights.shape) != (t, self.top_k) or weights.dtype != torch.float32 or not weights.is_contiguous():
            raise ValueError(f"weights must be contiguous fp32 [{t}, {self.top_k}]")
        if norm_weight is not None and (norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != self.hidden):
            raise ValueError(f"norm_weight must be bf16 [{self.hidden}]")
        if routed is not None and (tuple(routed.shape) != (t, self.hidden) or routed.dtype != torch.float32):
            raise ValueError(f"routed must be fp32 [{t}, {self.hidden}]")
        _lib.check(_lib.lib().ssmoe_moe_verify_layer_chain(
            stream.data_ptr(), _lib.ptr(norm_weight), float(eps), self.router_w.data_ptr(), _lib.ptr(self.router_bias),
            self.sh_gate.data_ptr(), self.sh_up.data_ptr(), self.sh_down.data_ptr(), self.sh_g.data_ptr(), self.layer,
            self.pool.map.data_ptr(), self.pool.map.numel(), self.pool.slot_ptr.data_ptr(), self.pool.slot_ptr.numel(),
            self.workspace.data_ptr(), self.workspace.numel(), ids.data_ptr(), weights.data_ptr(), y.data_ptr(),
            _lib.ptr(stream_out), _lib.ptr(routed), t, self.hidden, self.inter, self.shared_inter, self.top_k,
            self.experts, _lib.stream_of(stream)))
        return y, ids, weights
