"""One routed-MoE layer over a prompt chunk (prefill), every expert resident in HBM.

Mirrors SweepMoE.layer (slotstream_spark/model/moe_sweep.py:80-160) plus the router and shared expert around it
(model/layers.py:336-348, 398-402): router logits lin(x, W_gate) as a bf16 GEMM, softmax / stable top-k /
renormalisation on the device (ssmoe_router_topk), the routed experts as one plan over all E experts
(ssmoe_moe_prefill: moe_align, grouped gate/up, down, rank-order combine), and y = bf16(routed) + shared.
The dense projections run on libssmoe's bf16 MFMA GEMM (ssmoe_dense_gemm, lin's fp32 dot rounded once to bf16):
the router, one GEMM for the shared expert's gate, up and shared_expert_gate rows together (their weights
concatenated once at construction), and the shared down projection. The routed experts, the routing, the shared
expert's elementwise chain (ssmoe_shared_hs) and the final y (ssmoe_combine_shared) run in libssmoe as well, with the
reference's bf16 rounding of every op; torch only allocates.
"""
from __future__ import annotations

import torch

from .. import _lib
from ..kernels.router import gemm_bf16
from ..memory.slot_pool import SlotPool


class MoEPrefillLayer:
    def __init__(self, pool: SlotPool, layer: int, router_w, sh_gate, sh_up, sh_down, sh_g, top_k: int = 10,
                 router_bias: torch.Tensor | None = None, max_tokens: int = 2048):
        self.pool, self.layer, self.top_k = pool, layer, top_k
        self.router_w, self.sh_gate, self.sh_up, self.sh_down, self.sh_g = router_w, sh_gate, sh_up, sh_down, sh_g
        self.router_bias = router_bias
        self.hidden, self.inter = pool.hidden, pool.inter
        self.experts = router_w.shape[0]
        if self.experts != pool.experts:
            raise ValueError(f"router has {self.experts} experts, the pool {pool.experts}")
        for t in (router_w, sh_gate, sh_up, sh_down, sh_g):
            if t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError("router and shared-expert weights must be contiguous bf16")
        self.max_tokens = max_tokens
        self.shared_inter = sh_gate.shape[0]
        # shared gate, up and shared_expert_gate rows in one weight [2 Is + 1 (padded to 8), H]
        n_sh = 2 * self.shared_inter + 1
        pad = (-n_sh) % 8
        self.sh_cat = torch.cat([sh_gate, sh_up, sh_g] + ([sh_g.new_zeros((pad, self.hidden))] if pad else [])).contiguous()
        dev, R = pool.device, max_tokens * top_k
        L = _lib.lib()
        nb = L.ssmoe_moe_prefill_workspace_bytes(max_tokens, top_k, self.experts)
        self.workspace = torch.empty(int(nb), dtype=torch.uint8, device=dev)
        self.h_buf = torch.empty((R, self.inter), dtype=torch.bfloat16, device=dev)
        self.out_rows = torch.empty((R, self.hidden), dtype=torch.float32, device=dev)
        self.ids = torch.empty((max_tokens, top_k), dtype=torch.int32, device=dev)
        self.weights = torch.empty((max_tokens, top_k), dtype=torch.float32, device=dev)
        self.routed = torch.empty((max_tokens, self.hidden), dtype=torch.float32, device=dev)

    def route(self, x: torch.Tensor):
        t = x.shape[0]
        logits = gemm_bf16(x, self.router_w)
        ids, w = self.ids[:t], self.weights[:t]
        _lib.check(_lib.lib().ssmoe_router_topk(logits.data_ptr(), _lib.ptr(self.router_bias), None, ids.data_ptr(),
                                                w.data_ptr(), t, self.experts, self.top_k, _lib.stream_of(x)))
        return ids, w

    def routed_experts(self, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        t = x.shape[0]
        out = self.routed[:t]
        _lib.check(_lib.lib().ssmoe_moe_prefill(
            x.data_ptr(), ids.data_ptr(), w.data_ptr(), self.layer, self.pool.map.data_ptr(), self.pool.map.numel(),
            self.pool.slot_ptr.data_ptr(), self.pool.slot_ptr.numel(), self.workspace.data_ptr(),
            self.workspace.numel(), self.h_buf.data_ptr(), self.out_rows.data_ptr(), out.data_ptr(), t, self.hidden,
            self.inter, self.top_k, self.experts, _lib.stream_of(x)))
        return out

    def shared(self, x: torch.Tensor):
        """(sh bf16 [T, H] = lin(bf16(silu(g)) * u, sh_down), shared_expert_gate logits bf16 [T])."""
        t = x.shape[0]
        proj = gemm_bf16(x, self.sh_cat)
        hs = torch.empty((t, self.shared_inter), dtype=torch.bfloat16, device=x.device)
        sgl = torch.empty((t,), dtype=torch.bfloat16, device=x.device)
        _lib.check(_lib.lib().ssmoe_shared_hs(proj.data_ptr(), proj.shape[1], t, self.shared_inter, hs.data_ptr(),
                                              sgl.data_ptr(), _lib.stream_of(x)))
        return gemm_bf16(hs, self.sh_down), sgl

    def __call__(self, x: torch.Tensor):
        """x bf16 [T, H] -> (y bf16 [T, H], ids int32 [T, K], weights fp32 [T, K], routed fp32 [T, H]);
        y = routed.to(bf16) + sigmoid(x w_sg) * shared(x), each op rounded to bf16 as in the reference."""
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.hidden or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous bf16 [T, {self.hidden}] tensor")
        if x.shape[0] > self.max_tokens:
            raise ValueError(f"at most {self.max_tokens} tokens per call, got {x.shape[0]}")
        t = x.shape[0]
        ids, w = self.route(x)
        routed = self.routed_experts(x, ids, w)
        sh, sgl = self.shared(x)
        y = torch.empty((t, self.hidden), dtype=torch.bfloat16, device=x.device)
        _lib.check(_lib.lib().ssmoe_combine_shared(routed.data_ptr(), sh.data_ptr(), sgl.data_ptr(), y.data_ptr(), t,
                                                   self.hidden, _lib.stream_of(x)))
        return y, ids, w, routed
