"""One routed-MoE layer of the MTP verify step, fused on the device.

Mirrors the MoE segment of the reference verify graph, GraphSet._moe + Segments.seg_router
(slotstream_spark/runtime/graphs.py:160-178, model/layers.py:336-348): router logits, softmax, stable top-k and
renormalisation, the routed experts (moe_decode), the shared expert gated by sigmoid(shared_expert_gate x), and
y = routed.to(bf16) + shared, with the reference's bf16 rounding of every shared-expert projection. The whole layer
is one persistent launch per block of up to 4 tokens on the caller's stream (csrc/ss_verify.hip) with no host
sync, so a step over many layers can be captured in one HIP graph.

The shared expert's gate, up and down projections are bf16 tensors or, as the reference checkpoint keeps them, affine
4-bit (gs 64) AffineWeights (model/weights.py:84-92; lin -> gemv, model/layers.py:62-76); the router and the
shared_expert_gate row are bf16 (dense in the checkpoint).
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ..kernels.gemv_affine import AffineWeight
from ..memory.slot_pool import SlotPool


class SharedQ4(ctypes.Structure):
    """ssmoe_shared_q4 (include/ssmoe.h): the scales and biases of an affine 4-bit shared expert."""
    _fields_ = [("gate_s", ctypes.c_void_p), ("gate_b", ctypes.c_void_p), ("up_s", ctypes.c_void_p),
                ("up_b", ctypes.c_void_p), ("down_s", ctypes.c_void_p), ("down_b", ctypes.c_void_p)]


def _wptr(w) -> int:
    """Device address of a shared-expert weight: the packed words of an AffineWeight, else the bf16 tensor."""
    return w.q.data_ptr() if isinstance(w, AffineWeight) else w.data_ptr()


def _shape(w):
    return (w.n, w.k) if isinstance(w, AffineWeight) else tuple(w.shape)


class MoEVerifyLayer:
    def __init__(self, pool: SlotPool, layer: int, router_w, sh_gate, sh_up, sh_down, sh_g, top_k: int = 10,
                 router_bias: torch.Tensor | None = None, max_tokens: int = 4):
        self.pool, self.layer, self.top_k = pool, layer, top_k
        self.router_w, self.sh_gate, self.sh_up, self.sh_down, self.sh_g = router_w, sh_gate, sh_up, sh_down, sh_g
        self.router_bias = router_bias
        self.hidden, self.inter = pool.hidden, pool.inter
        self.experts = router_w.shape[0]
        self.shared_inter = _shape(sh_gate)[0]
        if tuple(router_w.shape) != (self.experts, self.hidden) or _shape(sh_down) != (self.hidden, self.shared_inter):
            raise ValueError("router_w must be [E, H] and sh_down [H, Is]")
        if _shape(sh_up) != _shape(sh_gate) or tuple(sh_g.shape) != (1, self.hidden):
            raise ValueError("sh_up must match sh_gate [Is, H] and sh_g must be [1, H]")
        q4 = [isinstance(w, AffineWeight) for w in (sh_gate, sh_up, sh_down)]
        if any(q4) and not all(q4):
            raise ValueError("the shared expert's gate, up and down projections are all AffineWeight or all bf16")
        self.sh_q4 = None
        if all(q4):
            for w in (sh_gate, sh_up, sh_down):
                if w.bits != 4 or w.gs != 64:
                    raise NotImplementedError(f"affine shared expert: bits 4, gs 64 (got bits={w.bits}, gs={w.gs})")
                for t in (w.q, w.s, w.b):
                    if not t.is_contiguous() or not t.is_cuda:
                        raise ValueError("shared-expert weights must be contiguous GPU tensors")
            self.sh_q4 = SharedQ4(sh_gate.s.data_ptr(), sh_gate.b.data_ptr(), sh_up.s.data_ptr(), sh_up.b.data_ptr(),
                                  sh_down.s.data_ptr(), sh_down.b.data_ptr())
        dense = (router_w, sh_g) if self.sh_q4 is not None else (router_w, sh_gate, sh_up, sh_down, sh_g)
        for t in dense:
            if t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError("router, shared_expert_gate and bf16 shared-expert weights must be contiguous bf16")
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
        head = (x.data_ptr(), self.router_w.data_ptr(), _lib.ptr(self.router_bias), _wptr(self.sh_gate),
                _wptr(self.sh_up), _wptr(self.sh_down), self.sh_g.data_ptr())
        tail = (self.layer, self.pool.map.data_ptr(), self.pool.map.numel(), self.pool.slot_ptr.data_ptr(),
                self.pool.slot_ptr.numel(), self.workspace.data_ptr(), self.workspace.numel(), ids.data_ptr(),
                weights.data_ptr(), y.data_ptr(), _lib.ptr(routed), t, self.hidden, self.inter, self.shared_inter,
                self.top_k, self.experts, _lib.stream_of(x))
        if self.sh_q4 is None:
            _lib.check(L.ssmoe_moe_verify_layer(*head, *tail))
        else:
            _lib.check(L.ssmoe_moe_verify_layer_q4s(*head, ctypes.addressof(self.sh_q4), *tail))
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
        L = _lib.lib()
        head = (stream.data_ptr(), _lib.ptr(norm_weight), float(eps), self.router_w.data_ptr(),
                _lib.ptr(self.router_bias), _wptr(self.sh_gate), _wptr(self.sh_up), _wptr(self.sh_down),
                self.sh_g.data_ptr())
        tail = (self.layer, self.pool.map.data_ptr(), self.pool.map.numel(), self.pool.slot_ptr.data_ptr(),
                self.pool.slot_ptr.numel(), self.workspace.data_ptr(), self.workspace.numel(), ids.data_ptr(),
                weights.data_ptr(), y.data_ptr(), _lib.ptr(stream_out), _lib.ptr(routed), t, self.hidden, self.inter,
                self.shared_inter, self.top_k, self.experts, _lib.stream_of(stream))
        if self.sh_q4 is None:
            _lib.check(L.ssmoe_moe_verify_layer_chain(*head, *tail))
        else:
            _lib.check(L.ssmoe_moe_verify_layer_chain_q4s(*head, ctypes.addressof(self.sh_q4), *tail))
        return y, ids, weights


class ChainLayerEntry(ctypes.Structure):
    """ssmoe_chain_layer (include/ssmoe.h): one layer of a chain launch."""
    _fields_ = [("router_w", ctypes.c_void_p), ("router_bias", ctypes.c_void_p), ("sh_gate", ctypes.c_void_p),
                ("sh_up", ctypes.c_void_p), ("sh_down", ctypes.c_void_p), ("sh_g", ctypes.c_void_p),
                ("norm_w", ctypes.c_void_p), ("layer", ctypes.c_int64), ("ids", ctypes.c_void_p),
                ("weights", ctypes.c_void_p), ("y", ctypes.c_void_p), ("stream_out", ctypes.c_void_p),
                ("routed_out", ctypes.c_void_p), ("sh_gate_s", ctypes.c_void_p), ("sh_gate_b", ctypes.c_void_p),
                ("sh_up_s", ctypes.c_void_p), ("sh_up_b", ctypes.c_void_p), ("sh_down_s", ctypes.c_void_p),
                ("sh_down_b", ctypes.c_void_p)]


class MoEVerifyChain:
    """Chained MoE layers of a verify step in one persistent launch (ssmoe_moe_verify_chain): layer l runs on
    bf16(rmsnorm(s_l) * norm_w_l) with s_0 the input stream and s_{l+1} = bf16(s_l + y_l), the bits of one
    MoEVerifyLayer.chain call per layer. The output buffers are fixed at construction (the device table holds their
    addresses): ys[l], ids[l], weights[l] and, when given, stream_outs[l] (the stream after layer l)."""

    def __init__(self, layers: list[MoEVerifyLayer], ys, ids, weights, stream_outs=None, norm_weights=None,
                 eps: float = 1e-6):
        if not layers:
            raise ValueError("need at least one layer")
        l0 = layers[0]
        self.pool = l0.pool
        self.hidden, self.inter, self.shared_inter = l0.hidden, l0.inter, l0.shared_inter
        self.top_k, self.experts = l0.top_k, l0.experts
        for q in layers:
            if (q.pool is not self.pool or q.hidden != self.hidden or q.inter != self.inter or q.top_k != self.top_k
                    or q.experts != self.experts or q.shared_inter != self.shared_inter):
                raise ValueError("chained layers must share the pool and the layer shape")
        n = len(layers)
        norm_weights = list(norm_weights) if norm_weights is not None else [None] * n
        stream_outs = list(stream_outs) if stream_outs is not None else [None] * n
        if not (len(ys) == len(ids) == len(weights) == len(norm_weights) == len(stream_outs) == n):
            raise ValueError("need one y, ids, weights, norm weight and stream_out entry per layer")
        self.eps = float(eps)
        self.layers = layers
        self._keep = (ys, ids, weights, stream_outs, norm_weights)
        table = (ChainLayerEntry * n)()
        for i, q in enumerate(layers):
            qs = q.sh_q4
            table[i] = ChainLayerEntry(q.router_w.data_ptr(), _lib.ptr(q.router_bias), _wptr(q.sh_gate),
                                       _wptr(q.sh_up), _wptr(q.sh_down), q.sh_g.data_ptr(),
                                       _lib.ptr(norm_weights[i]), q.layer, ids[i].data_ptr(), weights[i].data_ptr(),
                                       ys[i].data_ptr(), _lib.ptr(stream_outs[i]), None,
                                       *((qs.gate_s, qs.gate_b, qs.up_s, qs.up_b, qs.down_s, qs.down_b)
                                         if qs is not None else (None,) * 6))
        self.table_host = table
        raw = bytes(table)
        self.table_dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.pool.device)
        nb = _lib.lib().ssmoe_verify_chain_workspace_bytes(4, self.hidden, self.inter, self.shared_inter, self.top_k,
                                                            self.experts)
        if nb < 0:
            raise ValueError(f"no chain kernel for H={self.hidden}, I={self.inter}")
        self.workspace = torch.zeros(int(nb), dtype=torch.uint8, device=self.pool.device)

    @staticmethod
    def supported(hidden: int, inter: int, shared_inter: int, top_k: int, experts: int, device="cuda") -> bool:
        """True when the shape has a chain kernel, every wave of the grid (one workgroup of 4 waves per CU) owns a
        router or shared-expert row (E + Is >= 4 * CUs), which the chain's hand-offs rely on, and some workgroups
        have no output rows (H / 16 < CUs): they form the shared expert's rows."""
        cus = torch.cuda.get_device_properties(torch.device(device)).multi_processor_count
        return (_lib.lib().ssmoe_verify_chain_workspace_bytes(4, hidden, inter, shared_inter, top_k, experts) > 0
                and experts + shared_inter >= 4 * cus and hidden // 16 < cus)

    def run(self, stream_in: torch.Tensor) -> None:
        """All layers on the current stream; the rows are those of stream_in ([T, H] bf16, T <= 4)."""
        if (stream_in.dtype != torch.bfloat16 or stream_in.dim() != 2 or stream_in.shape[1] != self.hidden
                or not stream_in.is_contiguous() or not stream_in.is_cuda):
            raise ValueError(f"stream_in must be a contiguous bf16 [T, {self.hidden}] GPU tensor")
        t = stream_in.shape[0]
        ys = self._keep[0]
        if t != ys[0].shape[0]:
            raise ValueError(f"the chain's buffers hold {ys[0].shape[0]} rows, stream_in has {t}")
        p = self.pool
        _lib.check(_lib.lib().ssmoe_moe_verify_chain(
            stream_in.data_ptr(), self.eps, ctypes.addressof(self.table_host), self.table_dev.data_ptr(),
            len(self.layers), p.map.data_ptr(), p.map.numel(), p.slot_ptr.data_ptr(), p.slot_ptr.numel(),
            self.workspace.data_ptr(), self.workspace.numel(), t, self.hidden, self.inter, self.shared_inter,
            self.top_k, self.experts, _lib.stream_of(stream_in)))
