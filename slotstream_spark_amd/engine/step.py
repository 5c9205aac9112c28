"""A whole MTP verify round of the MoE path as one HIP graph.

The reference verifies `rows` = 1 + depth tokens with GraphSet.step (runtime/graphs.py:92-344): 49 segment graphs per
step, and between two of them the host waits for the layer's routing ids, calls ExpertPool.ensure and replays the
next segment; the fp32 logits then go to the host, where _mtp_decode (engine/generate.py:152-238) samples the rows
and runs the acceptance. With every expert resident in HBM nothing has to be loaded between layers, so here the
round is one graph with the ids of every layer staying on the device:

    mixed_0 = rmsnorm(x_in)
    for l in 0 .. NL-1:   y_l = verify_l(mixed_l)                       (router, routed experts, shared expert)
                          stream_{l+1} = stream_l + y_l;  mixed_{l+1} = rmsnorm(stream_{l+1})
    accept = greedy round of lm_head(mixed_NL) against the drafts          (fused, the logits stay in HBM)
    head_y = verify_NL(mixed_NL)                                        (the MTP head's MoE, map layer NL)

and the host reads back one int32 vector per round. The attention, linear-attention and hyper-connection segments
are outside this path; a single residual stream with an RMSNorm before every MoE stands in for them, so that the
chain keeps its scale over 48 layers. The head's MoE runs on the rows the head consumes after verification (the
pre-mixer rows GraphSet copies to `multi`, runtime/graphs.py:198-200); its attention and draft loop (engine/mtp.py)
are outside the path, so the caller supplies the drafts of the next round, as `draft_fn` does in _mtp_decode.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib
from ..kernels.gemv_affine import AffineWeight, LMHeadGreedy, LMHeadPQ
from .accept import AcceptResult
from .verify import MoEVerifyChain, MoEVerifyLayer


@dataclass
class MoEWeights:
    """Router and shared-expert weights of one MoE layer (bf16, the shapes MoEVerifyLayer takes)."""
    router_w: torch.Tensor
    sh_gate: torch.Tensor
    sh_up: torch.Tensor
    sh_down: torch.Tensor
    sh_g: torch.Tensor
    router_bias: torch.Tensor | None = None


def residual_rmsnorm(resid: torch.Tensor, y: torch.Tensor | None, mixed: torch.Tensor,
                     stream_out: torch.Tensor | None = None, weight: torch.Tensor | None = None,
                     eps: float = 1e-6) -> None:
    """stream_out = bf16(resid + y) (skipped when y is None), mixed = bf16(rmsnorm(stream_out or resid) * weight):
    `ssmoe_residual_rmsnorm` on the current stream."""
    for t in (resid, y, mixed, stream_out, weight):
        if t is not None and not t.is_cuda:
            raise ValueError("residual_rmsnorm takes GPU tensors only")
    for t in (resid, y, mixed, stream_out):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_contiguous() or t.shape != resid.shape):
            raise ValueError("resid, y, mixed and stream_out must be contiguous bf16 tensors of one shape [R, H]")
    if resid.dim() != 2:
        raise ValueError("resid must be [R, H]")
    if y is not None and stream_out is None:
        raise ValueError("stream_out is needed with y")
    if weight is not None and (weight.dtype != torch.bfloat16 or weight.numel() != resid.shape[1]):
        raise ValueError(f"weight must be bf16 [{resid.shape[1]}]")
    _lib.check(_lib.lib().ssmoe_residual_rmsnorm(
        resid.data_ptr(), _lib.ptr(y), _lib.ptr(weight), float(eps), resid.shape[0], resid.shape[1],
        _lib.ptr(stream_out), mixed.data_ptr(), torch.cuda.current_stream(resid.device).cuda_stream))


class MTPStepGraph:
    """One verify round over `depth` + 1 rows through `len(layers)` chained MoE layers, the lm_head with the greedy
    acceptance fused behind it, and the MTP head's MoE, captured in one HIP graph.

    `pool` holds the records of every layer and, when `head` is given, of map layer len(layers) (the MTP layer shares
    the table, runtime/pool.py:37-38). `norm_weights` (len(layers) + 1 bf16 [H] tensors, or None for ones) are the
    norms before each MoE and before the lm_head. Fill `x_in` [rows, H] bf16 and `drafts` int32 [depth], then
    `step()`; `result()` reads back the AcceptResult. `keep_logits` keeps the fp32 logits [rows, V] in `logits`.
    `fused` folds each norm and residual add into the verify launches (`mixed[l]` for l < NL then not written): one
    launch for all layers (ssmoe_moe_verify_chain) where the shape has a chain kernel and `single_launch`, else one
    ssmoe_moe_verify_layer_chain launch per layer; `fused=False` runs ssmoe_residual_rmsnorm between the layers. All
    give the same bits. `lm_head=None` leaves the lm_head and the acceptance out of the graph.

    `accept="pq"` fuses the p/q round (Leviathan et al. 2023, Alg. 1) instead of the greedy one. Its inputs are the
    draft head's logits of the round (`draft_logits` [depth, V]), the round's uniforms and drafts drawn from
    q = softmax(draft_logits / temperature): the rule divides by q(x), so it preserves the target distribution only
    for drafts drawn from q. `draw_drafts(uniforms)` draws them into `drafts` on the device (ssmoe_sample_rows);
    argmax drafts (the greedy proposal) belong to the greedy round."""

    def __init__(self, pool, layers: list[MoEWeights], lm_head: AffineWeight, depth: int,
                 head: MoEWeights | None = None, norm_weights: list[torch.Tensor | None] | None = None,
                 eps: float = 1e-6, top_k: int = 10, keep_logits: bool = False, fused: bool = True,
                 single_launch: bool = True, accept: str = "greedy", temperature: float = 1.0, device="cuda"):
        if not 1 <= depth <= 3:
            raise ValueError("depth must be 1..3 (the verify kernel takes up to 4 rows)")
        self.depth, self.rows = depth, depth + 1
        self.nl = len(layers)
        if self.nl < 1:
            raise ValueError("need at least one layer")
        if pool.map.numel() < (self.nl + (1 if head is not None else 0)) * pool.experts:
            raise ValueError("the pool's map has fewer layers than the step needs")
        H = pool.hidden
        if lm_head is not None and lm_head.k != H:
            raise ValueError(f"lm_head takes K = {lm_head.k}, the layers H = {H}")
        self.device = torch.device(device)
        self.eps = float(eps)
        self.fused = bool(fused)
        self.norm_weights = list(norm_weights) if norm_weights is not None else [None] * (self.nl + 1)
        if len(self.norm_weights) != self.nl + 1:
            raise ValueError(f"need {self.nl + 1} norm weights (one per layer and the final norm)")

        def verify(layer, w):
            return MoEVerifyLayer(pool, layer, w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, top_k=top_k,
                                  router_bias=w.router_bias, max_tokens=self.rows)

        self.layers = [verify(l, w) for l, w in enumerate(layers)]
        self.head = verify(self.nl, head) if head is not None else None
        R, dev = self.rows, self.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x_in = torch.zeros((R, H), **bf)
        self.drafts = torch.zeros(depth, dtype=torch.int32, device=dev)
        self.streams = [self.x_in] + [torch.zeros((R, H), **bf) for _ in range(self.nl)]
        self.mixed = [torch.zeros((R, H), **bf) for _ in range(self.nl + 1)]
        self.ys = [torch.zeros((R, H), **bf) for _ in range(self.nl)]
        self.ids = torch.zeros((self.nl, R, top_k), dtype=torch.int32, device=dev)
        self.weights = torch.zeros((self.nl, R, top_k), dtype=torch.float32, device=dev)
        self.head_y = torch.zeros((R, H), **bf)
        self.head_ids = torch.zeros((R, top_k), dtype=torch.int32, device=dev)
        self.head_weights = torch.zeros((R, top_k), dtype=torch.float32, device=dev)
        self.logits = (torch.zeros((R, lm_head.n), dtype=torch.float32, device=dev)
                       if keep_logits and lm_head is not None else None)
        # fused: one launch for every layer where the shape has a chain kernel (ssmoe_moe_verify_chain)
        self.chain = None
        l0 = self.layers[0]
        if self.fused and single_launch and MoEVerifyChain.supported(l0.hidden, l0.inter, l0.shared_inter,
                                                                     l0.top_k, l0.experts, dev):
            self.chain = MoEVerifyChain(self.layers, self.ys, list(self.ids), list(self.weights),
                                        stream_outs=self.streams[1:], norm_weights=self.norm_weights[:self.nl],
                                        eps=self.eps)
        if accept not in ("greedy", "pq"):
            raise ValueError(f"accept must be 'greedy' or 'pq', got {accept!r}")
        self.accept = accept
        self.temperature = float(temperature)
        self._drawer = None
        self.draft_logits = self.uniforms = None
        if lm_head is None:
            self.lm_head = None
        elif accept == "greedy":
            self.lm_head = LMHeadGreedy(lm_head, depth, device=dev)
        else:
            # p/q: the draft head's logits of the round's drafts and the round's uniforms are inputs like the drafts
            self.lm_head = LMHeadPQ(lm_head, depth, temperature, device=dev)
            self.draft_logits = torch.zeros((depth, lm_head.n), dtype=torch.float32, device=dev)
            self.uniforms = torch.zeros(depth + 1, dtype=torch.float32, device=dev)
            self.logits = self.lm_head.logits
        self.out = self.lm_head.out if lm_head is not None else None
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = None

    def _body(self) -> None:
        """Every launch of the round on the current stream, reading only the static buffers."""
        w = self.norm_weights
        if self.fused:
            if self.chain is not None:
                self.chain.run(self.streams[0])
            else:
                for l, layer in enumerate(self.layers):
                    layer.chain(self.streams[l], self.ys[l], self.ids[l], self.weights[l],
                                stream_out=self.streams[l + 1], norm_weight=w[l], eps=self.eps)
            residual_rmsnorm(self.streams[self.nl], None, self.mixed[self.nl], weight=w[self.nl], eps=self.eps)
        else:
            residual_rmsnorm(self.x_in, None, self.mixed[0], weight=w[0], eps=self.eps)
            for l, layer in enumerate(self.layers):
                layer(self.mixed[l], y=self.ys[l], ids=self.ids[l], weights=self.weights[l])
                residual_rmsnorm(self.streams[l], self.ys[l], self.mixed[l + 1], stream_out=self.streams[l + 1],
                                 weight=w[l + 1], eps=self.eps)
        if self.lm_head is not None and self.accept == "pq":
            self.lm_head.run_async(self.mixed[self.nl], self.draft_logits, self.drafts, self.uniforms)
        elif self.lm_head is not None:
            self.lm_head.run_async(self.mixed[self.nl], self.drafts, logits=self.logits)
        if self.head is not None:
            self.head(self.mixed[self.nl], y=self.head_y, ids=self.head_ids, weights=self.head_weights)

    def run_eager(self) -> torch.Tensor:
        """The round's launches without the graph (same kernels, same buffers)."""
        with torch.cuda.stream(self.stream):
            self._body()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        return self.out

    def capture(self) -> None:
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            self._body()                           # first launches outside the capture (module loads, workspaces)
        self.stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self._body()

    def step(self, x: torch.Tensor | None = None, drafts: torch.Tensor | None = None) -> torch.Tensor:
        """Replay the round (capturing it on first use) after copying `x` / `drafts` into the static inputs; returns
        the device result vector (int32 [depth + 5], Acceptor.greedy's layout) without waiting for it."""
        cur = torch.cuda.current_stream(self.device)
        if x is not None:
            self.x_in.copy_(x)
        if drafts is not None:
            self.drafts.copy_(drafts)
        if self.graph is None:
            self.capture()
        self.stream.wait_stream(cur)
        self.graph.replay()
        cur.wait_stream(self.stream)
        return self.out

    def draw_drafts(self, uniforms: torch.Tensor) -> torch.Tensor:
        """p/q rounds: draft token i ~ softmax(draft_logits[i] / temperature) with uniforms[i] (fp32 [depth] on the
        device) into `drafts`, on the current stream, before step() (the draft head's side of the round)."""
        if self.accept != "pq":
            raise ValueError("draw_drafts belongs to accept='pq' rounds; greedy rounds take argmax drafts")
        if self._drawer is None:
            from .accept import Acceptor
            self._drawer = Acceptor(self.depth, self.draft_logits.shape[1], device=self.device)
        return self._drawer.draw_drafts_async(self.draft_logits, uniforms, self.temperature, out=self.drafts)

    def result(self) -> AcceptResult:
        torch.cuda.current_stream(self.device).synchronize()
        return AcceptResult.from_out(self.out.cpu())
