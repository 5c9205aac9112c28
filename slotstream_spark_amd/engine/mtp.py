"""MTP draft head of the MoE path, without its attention (drop-in for slotstream_spark/engine/mtp.py:78-277).

One head step over S rows, as MTPHead.step (engine/mtp.py:209-227) with the attention output taken as zero:

    h     = fuse(embedded, multi)                              engine/mtp.py:184-192
            e = lin(rmsnorm(embedded)), per branch c: lin(rmsnorm_fullwidth(multi))[c] + e
    mixed, inj = hc_mix(mlp_hyper_connection, h)               model/layers.py:190-198 (seg_router :336-348)
    y     = MoE(mixed): router, routed experts of map row MAP_ROW, shared expert     (_moe, engine/mtp.py:194-207)
    h     = h + (y scaled per branch by inj)                   engine/mtp.py:226
    out   = hc_mix(hyper_connection_mixer, h)                  engine/mtp.py:229-230

Every op is a libssmoe.so launch (kernels/head_ops.py, the verify layer for the MoE, the affine lm_head argmax).
With hc = 4 the dense ops between the MoE and the lm_head run as six fused launches (ssmoe_head_gemv: each RMSNorm,
the embedding lookup and the injection inside the GEMV that consumes them, the inject rows beside the down rows, the
branch mean behind the up GEMV), with the bits of the separate ops. `draft(token, k)` chains k steps on the device:
each step's embedding row is read by the first launch at the token the previous step's lm_head argmax wrote, so the
k drafts reach the host once, at the end, and the chain can be captured in a HIP graph (DraftGraph).

Out of this path: the attention segment (hc_mix of attn_hyper_connection, QSA over the head's own KV/indexer cache,
its residual). MTPState keeps the position bookkeeping of the reference's state (pos, aligned, fork, reset) with no
cache behind it.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ..kernels.gemv_affine import AffineWeight, LMHeadArgmax, gemv
from ..kernels.head_ops import (EPI_ADD, EPI_INJECT, EPI_SIGMOID, EPI_SILU_DIV, gather_rows, hc_inject, hc_mean,
                                head_gemv, lin_epi, rmsnorm)
from .verify import MoEVerifyLayer

MAP_ROW = 48   # the head's layer index in the 49-row expert map (engine/mtp.py:38)
DEPTH = 2      # draft tokens per round (engine/mtp.py:48)


def draft_depth(max_ctx: int, pos: int, depth: int = DEPTH) -> int:
    """Drafts a round may verify: min(depth, max_ctx - pos - 1) (engine/mtp.py:78-81)."""
    return max(0, min(depth, max_ctx - pos - 1))


@dataclass
class HyperConnection:
    """Weights of one hc_mix (model/layers.py:190-198), bf16: hc_norm [hc H], down [L, hc H], up [hc H, L],
    inject [hc, hc H] (None for the final mixer, which injects nothing)."""
    hc_norm: torch.Tensor
    down: torch.Tensor
    up: torch.Tensor
    inject: torch.Tensor | None = None


@dataclass
class HeadWeights:
    """The head's dense weights, bf16 (engine/mtp.py:188-191 names): the main model's embedding table [V, H],
    pre_fc_norm_embedding [H], fc_embedding [H, H], pre_fc_norm_hidden [hc H], fc_hidden [H, H], and the two
    hyper-connections (layers.0.mlp_hyper_connection, hyper_connection_mixer)."""
    embed: torch.Tensor
    pre_fc_norm_embedding: torch.Tensor
    fc_embedding: torch.Tensor
    pre_fc_norm_hidden: torch.Tensor
    fc_hidden: torch.Tensor
    mlp_hc: HyperConnection
    mixer_hc: HyperConnection


class MTPState:
    """Position of the head's cache (engine/mtp.py:84-115): one entry per consumed token except the first."""

    def __init__(self, max_ctx: int):
        self.max_ctx, self.pos = max_ctx, 0

    @property
    def offset(self) -> int:
        return self.pos

    def aligned(self, consumed: int) -> bool:
        return consumed > 0 and self.pos == consumed - 1

    def fork(self) -> "MTPState":
        s = MTPState(self.max_ctx)
        s.pos = self.pos
        return s

    def reset(self) -> None:
        self.pos = 0


class _Rows:
    """Intermediates of head steps over S rows each, one slice per step (kept so a caller can read them back)."""

    def __init__(self, steps: int, S: int, H: int, hc: int, low_mlp: int, low_mix: int, K: int, device):
        bf = dict(dtype=torch.bfloat16, device=device)
        self.steps, self.S = steps, S
        self.emb = torch.empty(steps, S, H, **bf)
        self.e_norm = torch.empty(steps, S, H, **bf)
        self.e_proj = torch.empty(steps, S, H, **bf)
        self.m_norm = torch.empty(steps, S, hc * H, **bf)
        self.fused = torch.empty(steps, S, hc * H, **bf)
        self.hn = torch.empty(steps, S, hc * H, **bf)
        self.low = torch.empty(steps, S, low_mlp, **bf)
        self.mix_w = torch.empty(steps, S, hc * H, **bf)
        self.mixed = torch.empty(steps, S, H, **bf)
        self.inj = torch.empty(steps, S, hc, **bf)
        self.y = torch.empty(steps, S, H, **bf)
        self.ids = torch.empty(steps, S, K, dtype=torch.int32, device=device)
        self.weights = torch.empty(steps, S, K, dtype=torch.float32, device=device)
        self.h = torch.empty(steps, S, hc * H, **bf)
        self.hn2 = torch.empty(steps, S, hc * H, **bf)
        self.low2 = torch.empty(steps, S, low_mix, **bf)
        self.mix_w2 = torch.empty(steps, S, hc * H, **bf)
        self.out = torch.empty(steps, S, H, **bf)


class MTPHead:
    """The MoE-only MTP head (engine/mtp.py:144-277): fuse, the MLP hyper-connection, the head's MoE (a verify layer
    whose map row is the head's), the residual, the final mixer and the shared lm_head. `moe` must be built on
    the head's map row (MAP_ROW in the full model) with at least `max_rows` tokens per call."""

    def __init__(self, weights: HeadWeights, moe: MoEVerifyLayer, lm_head: AffineWeight, hc: int, eps: float = 1e-6,
                 max_ctx: int = 1 << 20, max_rows: int = 4):
        self.w, self.moe, self.lm_head = weights, moe, lm_head
        self.H, self.hc, self.eps = moe.hidden, int(hc), float(eps)
        self.topk = moe.top_k
        self.max_rows = min(max_rows, moe.max_tokens)
        H, n = self.H, self.hc * self.H
        w = weights
        if w.embed.dim() != 2 or w.embed.shape[1] != H:
            raise ValueError(f"embed must be [V, {H}]")
        checks = [("pre_fc_norm_embedding", w.pre_fc_norm_embedding, (H,)), ("fc_embedding", w.fc_embedding, (H, H)),
                  ("pre_fc_norm_hidden", w.pre_fc_norm_hidden, (n,)), ("fc_hidden", w.fc_hidden, (H, H))]
        for name, hcw, inject in (("mlp_hc", w.mlp_hc, True), ("mixer_hc", w.mixer_hc, False)):
            L = hcw.down.shape[0]
            checks += [(name + ".hc_norm", hcw.hc_norm, (n,)), (name + ".down", hcw.down, (L, n)),
                       (name + ".up", hcw.up, (n, L))]
            if inject:
                if hcw.inject is None:
                    raise ValueError(f"{name}.inject is required")
                checks.append((name + ".inject", hcw.inject, (self.hc, n)))
        for name, t, shape in checks:
            if tuple(t.shape) != shape or t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous bf16 {shape}, got {tuple(t.shape)} {t.dtype}")
        if lm_head.k != H:
            raise ValueError(f"lm_head has K={lm_head.k}, the head H={H}")
        self.vocab = lm_head.n
        if w.embed.shape[0] < self.vocab:
            raise ValueError("the embedding table must cover the lm_head's vocabulary")
        self.argmax = LMHeadArgmax(lm_head, max_rows=self.max_rows, round_bf16=True, device=w.embed.device)
        self.state = MTPState(max_ctx)
        self.prev_multi: torch.Tensor | None = None
        self.consumed = 0
        self._draft_rows: dict[int, _Rows] = {}

    # ------------------------------------------------------------------ one head step
    def _rows(self, steps: int, S: int) -> _Rows:
        return _Rows(steps, S, self.H, self.hc, self.w.mlp_hc.down.shape[0], self.w.mixer_hc.down.shape[0],
                     self.topk, self.w.embed.device)

    def fuse(self, embedded: torch.Tensor | None, multi: torch.Tensor, r: _Rows | None = None, i: int = 0,
             idx: torch.Tensor | None = None) -> torch.Tensor:
        """embedded bf16 [S, H] (or, with idx, the embedding rows idx: int32 [S] on the device), multi bf16
        [S, hc H] -> bf16 [S, hc H] (engine/mtp.py:184-192): two launches, each RMSNorm inside the GEMV after it."""
        S, H, hc, w = multi.shape[0], self.H, self.hc, self.w
        r = r if r is not None else self._rows(1, S)
        src = w.embed if idx is not None else embedded
        head_gemv(src, w.fc_embedding, r.e_proj[i], S=S, n=H, K=H, src_idx=idx, norm_w=w.pre_fc_norm_embedding,
                  eps=self.eps, group=H, x_out=r.e_norm[i], h_out=r.emb[i] if idx is not None else None)
        head_gemv(multi, w.fc_hidden, r.fused[i].view(S * hc, H), S=S, n=hc * H, K=H, norm_w=w.pre_fc_norm_hidden,
                  eps=self.eps, group=hc * H, epi=EPI_ADD, add=r.e_proj[i], add_div=hc, x_out=r.m_norm[i])
        return r.fused[i]

    def hc_mix(self, hcw: HyperConnection, hyp: torch.Tensor, hn: torch.Tensor, low: torch.Tensor,
               mix_w: torch.Tensor, mixed: torch.Tensor, inj: torch.Tensor | None = None):
        """model/layers.py:190-198 into the given buffers: hn = rmsnorm per branch, low = silu(lin(hn, down) / hc),
        mix_w = sigmoid(lin(low, up)), mixed = mean over branches of mix_w * hn, inj = 2 sigmoid(lin(hn, inject) / hc)
        -> (mixed, inj or None)."""
        rmsnorm(hyp, hcw.hc_norm, self.eps, group=self.H, out=hn)
        lin_epi(hn, hcw.down, EPI_SILU_DIV, hc=self.hc, out=low)
        lin_epi(low, hcw.up, EPI_SIGMOID, out=mix_w)
        hc_mean(mix_w, hn, self.hc, out=mixed)
        if inj is None:
            return mixed, None
        lin_epi(hn, hcw.inject, EPI_INJECT, hc=self.hc, out=inj)
        return mixed, inj

    def _step_rows(self, embedded, multi, r: _Rows, i: int, idx: torch.Tensor | None = None):
        h = self.fuse(embedded, multi, r, i, idx)
        if self.hc != 4:
            # the separate launches (the fused branch mean takes four branches)
            self.hc_mix(self.w.mlp_hc, h, r.hn[i], r.low[i], r.mix_w[i], r.mixed[i], r.inj[i])
            self.moe(r.mixed[i], y=r.y[i], ids=r.ids[i], weights=r.weights[i])
            hc_inject(h, r.y[i], r.inj[i], out=r.h[i])
            self.hc_mix(self.w.mixer_hc, r.h[i], r.hn2[i], r.low2[i], r.mix_w2[i], r.out[i])
            return r.out[i], r.h[i]
        S, H, hc, n, mlp, mix = h.shape[0], self.H, self.hc, self.hc * self.H, self.w.mlp_hc, self.w.mixer_hc
        # hc_mix of the MLP: norm + down rows + inject rows, then up + the branch mean (model/layers.py:190-198)
        head_gemv(h, mlp.down, r.low[i], S=S, n=n, K=n, norm_w=mlp.hc_norm, eps=self.eps, group=H,
                  epi=EPI_SILU_DIV, hc=hc, w2=mlp.inject, out2=r.inj[i], epi2=EPI_INJECT, x_out=r.hn[i])
        L = mlp.down.shape[0]
        head_gemv(r.low[i], mlp.up, r.mix_w[i], S=S, n=L, K=L, epi=EPI_SIGMOID, hc=hc, mean_hn=r.hn[i],
                  mean_out=r.mixed[i])
        self.moe(r.mixed[i], y=r.y[i], ids=r.ids[i], weights=r.weights[i])
        # the injection (engine/mtp.py:226), then hc_mix of the mixer
        head_gemv(h, mix.down, r.low2[i], S=S, n=n, K=n, inj=r.inj[i], inj_y=r.y[i], inj_hc=hc, norm_w=mix.hc_norm,
                  eps=self.eps, group=H, epi=EPI_SILU_DIV, hc=hc, h_out=r.h[i], x_out=r.hn2[i])
        L2 = mix.down.shape[0]
        head_gemv(r.low2[i], mix.up, r.mix_w2[i], S=S, n=L2, K=L2, epi=EPI_SIGMOID, hc=hc, mean_hn=r.hn2[i],
                  mean_out=r.out[i])
        return r.out[i], r.h[i]

    def step(self, embedded: torch.Tensor, multi: torch.Tensor, state: MTPState, state_only: bool = False):
        """One head step over S rows, advancing `state` -> (out bf16 [S, H] for the lm_head, h bf16 [S, hc H] for
        chaining); with `state_only` (None, the fused stream) (engine/mtp.py:209-227)."""
        S = embedded.shape[0]
        if state.pos + S > state.max_ctx:
            raise ValueError(f"head context {state.pos + S} exceeds {state.max_ctx}")
        if tuple(embedded.shape) != (S, self.H) or tuple(multi.shape) != (S, self.hc * self.H):
            raise ValueError(f"embedded must be [S, {self.H}] and multi [S, {self.hc * self.H}]")
        if S < 1 or (not state_only and S > self.max_rows):
            raise ValueError(f"a head step takes 1..{self.max_rows} rows, got {S}")
        r = self._rows(1, S)
        if state_only:
            h = self.fuse(embedded, multi, r, 0)
            state.pos += S
            return None, h
        state.pos += S
        return self._step_rows(embedded, multi, r, 0)

    def logits(self, out: torch.Tensor) -> torch.Tensor:
        """lm_head over the head's output rows -> fp32 [S, V]: lin's bf16 result as fp32 (engine/mtp.py:232-236)."""
        return gemv(out, self.lm_head).to(torch.bfloat16).float()

    # ------------------------------------------------------------------ the engine-facing calls
    def reset(self) -> None:
        self.state.reset()
        self.prev_multi = None
        self.consumed = 0

    def embed(self, ids) -> torch.Tensor:
        idx = torch.as_tensor(list(ids), dtype=torch.int32).to(self.w.embed.device)
        return gather_rows(self.w.embed, idx)

    def consume(self, ids, multi_rows: torch.Tensor) -> torch.Tensor:
        """Feed consumed main-model tokens with the main model's multi rows of the same positions (engine/mtp.py:
        244-263): the entry of ids[i] fuses the multi of the previous position with ids[i]; at sequence start ids[0]
        has none. Keeps the last multi row for the next call and for `draft`."""
        ids = [int(t) for t in ids]
        S = len(ids)
        if S == 0 or tuple(multi_rows.shape) != (S, self.hc * self.H):
            raise ValueError("consume needs a nonempty chunk and one multi row per token")
        start = 1 if self.prev_multi is None else 0
        if S - start > 0:
            e = self.embed(ids[start:])
            prev = multi_rows[:S - 1] if self.prev_multi is None else torch.cat([self.prev_multi, multi_rows[:S - 1]], 0)
            self.step(e, prev.contiguous(), self.state, state_only=True)
        self.prev_multi = multi_rows[-1:].clone()
        self.consumed += S
        if not self.state.aligned(self.consumed):
            raise RuntimeError(f"mtp.offset {self.state.pos} != token_count {self.consumed} - 1")
        return self.prev_multi

    def draft_rows(self, k: int) -> _Rows:
        """The per-step intermediates of the last draft of depth k (one-row steps)."""
        if k not in self._draft_rows:
            self._draft_rows[k] = self._rows(k, 1)
        return self._draft_rows[k]

    def draft_async(self, token: torch.Tensor, multi: torch.Tensor, k: int, out: torch.Tensor,
                    state: MTPState | None = None) -> torch.Tensor:
        """k greedy drafts after the device token `token` (int32 [1]) chained from `multi` (bf16 [1, hc H]) into
        `out` (int32 [k]) with no host synchronisation: step i embeds out[i - 1] (token for i = 0) by a device-side
        gather, runs the head, and writes the argmax of its lm_head row to out[i]. Same launches on every call."""
        if token.dtype != torch.int32 or token.numel() != 1 or out.dtype != torch.int32 or out.numel() != k:
            raise ValueError(f"token must be int32 [1] and out int32 [{k}]")
        if tuple(multi.shape) != (1, self.hc * self.H):
            raise ValueError(f"multi must be [1, {self.hc * self.H}]")
        st = state if state is not None else self.state.fork()
        if st.pos + k > st.max_ctx:
            raise ValueError(f"head context {st.pos + k} exceeds {st.max_ctx}")
        r = self.draft_rows(k)
        prev_h = multi
        for i in range(k):
            src = token if i == 0 else out[i - 1:i]
            o, prev_h = self._step_rows(None, prev_h, r, i, idx=src)
            self.argmax(o, ids=out[i:i + 1])
        st.pos += k
        return out

    def draft(self, token: int, k: int = 2) -> list[int]:
        """Greedy draft ids after the pending token (not consumed yet), chained from the last consumed multi, on a
        fork of the state (engine/mtp.py:265-277) -> list of k ints."""
        if self.prev_multi is None:
            raise RuntimeError("draft before any consume")
        dev = self.w.embed.device
        tok = torch.tensor([int(token)], dtype=torch.int32, device=dev)
        out = torch.empty(k, dtype=torch.int32, device=dev)
        self.draft_async(tok, self.prev_multi, k, out)
        return [int(t) for t in out.cpu()]


class DraftGraph:
    """The k-step draft chain captured once as a HIP graph: set `token` (int32 [1]) and `multi` (bf16 [1, hc H]) in
    place, replay, read `out` (int32 [k]). The head's state is not advanced (drafting runs on a fork)."""

    def __init__(self, head: MTPHead, k: int):
        dev = head.w.embed.device
        self.head, self.k = head, k
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.multi = torch.zeros(1, head.hc * head.H, dtype=torch.bfloat16, device=dev)
        self.out = torch.zeros(k, dtype=torch.int32, device=dev)
        self.graph = None

    def _body(self) -> None:
        self.head.draft_async(self.token, self.multi, self.k, self.out, state=MTPState(self.k))

    def capture(self) -> None:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._body()  # warm-up outside the capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._body()
        self.graph = g

    def replay(self) -> torch.Tensor:
        if self.graph is None:
            self.capture()
        self.graph.replay()
        return self.out
