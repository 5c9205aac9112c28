"""The self-speculative greedy loop over the MoE path (drop-in for _mtp_decode, slotstream_spark/engine/
generate.py:152-238, at temperature 0).

MoEStack is the main model of the loop as far as this path reaches: token rows -> embedding rows -> the chained MoE
layers of a verify round (MTPStepGraph, one HIP graph) -> final norm -> lm_head with the greedy round fused behind it.
Without attention each row depends on its own token only, so the greedy sequence is fixed by the first token, and a
speculative decode must emit exactly the sequence plain one-row steps emit, whatever the drafts are.

A round, as in the reference: the MTP head drafts DEPTH tokens after the pending one (on a fork of its state), the
stack verifies pending + drafts in one pass, the host walks the rows with the plain loop's stopping rules, keeps the
first 1 + good rows (rollback cuts the position and the token list; the MoE stack records no recurrent state) and
feeds the kept tokens with their final stream rows (the head's `multi`, hc = 1 here) to the head. Near the context end
(fewer than DEPTH drafts fit) the loop switches for good to plain steps.
"""
from __future__ import annotations

import time

import torch

from ..kernels.gemv_affine import AffineWeight, LMHeadArgmax
from ..kernels.head_ops import gather_rows
from . import mtp as mtp_mod
from . import rollback as rb
from .accept import AcceptResult
from .step import MoEWeights, MTPStepGraph


class MoEStack:
    """`len(layers)` MoE layers on one residual stream behind an embedding table and in front of the lm_head, run
    `depth` + 1 rows at a time. `st` (rollback.SeqState) and `record` (rollback.StepRecord, empty) hold the sequence."""

    def __init__(self, pool, layers: list[MoEWeights], lm_head: AffineWeight, embed: torch.Tensor,
                 depth: int = mtp_mod.DEPTH, norm_weights=None, eps: float = 1e-6, top_k: int = 10,
                 max_ctx: int = 1 << 20, device="cuda"):
        if embed.dim() != 2 or embed.shape[1] != pool.hidden or embed.dtype != torch.bfloat16:
            raise ValueError(f"embed must be bf16 [V, {pool.hidden}]")
        self.graph = MTPStepGraph(pool, layers, lm_head, depth, norm_weights=norm_weights, eps=eps, top_k=top_k,
                                  device=device)
        self.depth, self.rows, self.nl = depth, depth + 1, len(layers)
        self.embed, self.max_ctx, self.device = embed, max_ctx, torch.device(device)
        self.argmax = LMHeadArgmax(lm_head, max_rows=self.rows, round_bf16=True, device=device)
        # the plain steps' logits, kept for the finiteness check of _mtp_decode's plain loop (generate.py:186-189)
        self.plain_logits = torch.empty((self.rows, lm_head.n), dtype=torch.float32, device=self.device)
        self.last_finite: list[bool] = []
        self.tok_rows = torch.zeros(self.rows, dtype=torch.int32, device=self.device)
        self.row_ids = torch.zeros(self.rows, dtype=torch.int32, device=self.device)
        self.st = rb.SeqState()
        self.record = rb.StepRecord(self.st, self.rows)

    def reset(self) -> None:
        """A new sequence (the captured graph and the buffers stay)."""
        self.st = rb.SeqState()
        self.record = rb.StepRecord(self.st, self.rows)

    @property
    def multi(self) -> torch.Tensor:
        """The final stream rows of the last pass [rows, H] (the pre-mixer rows the head consumes)."""
        return self.graph.streams[self.nl]

    def _pass(self, tokens: list[int]) -> torch.Tensor:
        t = list(tokens) + [0] * (self.rows - len(tokens))
        self.tok_rows.copy_(torch.tensor(t, dtype=torch.int32))
        g = self.graph
        gather_rows(self.embed, self.tok_rows, out=g.x_in)
        g.drafts.copy_(self.tok_rows[1:])
        return g.step()

    def step(self, tokens: list[int]) -> AcceptResult:
        """The verify pass of a round over pending + drafts (exactly `rows` tokens) with the record begun."""
        if len(tokens) != self.rows:
            raise ValueError(f"a round verifies {self.rows} tokens, got {len(tokens)}")
        self.record.begin()
        self._pass(tokens)
        self.st.pos += self.rows
        self.st.tokens += [int(t) for t in tokens]
        return self.graph.result()

    def forward(self, tokens: list[int]) -> tuple[list[int], torch.Tensor]:
        """Plain steps over `tokens` (at most `rows` at a time): -> (the greedy next token after each, their final
        stream rows [len, H]). Advances the position by len(tokens). `last_finite[i]` says whether row i's logits
        were all finite (a non-finite row's token is torch.argmax's, NaN counting as the maximum)."""
        nxt, multi, fin = [], [], []
        for c0 in range(0, len(tokens), self.rows):
            chunk = [int(t) for t in tokens[c0:c0 + self.rows]]
            self._pass(chunk)
            g = self.graph
            self.argmax(g.mixed[self.nl], ids=self.row_ids, logits=self.plain_logits)
            nxt += self.row_ids.cpu().tolist()[:len(chunk)]
            fin += torch.isfinite(self.plain_logits[:len(chunk)]).all(dim=1).cpu().tolist()
            multi.append(self.multi[:len(chunk)].clone())
            self.st.pos += len(chunk)
            self.st.tokens += chunk
        self.last_finite = [bool(f) for f in fin]
        return nxt, torch.cat(multi, 0)


def mtp_decode(stack: MoEStack, head: mtp_mod.MTPHead, prompt: list[int], max_tokens: int, eos=(), on_token=None,
               draft_fn=None):
    """Greedy self-speculative decode after `prompt` -> (tokens, nan, round_seconds, stats), as _mtp_decode.
    `draft_fn(pending, depth, n_out)` replaces the head's drafts when given (as in the reference). Non-finite logits
    end the loop as in the reference (generate.py:163-164, 186-189, 210-212): no token for that row, `nan` True, and
    a verify round that met one still rolls back to its good rows and feeds them to the head before returning."""
    D = stack.depth
    out, step_s, nan = [], [], False
    st = {"rounds": 0, "plain_steps": 0, "drafted": 0, "accepted": 0, "attempts_by_depth": [0] * D,
          "accepted_by_depth": [0] * D, "emitted_by_round": [], "verify_rows": 0}
    nxt, multi = stack.forward(prompt)
    head.consume(prompt, multi)
    if not stack.last_finite[-1]:
        return out, True, step_s, st
    tok = nxt[-1]
    out.append(tok)
    if on_token:
        on_token(tok)
    if tok in eos or len(out) == max_tokens:
        return out, nan, step_s, st
    pending, use_mtp = tok, True
    while len(out) < max_tokens:
        if use_mtp:
            depth = mtp_mod.draft_depth(stack.max_ctx, stack.st.pos, D)
            if head.state.pos + 1 + D > head.state.max_ctx:
                depth = 0
            use_mtp = depth >= D
        t1 = time.perf_counter()
        if not use_mtp:
            if stack.st.pos + 1 > stack.max_ctx:
                break
            tok = stack.forward([pending])[0][0]
            step_s.append(time.perf_counter() - t1)
            st["plain_steps"] += 1
            if not stack.last_finite[0]:
                nan = True
                break
            out.append(tok)
            if on_token:
                on_token(tok)
            if tok in eos or len(out) == max_tokens:
                break
            pending = tok
            continue
        drafts = [int(d) for d in (draft_fn(pending, D, len(out)) if draft_fn else head.draft(pending, D))]
        ck = rb.checkpoint(stack)
        res = stack.step([pending] + drafts)
        st["rounds"] += 1
        st["drafted"] += len(drafts)
        st["verify_rows"] += 1 + len(drafts)
        good, nextp, done, before = 0, None, False, len(out)
        for i in range(res.n_emit):
            tok = res.tokens[i]
            out.append(tok)
            if on_token:
                on_token(tok)
            if tok in eos or len(out) == max_tokens:
                done = True
                break
            if i < len(drafts):
                st["attempts_by_depth"][i] += 1
                if tok == drafts[i]:
                    st["accepted_by_depth"][i] += 1
                    good += 1
                    continue
            nextp = tok
            break
        if nextp is None and not done:
            # the greedy round stopped at a non-finite row (flags bit 1): no token for it, as the reference's loop
            nan, done = True, True
        st["accepted"] += good
        st["emitted_by_round"].append(len(out) - before)
        keep = 1 + good
        rb.rollback(stack, stack.record, ck, keep, stack.rows)
        head.consume([pending] + drafts[:good], stack.multi[:keep].clone())
        step_s.append(time.perf_counter() - t1)
        if done:
            break
        pending = nextp
    return out, nan, step_s, st
