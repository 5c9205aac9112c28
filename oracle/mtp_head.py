"""CPU restatement of the MTP draft head without attention. TEST INFRASTRUCTURE ONLY.

Only tests/ import this module, to check the head's HIP path against it; the product package never imports it.
Arrays are bf16 bit patterns (uint16) unless stated. The elementary ops are the C restatement (oracle.rmsnorm_groups,
dense_epi, hc_mean, hc_inject), which fix the reduction orders the kernels use, so the head's dense part is
reproduced bit for bit; the MoE is supplied by the caller (`moe(mixed) -> y`), since its routed experts are checked
to a tolerance elsewhere.

Composition, following the reference:
  fuse        engine/mtp.py:184-192     e = lin(rmsnorm(embedded)); h = lin(rmsnorm(multi) as [S hc, H]) per branch;
                                         (e + h) flattened to [S, hc H]
  hc_mix      model/layers.py:190-198   hn = rmsnorm per H-group; m = silu(lin(hn, down) / hc);
                                         m = sigmoid(lin(m, up)); mixed = mean_c(m * hn); inj = 2 sigmoid(lin(hn, inj) / hc)
  step        engine/mtp.py:209-227     fuse -> (attention omitted) -> hc_mix(mlp) -> MoE -> h + y inj -> hc_mix(mixer)
  draft       engine/mtp.py:265-277     token -> embed -> step -> argmax(bf16 logits), k times

Pins (tests/test_mtp_oracle.py): rmsnorm and hc_mix against the reference's own torch functions
(reference_torch.rmsnorm, RefModel.gated_residual) on committed fixtures, to the difference of two fp32 summation
orders; fuse and step by closed forms that a transposed reshape, a per-group instead of a full-width norm, or a
missing residual would break.
"""
from __future__ import annotations

import numpy as np

from . import oracle as orc


def fuse(e, multi, W, hc, eps=1e-6):
    """e [S, H], multi [S, hc H] -> [S, hc H]."""
    S, H = e.shape
    en = orc.rmsnorm_groups(e, W["pre_fc_norm_embedding"], eps)
    ep = orc.dense_epi(en, W["fc_embedding"])
    mn = orc.rmsnorm_groups(multi, W["pre_fc_norm_hidden"], eps)
    h = orc.dense_epi(mn.reshape(S * hc, H), W["fc_hidden"], orc.EPI_ADD, add_bits=ep, add_div=hc)
    return h.reshape(S, hc * H), dict(e_norm=en, e_proj=ep, m_norm=mn)


def hc_mix(hyp, P, hc, eps=1e-6, inject=True):
    """hyp [S, hc H]; P with hc_norm, down, up (and inject) -> (mixed [S, H], inj [S, hc] or None, parts)."""
    H = hyp.shape[1] // hc
    hn = orc.rmsnorm_groups(hyp, P["hc_norm"], eps, group=H)
    low = orc.dense_epi(hn, P["down"], orc.EPI_SILU_DIV, hc=hc)
    mw = orc.dense_epi(low, P["up"], orc.EPI_SIGMOID)
    mixed = orc.hc_mean(mw, hn, hc)
    inj = orc.dense_epi(hn, P["inject"], orc.EPI_INJECT, hc=hc) if inject else None
    return mixed, inj, dict(hn=hn, low=low, mix_w=mw)


def step(e, multi, W, hc, moe, eps=1e-6):
    """One head step (attention omitted): -> (out [S, H], h [S, hc H], intermediates)."""
    h, parts = fuse(e, multi, W, hc, eps)
    mixed, inj, p1 = hc_mix(h, W["mlp_hc"], hc, eps)
    y = moe(mixed)
    h2 = orc.hc_inject(h, y, inj)
    out, _, p2 = hc_mix(h2, W["mixer_hc"], hc, eps, inject=False)
    parts.update(fused=h, mixed=mixed, inj=inj, y=y, h=h2, out=out, hn=p1["hn"], low=p1["low"], mix_w=p1["mix_w"],
                 hn2=p2["hn"], low2=p2["low"], mix_w2=p2["mix_w"])
    return out, h2, parts
