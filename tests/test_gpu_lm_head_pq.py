"""The lm_head GEMV with the p/q round fused behind it (ssmoe_lm_head_pq, kernels.gemv_affine.LMHeadPQ) on the GPU:
its logits equal the GEMV's own (lin's bf16 values) and its round equals ssmoe_accept_pq on those logits bit for bit
(accepted drafts, emitted tokens, uniforms used, flags), across seeds, depths 0 to 3, temperatures, all-accept and
early-reject drafts, a non-finite row and a draft out of range; the p/q round inside the step graph equals its eager
launches on every replay."""
import numpy as np
import pytest
import torch

from slotstream_spark_amd.engine.accept import Acceptor
from slotstream_spark_amd.kernels.gemv_affine import AffineWeight, LMHeadPQ, gemv
from slotstream_spark_amd.memory.synth import normal_bf16

pytestmark = pytest.mark.gpu

K = 2048


def _lm_head(n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randint(-2**31, 2**31 - 1, (n, K // 8), generator=g, device="cuda", dtype=torch.int32)
    sc = (torch.randn((n, K // 64), generator=g, device="cuda") * 0.02).abs().to(torch.bfloat16)
    return AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, n, K)


@pytest.mark.parametrize("n,depth,temp,mode,seed", [(151936, 3, 0.7, "argmax", 1), (151936, 3, 0.7, "random", 2),
                                                    (151936, 1, 1.3, "argmax", 3), (50000, 2, 0.5, "random", 4),
                                                    (4099, 3, 2.0, "argmax", 5), (1000, 0, 0.7, "random", 6)])
def test_fused_pq_equals_gemv_then_accept(n, depth, temp, mode, seed):
    print(f"[lm_head pq] V={n} D={depth} T={temp} drafts={mode} seed={seed}", flush=True)
    w = _lm_head(n, 100 + seed)
    x = normal_bf16((depth + 1, K), 1.0, 200 + seed)
    ref_logits = gemv(x, w).to(torch.bfloat16).float()
    g = torch.Generator(device="cuda").manual_seed(300 + seed)
    draft = (0.8 * ref_logits[:depth] + 0.6 * torch.randn((depth, n), generator=g, device="cuda") * 3).contiguous()
    if mode == "argmax":
        drafts = draft.argmax(dim=1).to(torch.int32)
    else:
        drafts = torch.randint(0, n, (depth,), generator=g, device="cuda", dtype=torch.int32)
    u = torch.rand(depth + 1, generator=g, device="cuda")
    head = LMHeadPQ(w, depth, temp)
    for rep in range(2):  # the workspace's counters are left zero for the next call
        out = head.run_async(x, draft, drafts, u).clone()
        torch.cuda.synchronize()
        assert torch.equal(head.logits, ref_logits)
        acc = Acceptor(depth, n)
        want = acc.pq_async(ref_logits, draft, drafts, u, temp)
        torch.cuda.synchronize()
        assert torch.equal(out, want), (rep, out.cpu().tolist(), want.cpu().tolist())
    print(f"out {out.cpu().tolist()}")


def test_fused_pq_non_finite_row_and_bad_draft():
    n, depth, temp = 3000, 3, 0.7
    w = _lm_head(n, 9)
    x = normal_bf16((depth + 1, K), 1.0, 10)
    x[2, 5] = float("nan")
    ref_logits = gemv(x, w).to(torch.bfloat16).float()
    draft = torch.randn((depth, n), device="cuda") * 3
    for drafts in (torch.tensor([0, 1, 2], dtype=torch.int32, device="cuda"),
                   torch.tensor([5, n + 7, 1], dtype=torch.int32, device="cuda")):
        u = torch.full((depth + 1,), 0.25, device="cuda")
        out = LMHeadPQ(w, depth, temp).run_async(x, draft, drafts, u)
        want = Acceptor(depth, n).pq_async(ref_logits, draft, drafts, u, temp)
        torch.cuda.synchronize()
        assert torch.equal(out, want), (out.cpu().tolist(), want.cpu().tolist())
