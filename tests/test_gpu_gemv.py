"""Affine 4-bit GEMV (gemv for AffineWeight bits=4 gs=64, kernels/gemv_affine.py:214-262) and the lm_head fused
with the greedy round: against the fp64 GEMV on the exactly dequantized weights (tolerance scaled by sum |x w|), the
reference's invariance rule (R rows = R one-row calls, bit for bit), and oracle.accept_greedy on the kernel's own
logits (bitwise)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.kernels.gemv_affine import AffineWeight, LMHeadGreedy, gemv

pytestmark = pytest.mark.gpu
TOL = 2e-5  # relative to sum_k |x_k w_k|: fp32 accumulation of exact bf16 products over K <= 4096


def make_weight(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-2**31, 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int64).to(torch.int32)
    s = (torch.randn((n, k // 64), generator=g) * 0.02).abs().to(torch.bfloat16)
    b = (-8 * s.float()).to(torch.bfloat16)
    b = b + (torch.randn((n, k // 64), generator=g) * 0.002).to(torch.bfloat16)
    return AffineWeight(q.cuda(), s.cuda(), b.cuda(), 4, 64, n, k)


def host(w):
    return w.q.cpu().numpy(), w.s.cpu().view(torch.int16).numpy().view(np.uint16), \
        w.b.cpu().view(torch.int16).numpy().view(np.uint16)


def check_fp64(y, x, w, rows=None):
    q, s, b = host(w)
    xs = x.float().cpu().numpy()
    if rows is not None:
        q, s, b = q[rows], s[rows], b[rows]
    y64, bound = O.gemv_affine4_fp64(xs, q, s, b)
    yy = y.cpu().numpy() if rows is None else y.cpu().numpy()[:, rows]
    err = np.abs(yy - y64)
    assert (err <= TOL * bound + 1e-6).all(), float((err / (bound + 1e-30)).max())


@pytest.mark.parametrize("k,n,r,xf32", [(1024, 1000, 1, False), (2560, 4099, 3, False), (2048, 777, 4, True),
                                          (4096, 2048, 2, False), (2560, 1024, 6, False), (4096, 333, 5, True)])
def test_gemv_fp64_and_invariance(k, n, r, xf32):
    print(f"[gemv] k={k} n={n} r={r} xf32={xf32}", flush=True)
    w = make_weight(n, k, 1000 + k + n)
    g = torch.Generator().manual_seed(k + r)
    x = torch.randn((r, k), generator=g).to(torch.float32 if xf32 else torch.bfloat16).cuda()
    y = gemv(x, w)
    torch.cuda.synchronize()
    check_fp64(y, x, w)
    for i in range(r):  # invariance: every row equals its one-row call
        yi = gemv(x[i:i + 1].contiguous(), w)
        assert torch.equal(yi[0], y[i]), i


def test_lm_head_shape_sampled_rows():
    """The lm_head shape (248,320 x 2560, 4 verify rows): fp64 check on a sample of rows, invariance on row 2."""
    n, k = 248320, 2560
    w = make_weight(n, k, 77)
    x = torch.randn((4, k), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    y = gemv(x, w)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(0).choice(n, 3000, replace=False))
    rows[-1] = n - 1
    check_fp64(y, x, w, rows)
    assert torch.equal(gemv(x[2:3].contiguous(), w)[0], y[2])


@pytest.mark.parametrize("n,depth,accept", [(248320, 3, 2), (5000, 3, 0), (1000, 1, 1), (777, 0, 0), (4096, 5, 5)])
def test_lm_head_greedy_bitwise(n, depth, accept):
    print(f"[lm_head greedy] n={n} depth={depth}", flush=True)
    k = 2560
    w = make_weight(n, k, 11 + n)
    x = torch.randn((depth + 1, k), generator=torch.Generator().manual_seed(n)).to(torch.bfloat16).cuda()
    logits = gemv(x, w).to(torch.bfloat16).float()  # lin's result for a bf16 x
    am = logits.argmax(dim=1).to(torch.int32).cpu()
    drafts = torch.tensor([int(am[i]) if i < accept else (int(am[i]) + 1) % n for i in range(depth)], dtype=torch.int32)
    head = LMHeadGreedy(w, depth)
    lg = torch.empty_like(logits)
    res = head(x, drafts.cuda(), logits=lg)
    assert torch.equal(lg, logits)
    want = O.accept_greedy(logits.cpu().numpy(), drafts.numpy())
    assert [res.n_accept, res.n_emit, res.n_uniform, res.flags] == want[:4].tolist()
    assert res.tokens == want[4: 4 + want[1]].tolist()
    assert res.n_accept == min(accept, depth)
    res2 = head(x, drafts.cuda())  # logits not written: same round
    assert (res2.n_accept, res2.tokens) == (res.n_accept, res.tokens)


def test_lm_head_greedy_nonfinite_row():
    n, k, depth = 3000, 2560, 3
    w = make_weight(n, k, 9)
    x = torch.randn((depth + 1, k), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    x[2, 100] = float("nan")
    logits = gemv(x, w).to(torch.bfloat16).float()
    drafts = logits.argmax(dim=1).to(torch.int32)[:depth].contiguous()
    res = LMHeadGreedy(w, depth)(x, drafts)
    want = O.accept_greedy(logits.cpu().numpy(), drafts.cpu().numpy())
    assert [res.n_accept, res.n_emit, res.flags] == [2, 2, 1] == [int(want[0]), int(want[1]), int(want[3])]
