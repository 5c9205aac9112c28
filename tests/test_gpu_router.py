"""Router, dense bf16 projection and topk_stable on the GPU, bit for bit against the CPU restatement."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.kernels.router import lin_bf16, route
from slotstream_spark_amd.kernels.topk_stable import topk_stable
from slotstream_spark_amd.memory.synth import normal_bf16, zipf_bias
from tests.gpu_util import bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("t,h,n", [(2, 2048, 512), (4, 2048, 1025), (3, 2560, 64), (1, 8, 3), (5, 1000, 7)])
def test_dense_rows_bitexact(t, h, n):
    x = normal_bf16((t, h), 1.0, 100 + n)
    w = normal_bf16((n, h), 0.02, 200 + n)
    out = lin_bf16(x, w)
    torch.cuda.synchronize()
    ref = O.dense_rows(bits(x), bits(w))
    assert np.array_equal(bits(out), ref)


@pytest.mark.parametrize("use_bias", [False, True])
@pytest.mark.parametrize("t,e,k", [(2, 512, 10), (4, 512, 10), (2, 64, 4), (3, 128, 16)])
def test_router_bitexact(t, e, k, use_bias):
    x = normal_bf16((t, 2048), 1.0, 300 + e + t)
    w = normal_bf16((e, 2048), 0.02, 400 + e)
    bias = zipf_bias(e, 1.1, 1731) if use_bias else None
    logits = torch.empty((t, e), dtype=torch.bfloat16, device="cuda")
    probs = torch.empty((t, e), dtype=torch.float32, device="cuda")
    ids, wts = route(x, w, k, bias, logits=logits, probs=probs)
    torch.cuda.synchronize()
    rl, rp, ri, rw = O.router(bits(x), bits(w), k, None if bias is None else bias.cpu().numpy())
    assert np.array_equal(bits(logits), rl)
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), rp.view(np.uint32))
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), rw.view(np.uint32))


def test_router_ties_take_lower_index():
    # Quantised router rows: many exactly equal logits and probabilities.
    t, e, k = 3, 512, 10
    x = torch.ones((t, 2048), dtype=torch.bfloat16, device="cuda")
    g = torch.Generator().manual_seed(5)
    w = (torch.randint(0, 3, (e, 2048), generator=g).float() * 0.001).to(torch.bfloat16).cuda()
    ids, wts = route(x, w, k)
    torch.cuda.synchronize()
    _, _, ri, rw = O.router(bits(x), bits(w), k)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), rw.view(np.uint32))


def _rand(r, n, seed, levels=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(r, n, generator=g)
    if levels:
        x = torch.round(x * levels) / levels
    return x


def _check_topk(x, k, n_valid=None):
    xc = x.contiguous().cuda()
    nv = None if n_valid is None else torch.tensor(n_valid, dtype=torch.int32, device="cuda")
    out_val = torch.empty((x.shape[0], k), dtype=torch.float32, device="cuda")
    idx, val = topk_stable(xc, k, nv, out_val=out_val)
    torch.cuda.synchronize()
    ri, rv = O.topk_stable(x.numpy(), k, n_valid)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.array_equal(val.cpu().numpy().view(np.uint32), rv.view(np.uint32))
    return idx


@pytest.mark.parametrize("n", [512, 513, 2048, 8192, 65536])
@pytest.mark.parametrize("k", [10, 512])
def test_topk_random_and_ties(n, k):
    _check_topk(_rand(3, n, n + k), k)
    _check_topk(_rand(3, n, n * 3 + k, levels=2), k)


def test_topk_all_equal_lowest_indices():
    idx = _check_topk(torch.full((2, 1000), 1.5), 10)
    assert idx[0].cpu().tolist() == list(range(10))


def test_topk_special_values():
    x = _rand(4, 512, 1)
    x[0, :20] = float("nan")
    x[1, 5:15] = float("-inf")
    x[1, 100:104] = float("inf")
    x[2, :] = 0.0
    x[2, ::3] = -0.0
    x[3, 7] = float("nan")
    _check_topk(x, 10)
    _check_topk(x, 40)


def test_topk_n_valid():
    x = _rand(4, 700, 3)
    _check_topk(x, 10, [700, 5, 0, 333])
    _check_topk(x, 100, [700, 50, 99, 1])
