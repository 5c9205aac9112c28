"""or_residual_rmsnorm (the residual add + RMSNorm between chained layers) against what the mathematics and torch
fix: known answers, torch's own bf16 add, scale and weight invariances, and the reference's rmsnorm formula
(model/reference_torch.py:30-38) in torch within one bf16 ulp."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def _bf(a):
    return O.f32_to_bf16(np.asarray(a, np.float32))


def _rows(r, h, seed, scale=1.0):
    return _bf(np.random.default_rng(seed).standard_normal((r, h)).astype(np.float32) * scale)


def test_constant_power_of_two_row_normalises_to_plus_minus_one():
    x = _bf(np.array([[4.0] * 512, [-0.25] * 512], np.float32))
    _, m = O.residual_rmsnorm(x, eps=0.0)
    assert (O.bf16_to_f32(m[0]) == 1.0).all() and (O.bf16_to_f32(m[1]) == -1.0).all()


def test_stream_is_torchs_bf16_add():
    a, b = _rows(3, 2048, 1), _rows(3, 2048, 2, 7.0)
    s, _ = O.residual_rmsnorm(a, b)
    ta = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    assert np.array_equal(s, (ta + tb).view(torch.int16).numpy().view(np.uint16))
    s0, _ = O.residual_rmsnorm(a)
    assert np.array_equal(s0, a)


def test_power_of_two_scale_and_weight_invariance():
    x = _rows(4, 2560, 3)
    _, m = O.residual_rmsnorm(x, eps=0.0)
    _, m8 = O.residual_rmsnorm(_bf(O.bf16_to_f32(x) * 8.0), eps=0.0)
    assert np.array_equal(m, m8)
    _, m2 = O.residual_rmsnorm(x, w_bits=_bf(np.full(2560, 2.0, np.float32)), eps=0.0)
    assert np.array_equal(O.bf16_to_f32(m2), 2.0 * O.bf16_to_f32(m))


@pytest.mark.parametrize("eps", [1e-6, 1e-2])
def test_reference_formula_in_torch_within_one_ulp(eps):
    x, y = _rows(5, 2048, 4), _rows(5, 2048, 5, 0.5)
    w = _bf(1.0 + 0.1 * np.random.default_rng(6).standard_normal(2048).astype(np.float32))
    s, m = O.residual_rmsnorm(x, y, w, eps)
    ts = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
    tw = torch.from_numpy(w.view(np.int16)).view(torch.bfloat16)
    xf = ts.float()                                    # reference_torch.rmsnorm, verbatim semantics
    ref = ((xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) * tw.float()).to(torch.bfloat16)
    got = torch.from_numpy(m.view(np.int16)).view(torch.bfloat16)
    diff = (got.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert diff.max().item() <= 1 and (diff == 0).float().mean().item() > 0.98
    # a plausible slip, eps outside the square root, is caught at the larger eps
    if eps > 1e-3:
        slip = ((xf / (xf.pow(2).mean(-1, keepdim=True).sqrt() + eps)) * tw.float()).to(torch.bfloat16)
        assert (got.view(torch.int16) != slip.view(torch.int16)).float().mean().item() > 0.2
