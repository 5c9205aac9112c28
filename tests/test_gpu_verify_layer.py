"""The fused MoE verify layer (router + routed experts + shared expert) on the GPU at BASELINE configs 0 and 1,
against the oracle: router ids and weights bit for bit, y within the north-star bound (2e-2 relative on bf16),
and against the torch CPU restatement of the reference's moe_ref."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.engine.verify import MoEVerifyLayer
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias
from tests.gpu_util import DenseCache, bits, make_pool

pytestmark = pytest.mark.gpu

REL_Y = 2e-2      # MoE outputs within 2e-2 relative on bf16


def _layer(experts, k, seed, bias):
    pool = make_pool(experts, 2048, 512, seed=seed)
    lw = LayerWeights(2048, experts, 512, seed=seed)
    b = zipf_bias(experts, 1.1, 1731) if bias else None
    return pool, lw, MoEVerifyLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=k,
                                    router_bias=b), b


def _oracle_y(pool, lw, x, k, bias):
    xb = bits(x)
    _, _, ids, w = O.router(xb, bits(lw.router_w), k, None if bias is None else bias.cpu().numpy())
    routed = O.moe_routed_fp64(O.bf16_to_f32(xb), ids, w, DenseCache(pool)).astype(np.float32)
    sh, sgl = O.shared_expert(xb, bits(lw.sh_gate), bits(lw.sh_up), bits(lw.sh_down), bits(lw.sh_g))
    return ids, w, routed, O.combine_shared(routed, sh, sgl)


@pytest.mark.parametrize("experts,k,bias,t", [(64, 4, False, 2), (512, 10, True, 2), (512, 10, True, 3),
                                             (512, 10, True, 4), (512, 10, False, 1)])
def test_verify_layer_vs_oracle(experts, k, bias, t):
    print(f"[verify] E={experts} K={k} bias={bias} T={t}", flush=True)
    pool, lw, layer, b = _layer(experts, k, 1729 + experts, bias)
    x = normal_bf16((t, 2048), 1.0, 1730 + t)
    routed = torch.empty((t, 2048), dtype=torch.float32, device="cuda")
    y, ids, w = layer(x, routed=routed)
    torch.cuda.synchronize()
    rids, rw, rrouted, ry = _oracle_y(pool, lw, x, k, b)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    err_r = O.rel_l2(routed.cpu().numpy(), rrouted)
    err_y = O.rel_l2(O.bf16_to_f32(bits(y)), O.bf16_to_f32(ry))
    same = float(np.mean(bits(y) == ry))
    print(f"routed rel_l2 {err_r:.3e}; y rel_l2 {err_y:.3e}; y bf16 bits equal {same:.4f}")
    assert err_r <= 1e-4
    assert err_y <= REL_Y


def test_verify_layer_extreme_router_logits():
    """Router logits spread over about +-130 (router weights x 50): in every token's row some probabilities fall in
    (0, 2^-64), where the kernel's softmax quotient takes the IEEE division instead of its one-division form, and
    many underflow to 0; ids and weights bit for bit against the oracle."""
    print("[verify] extreme router logits", flush=True)
    pool = make_pool(512, 2048, 512, seed=2201)
    lw = LayerWeights(2048, 512, 512, seed=2201)
    router_w = (lw.router_w.float() * 50.0).to(torch.bfloat16)
    layer = MoEVerifyLayer(pool, 0, router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=10)
    x = normal_bf16((2, 2048), 1.0, 2202)
    y, ids, w = layer(x)
    torch.cuda.synchronize()
    _, probs, rids, rw = O.router(bits(x), bits(router_w), 10)
    assert ((probs > 0) & (probs < 2.0 ** -64)).any(axis=1).all()
    assert (probs == 0).any(axis=1).all()
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))


def test_verify_layer_vs_torch_moe_ref():
    """Against the torch CPU restatement of reference_torch.moe_ref (config 0 shape, no bias)."""
    pool, lw, layer, _ = _layer(64, 4, 99, False)
    x = normal_bf16((2, 2048), 1.0, 5)
    y, ids, w = layer(x)
    torch.cuda.synchronize()
    dense = DenseCache(pool)

    def expert(e):
        return tuple(torch.from_numpy(d.astype(np.float32)) for d in dense(e))

    yr, ti, tv = O.moe_ref(x.cpu(), lw.router_w.cpu(), 4, expert, lw.sh_gate.cpu(), lw.sh_up.cpu(),
                           lw.sh_down.cpu(), lw.sh_g.cpu())
    assert np.array_equal(ids.cpu().numpy(), ti.numpy().astype(np.int32))
    err = O.rel_l2(y.float().cpu().numpy(), yr.float().numpy())
    print(f"y vs torch moe_ref rel_l2 {err:.3e}")
    assert err <= REL_Y


def test_verify_rows_independent():
    """A 2-token call equals two 1-token calls bit for bit (graphs.py 3-row == 3 x 1-row, tests/gates/test_h3.py)."""
    _, _, layer, _ = _layer(512, 10, 7, True)
    x = normal_bf16((2, 2048), 1.0, 8)
    y2, i2, w2 = layer(x)
    for t in range(2):
        y1, i1, w1 = layer(x[t:t + 1].contiguous())
        assert torch.equal(y1[0], y2[t]) and torch.equal(i1[0], i2[t]) and torch.equal(w1[0], w2[t])


def test_verify_router_ties_and_non_finite_fallback():
    """The verify kernel's router tail selects the top K by a threshold when at most 64 entries reach it and by K
    rounds otherwise; both must give the oracle's ids and weights bit for bit. Router columns 0 and 1 hold a few
    quantised values, so token 0 (x = e0: three distinct logits, about 170 tied at the top) takes the rounds,
    token 1 (x = e0 + e1: ten distinct logits, a tie group inside the top K) the threshold with ties, token 2 (a
    non-finite element: NaN probabilities) the rounds, token 3 (random x) the threshold. The path of each token is
    the one the numpy emulation of the selection (tests/test_oracle_pins.py) takes on the oracle's probabilities."""
    from tests.test_oracle_pins import _threshold_select

    E, K, H = 512, 10, 2048
    pool = make_pool(E, H, 512, seed=61)
    lw = LayerWeights(H, E, 512, seed=61)
    rng = np.random.default_rng(63)
    rw = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    rw[:, 0] = rng.integers(0, 3, E) / 128
    rw[:, 1] = rng.integers(0, 8, E) / 128
    x = np.zeros((4, H), np.float32)
    x[0, 0] = 1
    x[1, :2] = 1
    x[2, :] = 1
    x[2, 5] = np.inf
    x[3] = rng.standard_normal(H)
    rwb, xb = O.f32_to_bf16(rw), O.f32_to_bf16(x)
    _, probs, rids, rwt = O.router(xb, rwb, K)
    paths = [_threshold_select(probs[t], K) is not None for t in range(4)]
    assert paths == [False, True, False, True]
    assert len(np.unique(probs[1][rids[1]])) < K                 # ties inside token 1's top K
    dev = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()  # noqa: E731
    layer = MoEVerifyLayer(pool, 0, dev(rwb), lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K)
    xt = dev(xb)
    y, ids, w = layer(xt)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), rids)
    got = w.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(rwt))
    assert np.array_equal(np.nan_to_num(got).view(np.uint32), np.nan_to_num(rwt).view(np.uint32))
    # the finite tokens' layer outputs are the oracle's
    keep = [0, 1, 3]
    routed = O.moe_routed_fp64(O.bf16_to_f32(xb[keep]), rids[keep], rwt[keep], DenseCache(pool)).astype(np.float32)
    sh, sgl = O.shared_expert(xb[keep], bits(lw.sh_gate), bits(lw.sh_up), bits(lw.sh_down), bits(lw.sh_g))
    ry = O.combine_shared(routed, sh, sgl)
    assert O.rel_l2(O.bf16_to_f32(bits(y)[keep]), O.bf16_to_f32(ry)) <= REL_Y
