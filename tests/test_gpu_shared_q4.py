"""The MoE verify layer with the shared expert in the reference checkpoint's format: affine 4-bit (gs 64)
gate/up/down projections (model/weights.py:84-92, applied by lin -> gemv, model/layers.py:62-76, runtime/graphs.py:
165-167), the router and shared_expert_gate rows bf16, at the BASELINE layer (H 2048, I 512, Is 512) and at the
reference model's (H 2560, I 640, Is 640, config.py:8-21). Against the oracle: router ids and weights bit for bit,
the routed sum within 1e-4 of fp64, and the shared expert bit for bit (y equals or_combine_shared of the GPU's routed
sum and the oracle's q4 shared chain), y within the north-star bound; the chained launch equal to per-layer launches."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.engine.step import MoEWeights, MTPStepGraph
from slotstream_spark_amd.engine.verify import MoEVerifyLayer
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias
from tests.gpu_util import DenseCache, bits, make_pool

pytestmark = pytest.mark.gpu

REL_Y = 2e-2


def _q4(w):
    return (w.q.cpu().numpy().view(np.uint32), bits(w.s), bits(w.b))


def _check_layer(pool, lw, layer, x, y, ids, wts, routed, k, bias, map_layer=0):
    xb = bits(x)
    _, _, rids, rw = O.router(xb, bits(lw.router_w), k, None if bias is None else bias.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    r64 = O.moe_routed_fp64(O.bf16_to_f32(xb), rids, rw, DenseCache(pool, layer=map_layer)).astype(np.float32)
    err_r = O.rel_l2(routed.cpu().numpy(), r64)
    sh, sgl = O.shared_expert_q4(xb, _q4(lw.sh_gate), _q4(lw.sh_up), _q4(lw.sh_down), bits(lw.sh_g))
    y_exact = O.combine_shared(routed.cpu().numpy(), sh, sgl)   # the GPU's routed sum with the oracle's shared chain
    assert np.array_equal(bits(y), y_exact), float(np.mean(bits(y) != y_exact))
    err_y = O.rel_l2(O.bf16_to_f32(bits(y)), O.bf16_to_f32(O.combine_shared(r64, sh, sgl)))
    print(f"routed rel_l2 {err_r:.3e}; y rel_l2 {err_y:.3e}")
    assert err_r <= 1e-4 and err_y <= REL_Y


@pytest.mark.parametrize("H,I,E,K,bias,T", [(2048, 512, 64, 4, False, 2), (2048, 512, 512, 10, True, 1),
                                            (2048, 512, 512, 10, True, 2), (2048, 512, 512, 10, True, 3),
                                            (2048, 512, 512, 10, True, 4), (2560, 640, 512, 10, True, 3),
                                            (2560, 640, 512, 10, False, 1)])
def test_verify_layer_q4_shared_vs_oracle(H, I, E, K, bias, T):
    print(f"[q4 shared] H={H} I={I} E={E} K={K} bias={bias} T={T}", flush=True)
    pool = make_pool(E, H, I, seed=901 + H + E)
    lw = LayerWeights(H, E, I, seed=903 + E, shared_q4=True)
    b = zipf_bias(E, 1.1, 905) if bias else None
    layer = MoEVerifyLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K, router_bias=b)
    assert layer.sh_q4 is not None
    x = normal_bf16((T, H), 1.0, 907 + T)
    routed = torch.empty((T, H), dtype=torch.float32, device="cuda")
    y, ids, wts = layer(x, routed=routed)
    torch.cuda.synchronize()
    _check_layer(pool, lw, 0, x, y, ids, wts, routed, K, b)


def test_q4_shared_rows_are_call_independent():
    """A 3-token call equals three 1-token calls bit for bit with the q4 shared expert."""
    pool = make_pool(512, 2048, 512, seed=911)
    lw = LayerWeights(2048, 512, 512, seed=912, shared_q4=True)
    layer = MoEVerifyLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=10,
                           router_bias=zipf_bias(512, 1.1, 913))
    x = normal_bf16((3, 2048), 1.0, 914)
    y3, i3, w3 = layer(x)
    for t in range(3):
        y1, i1, w1 = layer(x[t:t + 1].contiguous())
        assert torch.equal(y1[0], y3[t]) and torch.equal(i1[0], i3[t]) and torch.equal(w1[0], w3[t])


@pytest.mark.parametrize("T", [2, 3])
def test_chain_with_q4_shared_expert(T):
    """Three chained config-1 layers with q4 shared experts: the single launch equals one launch per layer bit for
    bit, and each layer matches the oracle on its own input (shared expert bit for bit)."""
    H, I, E, K, NL = 2048, 512, 512, 10, 3
    print(f"[q4 chain] {NL} layers T={T}", flush=True)
    pool = make_pool(E, H, I, seed=921, layers=NL)
    lws = [LayerWeights(H, E, I, seed=922 + l, shared_q4=True) for l in range(NL)]
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(E, 1.1, 930 + l))
          for l, w in enumerate(lws)]
    norms = [normal_bf16((H,), 0.1, 940 + l) + 1 for l in range(NL + 1)]
    sg = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K)
    per_layer = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K, single_launch=False)
    assert sg.chain is not None
    for trial in range(2):
        x = normal_bf16((T, H), 1.0, 950 + trial)
        per_layer.step(x)
        sg.step(x)
        torch.cuda.synchronize()
        for l in range(NL):
            assert torch.equal(sg.ids[l], per_layer.ids[l]) and torch.equal(sg.weights[l], per_layer.weights[l])
            assert torch.equal(sg.ys[l], per_layer.ys[l]) and torch.equal(sg.streams[l + 1], per_layer.streams[l + 1])
    for l in range(NL):
        xb_bits = O.residual_rmsnorm(bits(sg.streams[l]), None, bits(norms[l]))[1]
        xb = torch.from_numpy(xb_bits.view(np.int16)).view(torch.bfloat16).cuda()
        layer = MoEVerifyLayer(pool, l, lws[l].router_w, lws[l].sh_gate, lws[l].sh_up, lws[l].sh_down, lws[l].sh_g,
                               top_k=K, router_bias=mw[l].router_bias)
        routed = torch.empty((T, H), dtype=torch.float32, device="cuda")
        y, ids, wts = layer(xb, routed=routed)
        torch.cuda.synchronize()
        assert torch.equal(y, sg.ys[l]) and torch.equal(ids, sg.ids[l]), l
        _check_layer(pool, lws[l], l, xb, y, ids, wts, routed, K, mw[l].router_bias, map_layer=l)


@pytest.mark.parametrize("T,q4", [(2, True), (3, True), (4, True), (3, False)])
def test_chain_at_the_reference_model_shape(T, q4):
    """The single-launch chain at the reference model's MoE layer (config.py:8-21: H 2560, 512 experts top-10,
    moe_intermediate 640, shared 640; the shared expert affine 4-bit as the checkpoint keeps it, or bf16): equal to
    one launch per layer bit for bit, each layer against the oracle on its own input."""
    H, I, E, K, NL = 2560, 640, 512, 10, 3
    print(f"[ref-shape chain] H={H} I={I} T={T} q4={q4}", flush=True)
    pool = make_pool(E, H, I, seed=961, layers=NL)
    lws = [LayerWeights(H, E, I, seed=962 + l, shared_q4=q4) for l in range(NL)]
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(E, 1.1, 970 + l))
          for l, w in enumerate(lws)]
    norms = [normal_bf16((H,), 0.1, 980 + l) + 1 for l in range(NL + 1)]
    sg = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K)
    per_layer = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K, single_launch=False)
    assert sg.chain is not None
    for trial in range(2):
        x = normal_bf16((T, H), 1.0, 990 + trial)
        per_layer.step(x)
        sg.step(x)
        torch.cuda.synchronize()
        for l in range(NL):
            assert torch.equal(sg.ids[l], per_layer.ids[l]) and torch.equal(sg.weights[l], per_layer.weights[l])
            assert torch.equal(sg.ys[l], per_layer.ys[l]) and torch.equal(sg.streams[l + 1], per_layer.streams[l + 1])
    for l in range(NL):
        xb_bits = O.residual_rmsnorm(bits(sg.streams[l]), None, bits(norms[l]))[1]
        w = lws[l]
        _, _, rids, rw = O.router(xb_bits, bits(w.router_w), K, mw[l].router_bias.cpu().numpy())
        assert np.array_equal(sg.ids[l].cpu().numpy(), rids), l
        assert np.array_equal(sg.weights[l].cpu().numpy().view(np.uint32), rw.view(np.uint32)), l
        r64 = O.moe_routed_fp64(O.bf16_to_f32(xb_bits), rids, rw, DenseCache(pool, layer=l)).astype(np.float32)
        if q4:
            sh, sgl = O.shared_expert_q4(xb_bits, _q4(w.sh_gate), _q4(w.sh_up), _q4(w.sh_down), bits(w.sh_g))
        else:
            sh, sgl = O.shared_expert(xb_bits, bits(w.sh_gate), bits(w.sh_up), bits(w.sh_down), bits(w.sh_g))
        err = O.rel_l2(O.bf16_to_f32(bits(sg.ys[l])), O.bf16_to_f32(O.combine_shared(r64, sh, sgl)))
        assert err <= REL_Y, (l, err)
