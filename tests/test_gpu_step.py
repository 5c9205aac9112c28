"""The whole verify round in one HIP graph (engine/step.py, MTPStepGraph) on the GPU: the residual + RMSNorm kernel
against or_residual_rmsnorm bit for bit; graph replays equal to the eager launches on every replay, with eager
work between replays; each layer of the chain against the oracle on that layer's own input (router ids and weights
bit for bit, y within the north-star bound, the stream and the next norm bit for bit); the fused greedy round equal
to or_accept_greedy on the kept logits; the head MoE equal to a separate verify call of map layer NL."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.engine.step import MoEWeights, MTPStepGraph, residual_rmsnorm
from slotstream_spark_amd.engine.verify import MoEVerifyChain, MoEVerifyLayer
from slotstream_spark_amd.kernels.gemv_affine import AffineWeight, gemv
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias
from tests.gpu_util import DenseCache, bits, make_pool

pytestmark = pytest.mark.gpu

REL_Y = 2e-2
H, I, E, K, NL, V = 2048, 512, 64, 4, 3, 12_352


def _dev_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


@pytest.mark.parametrize("r,h,with_y,with_w,inplace", [(1, 2048, True, False, False), (4, 2048, True, True, False),
                                                       (3, 2560, False, True, False), (5, 520, True, True, True),
                                                       (9, 8, True, False, False), (2, 4096, False, False, False)])
def test_residual_rmsnorm_bitwise(r, h, with_y, with_w, inplace):
    print(f"[norm] R={r} H={h} y={with_y} w={with_w} inplace={inplace}", flush=True)
    rng = np.random.default_rng(r * 1000 + h)
    x = O.f32_to_bf16(rng.standard_normal((r, h)).astype(np.float32) * 3)
    y = O.f32_to_bf16(rng.standard_normal((r, h)).astype(np.float32)) if with_y else None
    w = O.f32_to_bf16(1 + 0.1 * rng.standard_normal(h).astype(np.float32)) if with_w else None
    eps = 1e-6 if h > 8 else 0.5
    so_ref, mx_ref = O.residual_rmsnorm(x, y, w, eps)
    xt = _dev_bits(x)
    so = xt if inplace else torch.empty_like(xt)
    mx = torch.empty_like(xt)
    residual_rmsnorm(xt, None if y is None else _dev_bits(y), mx, stream_out=so if with_y else None,
                     weight=None if w is None else _dev_bits(w), eps=eps)
    torch.cuda.synchronize()
    assert np.array_equal(bits(mx), mx_ref)
    if with_y:
        assert np.array_equal(bits(so), so_ref)


@pytest.fixture(scope="module")
def step():
    print(f"[step] {NL} layers + head, E={E} K={K}, lm_head {V} x {H}", flush=True)
    pool = make_pool(E, H, I, seed=404, layers=NL + 1)
    lws = [LayerWeights(H, E, 512, seed=410 + l) for l in range(NL + 1)]
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(E, 1.1, 420 + l))
          for l, w in enumerate(lws)]
    g = torch.Generator(device="cuda").manual_seed(430)
    q = torch.randint(-2**31, 2**31 - 1, (V, H // 8), generator=g, device="cuda", dtype=torch.int32)
    sc = (torch.randn((V, H // 64), generator=g, device="cuda") * 0.02).abs().to(torch.bfloat16)
    lm = AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, V, H)
    norms = [None] + [normal_bf16((H,), 0.1, 440 + l) + 1 for l in range(NL)]
    sg = MTPStepGraph(pool, mw[:NL], lm, depth=3, head=mw[NL], norm_weights=norms, top_k=K, keep_logits=True)
    return pool, mw, lm, norms, sg


@pytest.fixture(scope="module")
def step_unfused(step):
    pool, mw, lm, norms, _ = step
    return MTPStepGraph(pool, mw[:NL], lm, depth=3, head=mw[NL], norm_weights=norms, top_k=K, keep_logits=True,
                        fused=False)


def _snapshot(sg):
    keep = [sg.out, sg.logits, sg.head_y, sg.head_ids, sg.ids, sg.weights, sg.mixed[NL]] + sg.streams[1:] + sg.ys
    return [t.clone() for t in keep]


def test_fused_chain_equals_separate_norm_launches(step, step_unfused):
    """ssmoe_moe_verify_layer_chain (norm staged inside the verify launch, residual add in its combine) gives the
    same bits as ssmoe_residual_rmsnorm + ssmoe_moe_verify_layer."""
    _, _, _, _, sg = step
    x = normal_bf16((4, H), 1.0, 455)
    d = torch.tensor([3, 30, 300], dtype=torch.int32, device="cuda")
    for g in (sg, step_unfused):
        g.step(x, d)
        torch.cuda.synchronize()
    for n, (u, v) in enumerate(zip(_snapshot(sg), _snapshot(step_unfused))):
        assert torch.equal(u, v), n
    for l in range(NL + 1):   # the unfused graph wrote every norm: the fused launch staged the same inputs
        want = O.residual_rmsnorm(bits(sg.streams[l]), None, None if step[3][l] is None else bits(step[3][l]))[1]
        assert np.array_equal(bits(step_unfused.mixed[l]), want), l


def test_graph_replays_equal_eager(step):
    _, _, _, _, sg = step
    x1, x2 = normal_bf16((4, H), 1.0, 450), normal_bf16((4, H), 1.0, 451)
    d1 = torch.tensor([5, 77, 4000], dtype=torch.int32, device="cuda")
    d2 = torch.tensor([1, 2, 3], dtype=torch.int32, device="cuda")
    ref = {}
    for key, (x, d) in {"a": (x1, d1), "b": (x2, d2)}.items():
        sg.x_in.copy_(x)
        sg.drafts.copy_(d)
        sg.run_eager()
        torch.cuda.synchronize()
        ref[key] = _snapshot(sg)
    assert not torch.equal(ref["a"][1], ref["b"][1])
    for i, key in enumerate(["a", "b", "a", "a", "b"]):
        x, d = (x1, d1) if key == "a" else (x2, d2)
        sg.step(x, d)
        torch.cuda.synchronize()
        got = _snapshot(sg)
        for n, (u, v) in enumerate(zip(got, ref[key])):
            assert torch.equal(u, v), (i, key, n)
        torch.randn(1000, device="cuda").sum().item()     # eager work and a sync between replays


def test_chain_against_oracle_layer_by_layer(step):
    pool, mw, lm, norms, sg = step
    sg.step(normal_bf16((4, H), 1.0, 452), torch.tensor([9, 99, 999], dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    for l in range(NL):
        # the layer's input: the norm of its residual stream (staged inside the fused launch, recomputed here)
        xb = O.residual_rmsnorm(bits(sg.streams[l]), None, None if norms[l] is None else bits(norms[l]))[1]
        w = mw[l]
        _, _, rids, rw = O.router(xb, bits(w.router_w), K, w.router_bias.cpu().numpy())
        assert np.array_equal(sg.ids[l].cpu().numpy(), rids), l
        assert np.array_equal(sg.weights[l].cpu().numpy().view(np.uint32), rw.view(np.uint32)), l
        routed = O.moe_routed_fp64(O.bf16_to_f32(xb), rids, rw, DenseCache(pool, layer=l)).astype(np.float32)
        sh, sgl = O.shared_expert(xb, bits(w.sh_gate), bits(w.sh_up), bits(w.sh_down), bits(w.sh_g))
        ry = O.combine_shared(routed, sh, sgl)
        assert O.rel_l2(O.bf16_to_f32(bits(sg.ys[l])), O.bf16_to_f32(ry)) <= REL_Y, l
        so, mx = O.residual_rmsnorm(bits(sg.streams[l]), bits(sg.ys[l]), bits(norms[l + 1]))
        assert np.array_equal(bits(sg.streams[l + 1]), so), l
    assert np.array_equal(bits(sg.mixed[NL]), mx)
    # the chain keeps its scale: every mixed row has unit RMS up to the norm weights
    rms = O.bf16_to_f32(bits(sg.mixed[NL])).astype(np.float64)
    assert np.all(np.abs(np.sqrt((rms ** 2).mean(axis=1)) - 1.0) < 0.1)


def test_round_acceptance_and_logits(step):
    pool, mw, lm, norms, sg = step
    x = normal_bf16((4, H), 1.0, 453)
    sg.step(x, torch.zeros(3, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    logits = sg.logits.cpu().numpy()
    greedy = logits.argmax(axis=1).astype(np.int32)
    for drafts in ([greedy[0], greedy[1], greedy[2]], [greedy[0], greedy[1] ^ 1, 7], [greedy[0] ^ 1, 0, 0]):
        d = torch.tensor(drafts, dtype=torch.int32, device="cuda")
        out = sg.step(x, d)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), O.accept_greedy(logits, np.array(drafts, np.int32))), drafts
        assert torch.equal(sg.logits.cpu(), torch.from_numpy(logits))
    # The round ranks lin's result: the fp32 GEMV of the final norm rounded to bf16.
    raw = gemv(sg.mixed[NL], lm)
    assert torch.equal(sg.logits, raw.to(torch.bfloat16).float())
    xm = O.bf16_to_f32(bits(sg.mixed[NL]))
    y64, bound = O.gemv_affine4_fp64(xm, lm.q.cpu().numpy(), bits(lm.s), bits(lm.b))
    assert np.max(np.abs(raw.cpu().numpy() - y64) / bound) <= 2e-5
    res = sg.result()
    assert res.n_accept == 0 and res.n_emit == 1


def test_head_moe_is_map_layer_nl(step):
    pool, mw, lm, norms, sg = step
    from slotstream_spark_amd.engine.verify import MoEVerifyLayer
    sg.step(normal_bf16((4, H), 1.0, 454), torch.zeros(3, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    w = mw[NL]
    sep = MoEVerifyLayer(pool, NL, w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, top_k=K, router_bias=w.router_bias)
    y, ids, wt = sep(sg.mixed[NL].clone())
    torch.cuda.synchronize()
    assert torch.equal(y, sg.head_y) and torch.equal(ids, sg.head_ids) and torch.equal(wt, sg.head_weights)
    _, _, rids, _ = O.router(bits(sg.mixed[NL]), bits(w.router_w), K, w.router_bias.cpu().numpy())
    assert np.array_equal(sg.head_ids.cpu().numpy(), rids)


@pytest.mark.parametrize("T,NL4", [(2, 4), (3, 3), (4, 3)])
def test_chain_at_config4_layer_shape(T, NL4):
    """BASELINE config 4's layer (E=512, top-10, Zipf bias, I 512, shared 512) chained, T = 2 (config 4), T = 3 (the
    reference's verify width, 1 + DEPTH rows: engine/mtp.py:48, runtime/graphs.py:95-96) and T = 4 (config 2's rows),
    replayed twice with different inputs: the single launch of every layer
    (ssmoe_moe_verify_chain) equals one launch per layer bit for bit, and each layer matches the oracle on its own
    input (ids and weights bit for bit, y within the north-star bound, the stream and the final norm bit for bit)."""
    E4, K4 = 512, 10
    print(f"[chain config4] {NL4} layers, E={E4} K={K4} T={T}", flush=True)
    pool = make_pool(E4, H, I, seed=505, layers=NL4)
    lws = [LayerWeights(H, E4, 512, seed=510 + l) for l in range(NL4)]
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(E4, 1.1, 520 + l))
          for l, w in enumerate(lws)]
    norms = [normal_bf16((H,), 0.1, 530 + l) + 1 for l in range(NL4 + 1)]
    sg = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K4)
    per_layer = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K4, single_launch=False)
    assert sg.chain is not None
    for trial in range(2):
        x = normal_bf16((T, H), 1.0, 540 + trial)
        per_layer.step(x)
        sg.step(x)
        torch.cuda.synchronize()
        for l in range(NL4):     # one launch for the chain = one launch per layer, bit for bit
            assert torch.equal(sg.ids[l], per_layer.ids[l]) and torch.equal(sg.weights[l], per_layer.weights[l])
            assert torch.equal(sg.ys[l], per_layer.ys[l]) and torch.equal(sg.streams[l + 1], per_layer.streams[l + 1])
        for l in range(NL4):
            xb = O.residual_rmsnorm(bits(sg.streams[l]), None, bits(norms[l]))[1]
            w = mw[l]
            _, _, rids, rw = O.router(xb, bits(w.router_w), K4, w.router_bias.cpu().numpy())
            assert np.array_equal(sg.ids[l].cpu().numpy(), rids), (trial, l)
            assert np.array_equal(sg.weights[l].cpu().numpy().view(np.uint32), rw.view(np.uint32)), (trial, l)
            routed = O.moe_routed_fp64(O.bf16_to_f32(xb), rids, rw, DenseCache(pool, layer=l)).astype(np.float32)
            sh, sgl = O.shared_expert(xb, bits(w.sh_gate), bits(w.sh_up), bits(w.sh_down), bits(w.sh_g))
            ry = O.combine_shared(routed, sh, sgl)
            err = O.rel_l2(O.bf16_to_f32(bits(sg.ys[l])), O.bf16_to_f32(ry))
            assert err <= REL_Y, (trial, l, err)
            so, mx = O.residual_rmsnorm(bits(sg.streams[l]), bits(sg.ys[l]), bits(norms[l + 1]))
            assert np.array_equal(bits(sg.streams[l + 1]), so), (trial, l)
        assert np.array_equal(bits(sg.mixed[NL4]), mx)
        print(f"trial {trial}: unique experts per layer "
              f"{[len(set(sg.ids[l].cpu().flatten().tolist())) for l in range(NL4)]}", flush=True)


def test_chain_one_row_equals_per_layer_launches():
    """The chain launch at T = 1 (MoEVerifyChain directly: a step graph always verifies at least two rows), where the
    dense rows' token pairs and the two-token item paths run with an absent token: three E 512 / top-10 layers in one
    launch equal one ssmoe_moe_verify_layer_chain launch per layer bit for bit, and layer 0 routes as the oracle."""
    E4, K4, NL = 512, 10, 3
    print(f"[chain T=1] {NL} layers, E={E4} K={K4}", flush=True)
    pool = make_pool(E4, H, I, seed=705, layers=NL)
    lws = [LayerWeights(H, E4, 512, seed=710 + l) for l in range(NL)]
    layers = [MoEVerifyLayer(pool, l, w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, top_k=K4,
                             router_bias=zipf_bias(E4, 1.1, 720 + l)) for l, w in enumerate(lws)]
    if not MoEVerifyChain.supported(H, I, 512, K4, E4):
        pytest.skip("the chain needs E + Is >= 4 x CUs and H / 16 < CUs")
    norms = [normal_bf16((H,), 0.1, 730 + l) + 1 for l in range(NL)]
    dev = pool.device

    def bufs():
        return ([torch.empty((1, H), dtype=torch.bfloat16, device=dev) for _ in range(NL)],
                [torch.empty((1, K4), dtype=torch.int32, device=dev) for _ in range(NL)],
                [torch.empty((1, K4), dtype=torch.float32, device=dev) for _ in range(NL)],
                [torch.empty((1, H), dtype=torch.bfloat16, device=dev) for _ in range(NL)])

    ys, ids, ws, so = bufs()
    chain = MoEVerifyChain(layers, ys, ids, ws, stream_outs=so, norm_weights=norms)
    for trial in range(2):
        x = normal_bf16((1, H), 1.0, 740 + trial).to(dev)
        chain.run(x)
        ys1, ids1, ws1, so1 = bufs()
        s = x
        for l in range(NL):
            layers[l].chain(s, ys1[l], ids1[l], ws1[l], stream_out=so1[l], norm_weight=norms[l])
            s = so1[l]
        torch.cuda.synchronize()
        for l in range(NL):
            assert torch.equal(ids[l], ids1[l]) and torch.equal(ws[l], ws1[l]), (trial, l)
            assert torch.equal(ys[l], ys1[l]) and torch.equal(so[l], so1[l]), (trial, l)
        xb = O.residual_rmsnorm(bits(x), None, bits(norms[0]))[1]
        _, _, rids, rw = O.router(xb, bits(lws[0].router_w), K4, layers[0].router_bias.cpu().numpy())
        assert np.array_equal(ids[0].cpu().numpy(), rids)
        assert np.array_equal(ws[0].cpu().numpy().view(np.uint32), rw.view(np.uint32))


@pytest.mark.parametrize("T", [2, 3])
def test_chain_of_16_layers_equals_per_layer_launches(T):
    """The chain as the bench times it: 16 distinct config-1 layers (E 512, top-10, Zipf bias) in one launch, three
    replays with new inputs, every layer's ids, weights, y and stream equal to one launch per layer bit for bit, and
    the last layer against the oracle on its own input."""
    E4, K4, NL16 = 512, 10, 16
    print(f"[chain 16] {NL16} layers, E={E4} K={K4} T={T}", flush=True)
    pool = make_pool(E4, H, I, seed=605, layers=NL16)
    lws = [LayerWeights(H, E4, 512, seed=610 + l) for l in range(NL16)]
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(E4, 1.1, 640 + l))
          for l, w in enumerate(lws)]
    norms = [normal_bf16((H,), 0.1, 660 + l) + 1 for l in range(NL16 + 1)]
    sg = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K4)
    per_layer = MTPStepGraph(pool, mw, None, depth=T - 1, norm_weights=norms, top_k=K4, single_launch=False)
    assert sg.chain is not None
    for trial in range(3):
        x = normal_bf16((T, H), 1.0, 680 + trial)
        per_layer.step(x)
        sg.step(x)
        torch.cuda.synchronize()
        for l in range(NL16):
            assert torch.equal(sg.ids[l], per_layer.ids[l]) and torch.equal(sg.weights[l], per_layer.weights[l]), \
                (trial, l)
            assert torch.equal(sg.ys[l], per_layer.ys[l]) and torch.equal(sg.streams[l + 1], per_layer.streams[l + 1]), \
                (trial, l)
    l = NL16 - 1
    xb = O.residual_rmsnorm(bits(sg.streams[l]), None, bits(norms[l]))[1]
    w = mw[l]
    _, _, rids, rw = O.router(xb, bits(w.router_w), K4, w.router_bias.cpu().numpy())
    assert np.array_equal(sg.ids[l].cpu().numpy(), rids)
    assert np.array_equal(sg.weights[l].cpu().numpy().view(np.uint32), rw.view(np.uint32))
    routed = O.moe_routed_fp64(O.bf16_to_f32(xb), rids, rw, DenseCache(pool, layer=l)).astype(np.float32)
    sh, sgl = O.shared_expert(xb, bits(w.sh_gate), bits(w.sh_up), bits(w.sh_down), bits(w.sh_g))
    err = O.rel_l2(O.bf16_to_f32(bits(sg.ys[l])), O.bf16_to_f32(O.combine_shared(routed, sh, sgl)))
    assert err <= REL_Y, err
    del pool, sg, per_layer
    torch.cuda.empty_cache()


def test_pq_round_in_the_step_graph(step):
    """The round with p/q acceptance fused behind the lm_head (accept="pq"), drafts drawn from q by draw_drafts (the
    proposal the rule needs): the drafts equal the sampler's definition, the logits are the greedy graph's on the
    same rows, and every replay's result equals ssmoe_accept_pq on those logits."""
    from slotstream_spark_amd.engine.accept import Acceptor

    pool, mw, lm, norms, sg = step
    pq = MTPStepGraph(pool, mw[:NL], lm, depth=3, norm_weights=norms, top_k=K, accept="pq", temperature=0.7)
    g = torch.Generator(device="cuda").manual_seed(461)
    acc = Acceptor(3, V)
    for rep in range(3):
        x = normal_bf16((4, H), 1.0, 470 + rep)
        sg.step(x, torch.zeros(3, dtype=torch.int32, device="cuda"))
        torch.cuda.synchronize()
        pq.draft_logits.copy_(0.8 * sg.logits[:3] + torch.randn((3, V), generator=g, device="cuda") * 1.8)
        pq.uniforms.copy_(torch.rand(4, generator=g, device="cuda"))
        ud = torch.rand(3, generator=g, device="cuda")
        drafts = pq.draw_drafts(ud).clone()
        ql, un = pq.draft_logits.cpu().numpy(), ud.cpu().numpy()
        assert drafts.cpu().tolist() == O.draw_rows(ql, 0.7, un).tolist()
        out = pq.step(x, drafts).clone()
        torch.cuda.synchronize()
        assert torch.equal(pq.logits, sg.logits), rep
        want = acc.pq_async(sg.logits, pq.draft_logits, drafts, pq.uniforms, 0.7)
        torch.cuda.synchronize()
        assert torch.equal(out, want), (rep, out.cpu().tolist(), want.cpu().tolist())
