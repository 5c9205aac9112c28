"""The MoE-only MTP draft head (engine/mtp.py) on the GPU against its CPU restatement (oracle/mtp_head.py):

  * each dense op (rmsnorm, the GEMV with every epilogue, the hyper-connection mean and residual, the row gather)
    bit for bit, at the head's shapes and at ragged ones;
  * the lm_head argmax: the ids equal the first maximal index of the bf16-rounded logits the same launch wrote;
  * a 3-step draft chain teacher-forced against the oracle: every intermediate of step i recomputed on the CPU
    from the GPU's own inputs of that step (the dense part bit for bit; the MoE's router ids and weights bit for
    bit and y within the north-star bound), and the drafted token the argmax of that step's logits;
  * the captured draft graph equal to the eager chain on every replay, and consume/draft bookkeeping
    (engine/mtp.py:244-277).
"""
import numpy as np
import pytest
import torch

from oracle import mtp_head as MH
from oracle import oracle as O
from slotstream_spark_amd import _lib
from slotstream_spark_amd.engine.mtp import DraftGraph, MTPHead
from slotstream_spark_amd.engine.verify import MoEVerifyLayer
from slotstream_spark_amd.kernels import head_ops as HO
from slotstream_spark_amd.kernels.gemv_affine import AffineWeight, LMHeadArgmax, gemv
from slotstream_spark_amd.memory.synth import LayerWeights, head_weights, normal_bf16
from tests.gpu_util import DenseCache, bits, make_pool

pytestmark = pytest.mark.gpu

REL_Y = 2e-2
H, I, E, K, HC, LOW, V = 2048, 512, 64, 4, 4, 64, 4096


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _rand_bits(shape, std, seed, mean=0.0):
    rng = np.random.default_rng(seed)
    return O.f32_to_bf16((rng.standard_normal(shape) * std + mean).astype(np.float32))


@pytest.mark.parametrize("R,n,group", [(1, 8192, None), (3, 8192, 2048), (2, 2048, None), (5, 520, 8), (4, 96, 32)])
def test_rmsnorm_groups_bitwise(R, n, group):
    print(f"[rmsnorm] R={R} n={n} group={group}", flush=True)
    x = _rand_bits((R, n), 3.0, R * n)
    w = _rand_bits((n,), 0.1, n, 1.0)
    out = HO.rmsnorm(_dev(x), _dev(w), 1e-6, group=group)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), O.rmsnorm_groups(x, w, 1e-6, group=group))


@pytest.mark.parametrize("R,Kd,N", [(1, 8192, 64), (4, 64, 8192), (1, 8192, 4), (5, 2048, 2048), (2, 320, 77)])
@pytest.mark.parametrize("epi", [HO.EPI_NONE, HO.EPI_ADD, HO.EPI_SILU_DIV, HO.EPI_SIGMOID, HO.EPI_INJECT])
def test_lin_epi_bitwise(R, Kd, N, epi):
    print(f"[lin_epi] R={R} K={Kd} N={N} epi={epi}", flush=True)
    x = _rand_bits((R, Kd), 1.0, R + Kd)
    w = _rand_bits((N, Kd), Kd ** -0.5 * 3, N + Kd)
    add = _rand_bits(((R + 1) // 2, N), 1.0, 7) if epi == HO.EPI_ADD else None
    out = HO.lin_epi(_dev(x), _dev(w), epi, hc=4, add=None if add is None else _dev(add), add_div=2)
    torch.cuda.synchronize()
    ref = O.dense_epi(x, w, epi, hc=4, add_bits=add, add_div=2)
    assert np.array_equal(bits(out), ref)


@pytest.mark.parametrize("S,hc,Hh", [(1, 4, 2048), (3, 4, 2048), (2, 1, 96), (2, 3, 40)])
def test_hc_mean_and_inject_bitwise(S, hc, Hh):
    print(f"[hc] S={S} hc={hc} H={Hh}", flush=True)
    m = O.f32_to_bf16(np.random.default_rng(1).random((S, hc * Hh)).astype(np.float32))
    hn = _rand_bits((S, hc * Hh), 1.0, 2)
    y = _rand_bits((S, Hh), 1.0, 3)
    inj = O.f32_to_bf16(np.random.default_rng(4).random((S, hc)).astype(np.float32) * 2)
    mixed = HO.hc_mean(_dev(m), _dev(hn), hc)
    hyp = _dev(hn)
    out = HO.hc_inject(hyp, _dev(y), _dev(inj))
    HO.hc_inject(hyp, _dev(y), _dev(inj), out=hyp)  # in place
    torch.cuda.synchronize()
    assert np.array_equal(bits(mixed), O.hc_mean(m, hn, hc))
    ref = O.hc_inject(hn, y, inj)
    assert np.array_equal(bits(out), ref) and np.array_equal(bits(hyp), ref)


def test_gather_rows_wide_narrow_and_out_of_range():
    print("[gather]", flush=True)
    _lib.device_error(clear=True)
    src = normal_bf16((50, 2048), 1.0, 11)
    idx = torch.tensor([3, 49, 0, 3], dtype=torch.int32, device="cuda")
    out = HO.gather_rows(src, idx, idx_add=0)
    ints = torch.arange(10, dtype=torch.int32, device="cuda") * 7
    one = torch.tensor([2], dtype=torch.int32, device="cuda")
    pick = HO.gather_rows(ints, one, idx_add=3)  # 4-byte rows: element 5
    torch.cuda.synchronize()
    assert torch.equal(out, src[[3, 49, 0, 3]]) and int(pick[0]) == 35
    assert _lib.device_error(clear=True) == 0
    bad = HO.gather_rows(src, torch.tensor([1, 50], dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(bad[0], src[1]) and not bad[1].float().abs().sum()
    assert _lib.device_error(clear=True) == 4


def _lm_head(seed, vocab=V):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randint(-2**31, 2**31 - 1, (vocab, H // 8), generator=g, device="cuda", dtype=torch.int32)
    sc = (torch.randn((vocab, H // 64), generator=g, device="cuda") * 0.02).abs().to(torch.bfloat16)
    return AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, vocab, H)


@pytest.mark.parametrize("R,rounded", [(1, True), (3, True), (2, False)])
def test_lm_head_argmax(R, rounded):
    print(f"[argmax] R={R} round_bf16={rounded}", flush=True)
    lm = _lm_head(21)
    am = LMHeadArgmax(lm, max_rows=4, round_bf16=rounded)
    x = normal_bf16((R, H), 1.0, 22 + R)
    logits = torch.empty((R, V), dtype=torch.float32, device="cuda")
    ids = am(x, logits=logits)
    ref = gemv(x, lm)
    if rounded:
        ref = ref.to(torch.bfloat16).float()
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    assert np.array_equal(lg.view(np.uint32), ref.cpu().numpy().view(np.uint32))
    want = O.argmax_bf16(lg) if rounded else np.argmax(lg, axis=-1)
    assert np.array_equal(ids.cpu().numpy(), want)


@pytest.fixture(scope="module")
def head():
    print(f"[head] H={H} hc={HC} low={LOW} E={E} K={K} V={V}", flush=True)
    pool = make_pool(E, H, I, seed=515, layers=2)
    lw = LayerWeights(H, E, 512, seed=516)
    moe = MoEVerifyLayer(pool, 1, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K, max_tokens=4)
    hw = head_weights(H, HC, LOW, V, seed=517)
    h = MTPHead(hw, moe, _lm_head(518), hc=HC, max_ctx=64)
    return h, pool, lw, hw


def _np_weights(hw):
    def hcd(c):
        d = {"hc_norm": bits(c.hc_norm), "down": bits(c.down), "up": bits(c.up)}
        if c.inject is not None:
            d["inject"] = bits(c.inject)
        return d

    return {"pre_fc_norm_embedding": bits(hw.pre_fc_norm_embedding), "fc_embedding": bits(hw.fc_embedding),
            "pre_fc_norm_hidden": bits(hw.pre_fc_norm_hidden), "fc_hidden": bits(hw.fc_hidden),
            "mlp_hc": hcd(hw.mlp_hc), "mixer_hc": hcd(hw.mixer_hc)}


# Launches with norm groups of 2048 elements, at most four per launch, take the grouped pre-step (the first,
# second, fourth and seventh shapes here); the others the staged one.
@pytest.mark.parametrize("S,n,K,group,inject,two", [(1, 8192, 8192, 2048, False, True), (1, 8192, 8192, 2048, True, False),
                                                     (1, 8192, 2048, 8192, False, False), (2, 2048, 2048, 2048, True, True),
                                                     (3, 2048, 2048, 512, False, False),
                                                     (3, 8192, 8192, 2048, True, False),
                                                     (1, 2048, 2048, 2048, False, False), (4, 8192, 2048, 8192, False,
                                                                                              False),
                                                     (2, 520, 520, 40, False, True), (5, 96, 32, 32, True, False)])
def test_head_gemv_equals_the_separate_ops(S, n, K, group, inject, two):
    """ssmoe_head_gemv against the separate launches it replaces (hc_inject, rmsnorm, dense_gemv_epi, twice),
    bit for bit, at the head's shapes and at ragged ones: h, x, both outputs."""
    print(f"[head_gemv] S={S} n={n} K={K} group={group} inject={inject} two={two}", flush=True)
    hcj = 4
    src = _dev(_rand_bits((S, n), 2.0, S + n))
    nw = _dev(_rand_bits((n,), 0.1, n + 1, 1.0))
    w = _dev(_rand_bits((77, K), K ** -0.5 * 3, K + 2))
    w2 = _dev(_rand_bits((4, K), K ** -0.5 * 3, K + 3)) if two else None
    y = _dev(_rand_bits((S, n // hcj), 1.0, 9)) if inject else None
    inj = _dev(_rand_bits((S, hcj), 0.5, 10, 1.0)) if inject else None
    R = S * n // K
    out, hout, xout = (torch.empty((R, 77), dtype=torch.bfloat16, device="cuda"),
                       torch.empty((S, n), dtype=torch.bfloat16, device="cuda"),
                       torch.empty((S, n), dtype=torch.bfloat16, device="cuda"))
    out2 = torch.empty((R, 4), dtype=torch.bfloat16, device="cuda") if two else None
    HO.head_gemv(src, w, out, S=S, n=n, K=K, inj=inj, inj_y=y, inj_hc=hcj, norm_w=nw, eps=1e-6, group=group,
                 epi=HO.EPI_SILU_DIV, hc=4, w2=w2, out2=out2, epi2=HO.EPI_INJECT, h_out=hout, x_out=xout)
    h = HO.hc_inject(src, y, inj) if inject else src
    x = HO.rmsnorm(h, nw, 1e-6, group=group)
    ref = HO.lin_epi(x.view(R, K), w, HO.EPI_SILU_DIV, hc=4)
    torch.cuda.synchronize()
    assert torch.equal(hout, h) and torch.equal(xout, x) and torch.equal(out, ref)
    if two:
        assert torch.equal(out2, HO.lin_epi(x.view(R, K), w2, HO.EPI_INJECT, hc=4))


@pytest.mark.parametrize("S,L,H4", [(1, 64, 2048), (3, 320, 512), (2, 40, 96)])
def test_head_gemv_mean_and_table_rows(S, L, H4):
    """The up GEMV with the branch mean fused behind it equals lin_epi + hc_mean; table rows by device index equal
    gather_rows + rmsnorm + lin_epi, and an index outside the table reads zeros and raises the token error."""
    print(f"[head_gemv mean] S={S} L={L} H={H4}", flush=True)
    low = _dev(_rand_bits((S, L), 1.0, L))
    up = _dev(_rand_bits((4 * H4, L), L ** -0.5 * 3, L + 1))
    hn = _dev(_rand_bits((S, 4 * H4), 1.0, L + 2))
    mw, mixed = (torch.empty((S, 4 * H4), dtype=torch.bfloat16, device="cuda"),
                 torch.empty((S, H4), dtype=torch.bfloat16, device="cuda"))
    HO.head_gemv(low, up, mw, S=S, n=L, K=L, epi=HO.EPI_SIGMOID, hc=4, mean_hn=hn, mean_out=mixed)
    ref = HO.lin_epi(low, up, HO.EPI_SIGMOID)
    torch.cuda.synchronize()
    assert torch.equal(mw, ref) and torch.equal(mixed, HO.hc_mean(ref, hn, 4))
    table = _dev(_rand_bits((50, H4), 1.0, 3))
    nw = _dev(_rand_bits((H4,), 0.1, 4, 1.0))
    w = _dev(_rand_bits((33, H4), H4 ** -0.5, 5))
    idx = torch.tensor([7, 49, 0][:S] if S <= 3 else [7] * S, dtype=torch.int32, device="cuda")
    out, emb = (torch.empty((S, 33), dtype=torch.bfloat16, device="cuda"),
                torch.empty((S, H4), dtype=torch.bfloat16, device="cuda"))
    HO.head_gemv(table, w, out, S=S, n=H4, K=H4, src_idx=idx, norm_w=nw, eps=1e-6, group=H4, h_out=emb)
    g = HO.gather_rows(table, idx)
    ref = HO.lin_epi(HO.rmsnorm(g, nw, 1e-6), w)
    torch.cuda.synchronize()
    assert torch.equal(emb, g) and torch.equal(out, ref)
    _lib.device_error(clear=True)
    bad = torch.tensor([50] * S, dtype=torch.int32, device="cuda")
    HO.head_gemv(table, w, out, S=S, n=H4, K=H4, src_idx=bad, norm_w=nw, eps=1e-6, group=H4, h_out=emb)
    torch.cuda.synchronize()
    assert _lib.device_error(clear=True) & 4 and not emb.float().abs().sum().item()


def test_draft_chain_teacher_forced(head):
    h, pool, lw, hw = head
    k = 3
    print(f"[draft] k={k}", flush=True)
    token = torch.tensor([1234], dtype=torch.int32, device="cuda")
    multi = normal_bf16((1, HC * H), 1.0, 519)
    out = torch.empty(k, dtype=torch.int32, device="cuda")
    h.draft_async(token, multi, k, out)
    torch.cuda.synchronize()
    r = h.draft_rows(k)
    toks = out.cpu().numpy()
    W = _np_weights(hw)
    emb = bits(hw.embed)
    dense = DenseCache(pool, layer=1)
    prev_tok, prev_multi = 1234, bits(multi)
    for i in range(k):
        e = bits(r.emb[i])[0:1]
        assert np.array_equal(e, emb[prev_tok:prev_tok + 1]), i
        gpu_y = bits(r.y[i])
        o_out, o_h, p = MH.step(e, prev_multi, W, HC, lambda mixed, y=gpu_y: y)
        for name in ("e_norm", "e_proj", "m_norm", "fused", "hn", "low", "mix_w", "mixed", "inj", "h", "hn2", "low2",
                     "mix_w2", "out"):
            assert np.array_equal(bits(getattr(r, name)[i]), p[name]), (i, name)
        # The head's MoE on the GPU's mixed row: router bit for bit, y within the bound.
        _, _, ids, wts = O.router(p["mixed"], bits(lw.router_w), K)
        assert np.array_equal(r.ids[i].cpu().numpy(), ids) and np.array_equal(r.weights[i].cpu().numpy(), wts)
        routed = O.moe_routed_fp64(O.bf16_to_f32(p["mixed"]), ids, wts, dense).astype(np.float32)
        sh, sgl = O.shared_expert(p["mixed"], bits(lw.sh_gate), bits(lw.sh_up), bits(lw.sh_down), bits(lw.sh_g))
        y_ref = O.combine_shared(routed, sh, sgl)
        assert O.rel_l2(O.bf16_to_f32(gpu_y), O.bf16_to_f32(y_ref)) <= REL_Y
        logits = gemv(r.out[i], h.lm_head).cpu().numpy()
        assert toks[i] == O.argmax_bf16(logits)[0], i
        prev_tok, prev_multi = int(toks[i]), bits(r.h[i])
    print(f"drafts {toks.tolist()}")


def test_draft_graph_replays_equal_eager(head):
    h, _, _, _ = head
    k = 3
    dg = DraftGraph(h, k)
    dg.capture()
    for rep, (tok, seed) in enumerate([(7, 600), (4000, 601), (7, 600)]):
        print(f"[draft graph] replay {rep}", flush=True)
        multi = normal_bf16((1, HC * H), 1.0, seed)
        dg.token.fill_(tok)
        dg.multi.copy_(multi)
        got = dg.replay().clone()
        snap = bits(h.draft_rows(k).h)
        torch.cuda.synchronize()
        want = torch.empty(k, dtype=torch.int32, device="cuda")
        h.draft_async(torch.tensor([tok], dtype=torch.int32, device="cuda"), multi, k, want)
        torch.cuda.synchronize()
        assert torch.equal(got, want), rep
        assert np.array_equal(snap, bits(h.draft_rows(k).h)), rep


def test_consume_and_draft_bookkeeping(head):
    h, _, _, _ = head
    h.reset()
    multi_rows = normal_bf16((3, HC * H), 1.0, 700)
    with pytest.raises(RuntimeError):
        h.draft(5, 2)
    with pytest.raises(ValueError):
        h.consume([], multi_rows[:0])
    with pytest.raises(ValueError):
        h.consume([1, 2], multi_rows)
    h.consume([10, 11, 12], multi_rows)
    assert h.state.pos == 2 and h.consumed == 3 and torch.equal(h.prev_multi, multi_rows[2:3])
    h.consume([13], multi_rows[:1])
    assert h.state.pos == 3 and h.consumed == 4 and torch.equal(h.prev_multi, multi_rows[0:1])
    d = h.draft(99, 3)
    assert h.state.pos == 3  # drafting runs on a fork
    out = torch.empty(3, dtype=torch.int32, device="cuda")
    h.draft_async(torch.tensor([99], dtype=torch.int32, device="cuda"), h.prev_multi, 3, out)
    assert out.cpu().tolist() == d and all(0 <= t < V for t in d)
    h.reset()
    assert h.state.pos == 0 and h.prev_multi is None and h.consumed == 0
