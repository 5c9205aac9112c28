"""Pins of the MTP head's CPU restatement (oracle/mtp_head.py and the or_rmsnorm_groups / or_dense_epi / or_hc_mean /
or_hc_inject C functions) and of the head's host-side bookkeeping (engine/mtp.py draft_depth, MTPState):

  * rmsnorm and hc_mix against the reference's own torch CPU functions (model/reference_torch.py:30-38 rmsnorm,
    :174-183 RefModel.gated_residual) on tests/golden/mtp_ref.npz: equal up to the order of two fp32 sums
    (each value within one bf16 ulp, most bit-identical); a per-group norm where the reference normalises the full
    width, or the reverse, fails;
  * the epilogues against float64 numpy silu / sigmoid;
  * fuse (engine/mtp.py:184-192) and the head step (:209-227 without attention) by closed forms: zero multi gives
    the embedding projection in every branch; an identity fc_hidden exposes the full-width norm in branch order;
    zero hyper-connection weights reduce the step to a residual add and a half-weighted branch mean.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import mtp_head as MH
from oracle import oracle as O

GOLD = Path(__file__).resolve().parent / "golden" / "mtp_ref.npz"


def _f(b):
    return O.bf16_to_f32(b).astype(np.float64)


def _within_ulp(a_bits, b_bits, ulps=1):
    a, b = _f(a_bits), _f(b_bits)
    tol = ulps * np.maximum(np.abs(b), 1e-30) * 2.0 ** -7
    return bool(np.all(np.abs(a - b) <= tol))


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def test_rmsnorm_against_reference(gold):
    x, w = gold["norm_x"], gold["norm_w"]
    full = O.rmsnorm_groups(x, w, 1e-6)
    grp = O.rmsnorm_groups(x, w, 1e-6, group=128)
    for mine, ref in ((full, gold["norm_full"]), (grp, gold["norm_group"])):
        assert _within_ulp(mine, ref)
        assert np.mean(mine == ref) > 0.97
    # The two variants differ (branch scales 0.5 .. 4): swapping them would not pass.
    assert np.mean(full == gold["norm_group"]) < 0.5 and np.mean(grp == gold["norm_full"]) < 0.5


def test_hc_mix_against_reference(gold):
    P = {"hc_norm": gold["hc_hc_norm"], "down": gold["hc_input_mix_weight_down"],
         "up": gold["hc_input_mix_weight_up"], "inject": gold["hc_block_inject_weight"]}
    mixed, inj, _ = MH.hc_mix(gold["hc_hyp"], P, 4)
    assert O.rel_l2(_f(mixed), _f(gold["hc_mixed"])) < 5e-3
    assert np.mean(mixed == gold["hc_mixed"]) > 0.9
    assert _within_ulp(inj, gold["hc_inj"], 2)
    mixed_ni, none, _ = MH.hc_mix(gold["hc_hyp"], P, 4, inject=False)
    assert none is None and np.array_equal(mixed_ni, mixed)
    assert np.mean(mixed_ni == gold["hc_mixed_noinject"]) > 0.9
    # Negative control: the transposed branch layout (element-major instead of branch-major) is far off.
    hyp_t = gold["hc_hyp"].reshape(3, 4, 128).transpose(0, 2, 1).reshape(3, 512).copy()
    bad, _, _ = MH.hc_mix(hyp_t, P, 4)
    assert O.rel_l2(_f(bad), _f(gold["hc_mixed"])) > 0.1


def test_epilogues_against_float64():
    rng = np.random.default_rng(5)
    R, K, N, hc = 3, 320, 96, 4
    x = O.f32_to_bf16(rng.standard_normal((R, K)).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal((N, K)) * 0.2).astype(np.float32))
    v = _f(O.dense_epi(x, w))
    assert np.array_equal(O.dense_epi(x, w), O.dense_rows(x, w))

    def rb(a):
        return _f(O.f32_to_bf16(a.astype(np.float32)))

    u = rb(v / hc)
    cases = {O.EPI_SILU_DIV: u / (1 + np.exp(-u)), O.EPI_SIGMOID: 1 / (1 + np.exp(-v)),
             O.EPI_INJECT: 2 * rb(1 / (1 + np.exp(-u)))}
    for epi, ref in cases.items():
        got = O.dense_epi(x, w, epi, hc=hc)
        assert _within_ulp(got, O.f32_to_bf16(ref.astype(np.float32))), epi
    add = O.f32_to_bf16(rng.standard_normal((1, N)).astype(np.float32))
    got = O.dense_epi(x, w, O.EPI_ADD, add_bits=add, add_div=3)
    assert np.array_equal(got, O.f32_to_bf16((v + _f(add)).astype(np.float32)))


def test_hc_mean_and_inject_closed_form():
    rng = np.random.default_rng(6)
    S, hc, H = 2, 4, 40
    m = O.f32_to_bf16(rng.random((S, hc * H)).astype(np.float32))
    hn = O.f32_to_bf16(rng.standard_normal((S, hc * H)).astype(np.float32))
    prod = _f(O.f32_to_bf16((_f(m) * _f(hn)).astype(np.float32))).reshape(S, hc, H)
    acc = np.zeros((S, H), np.float32)
    for c in range(hc):
        acc = (acc + prod[:, c].astype(np.float32)).astype(np.float32)
    assert np.array_equal(O.hc_mean(m, hn, hc), O.f32_to_bf16(acc / np.float32(hc)))
    y = O.f32_to_bf16(rng.standard_normal((S, H)).astype(np.float32))
    inj = O.f32_to_bf16(rng.random((S, hc)).astype(np.float32) * 2)
    t = _f(O.f32_to_bf16((_f(y)[:, None, :] * _f(inj)[:, :, None]).astype(np.float32)))
    ref = O.f32_to_bf16((_f(hn).reshape(S, hc, H) + t).astype(np.float32)).reshape(S, hc * H)
    assert np.array_equal(O.hc_inject(hn, y, inj), ref)


def _weights(H, hc, low, seed, zero_hc=False, **over):
    rng = np.random.default_rng(seed)
    n = hc * H

    def b(shape, std, mean=0.0):
        return O.f32_to_bf16((rng.standard_normal(shape) * std + mean).astype(np.float32))

    def hcw(inject):
        d = {"hc_norm": b((n,), 0.1, 1.0), "down": b((low, n), n ** -0.5), "up": b((n, low), low ** -0.5)}
        if inject:
            d["inject"] = b((hc, n), n ** -0.5)
        if zero_hc:
            for k in ("down", "up", "inject"):
                if k in d:
                    d[k] = np.zeros_like(d[k])
        return d

    W = {"pre_fc_norm_embedding": b((H,), 0.1, 1.0), "fc_embedding": b((H, H), H ** -0.5),
         "pre_fc_norm_hidden": b((n,), 0.1, 1.0), "fc_hidden": b((H, H), H ** -0.5), "mlp_hc": hcw(True),
         "mixer_hc": hcw(False)}
    W.update(over)
    return W


def test_fuse_closed_forms():
    H, hc, S = 64, 4, 2
    rng = np.random.default_rng(7)
    e = O.f32_to_bf16(rng.standard_normal((S, H)).astype(np.float32))
    W = _weights(H, hc, 16, 8)
    # Zero multi: rmsnorm(0) = 0, so every branch is the embedding projection.
    h, parts = MH.fuse(e, np.zeros((S, hc * H), np.uint16), W, hc)
    ep = O.dense_rows(O.rmsnorm_groups(e, W["pre_fc_norm_embedding"]), W["fc_embedding"])
    assert np.array_equal(h, np.tile(ep, (1, hc)))
    # Identity fc_hidden, unit norm weight, zero fc_embedding: h is the full-width norm of multi, branch-major.
    scale = np.repeat(np.array([0.25, 1.0, 4.0, 16.0], np.float32), H)
    multi = O.f32_to_bf16((rng.standard_normal((S, hc * H)) * scale).astype(np.float32))
    W2 = dict(W, fc_hidden=O.f32_to_bf16(np.eye(H, dtype=np.float32)),
              pre_fc_norm_hidden=O.f32_to_bf16(np.ones(hc * H, np.float32)),
              fc_embedding=np.zeros((H, H), np.uint16))
    h2, _ = MH.fuse(e, multi, W2, hc)
    mf = _f(multi)
    r = 1.0 / np.sqrt((mf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert _within_ulp(h2, O.f32_to_bf16((mf * r).astype(np.float32)))


def test_step_closed_form_with_zero_mixing():
    H, hc, S = 64, 4, 2
    rng = np.random.default_rng(9)
    e = O.f32_to_bf16(rng.standard_normal((S, H)).astype(np.float32))
    multi = O.f32_to_bf16(rng.standard_normal((S, hc * H)).astype(np.float32))
    W = _weights(H, hc, 16, 10, zero_hc=True)
    y = O.f32_to_bf16(rng.standard_normal((S, H)).astype(np.float32))
    seen = []

    def moe(mixed):
        seen.append(mixed)
        return y

    out, h2, parts = MH.step(e, multi, W, hc, moe)
    h, _ = MH.fuse(e, multi, W, hc)

    def half_mean(hyp, P):
        hn = _f(O.rmsnorm_groups(hyp, P["hc_norm"], group=H)).reshape(S, hc, H)
        half = _f(O.f32_to_bf16((0.5 * hn).astype(np.float32)))
        acc = np.zeros((S, H), np.float32)
        for c in range(hc):
            acc = (acc + half[:, c].astype(np.float32)).astype(np.float32)
        return O.f32_to_bf16(acc / np.float32(hc))

    # Zero down/up/inject weights: mix weights sigmoid(0) = 1/2, injection 2 sigmoid(0) = 1.
    assert np.array_equal(seen[0], half_mean(h, W["mlp_hc"]))
    assert np.all(parts["inj"] == O.f32_to_bf16(np.float32(1.0)))
    h_ref = O.f32_to_bf16((_f(h).reshape(S, hc, H) + _f(y)[:, None, :]).astype(np.float32)).reshape(S, hc * H)
    assert np.array_equal(h2, h_ref)
    assert np.array_equal(out, half_mean(h2, W["mixer_hc"]))


def test_argmax_bf16_first_index_and_nan():
    x = np.array([[1.0, 3.0, 3.0000001, -1.0], [0.0, np.nan, 5.0, np.nan], [2.0, 2.0, 1.0, 2.0]], np.float32)
    # 3.0 and 3.0000001 round to the same bf16 value: the first one wins; NaN counts as the maximum.
    assert O.argmax_bf16(x).tolist() == [1, 1, 0]


def test_draft_depth_and_state():
    from slotstream_spark_amd.engine.mtp import DEPTH, MAP_ROW, MTPState, draft_depth

    assert (MAP_ROW, DEPTH) == (48, 2)
    assert draft_depth(100, 0) == 2 and draft_depth(100, 97) == 2 and draft_depth(100, 98) == 1
    assert draft_depth(100, 99) == 0 and draft_depth(100, 150) == 0 and draft_depth(100, 0, 5) == 5
    st = MTPState(16)
    assert not st.aligned(0) and st.aligned(1)
    st.pos = 3
    f = st.fork()
    f.pos += 2
    assert st.pos == 3 and f.pos == 5 and f.max_ctx == 16 and st.aligned(4)
    st.reset()
    assert st.pos == 0 and st.offset == 0
