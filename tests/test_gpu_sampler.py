"""The reference sampler on the GPU (ssmoe_sample through engine.sampler.Sampler) against its definition
(oracle.sample): token and flags bit for bit over the reference's fixture grid and over random rows with every
filter, edge values (NaN, -inf, ties, tiny and large vocabularies); and the reference's own draws."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd import _lib
from slotstream_spark_amd.engine.sampler import SampleParams, Sampler
from tests.golden.gen import replay_sampler_case, sampler_logits

pytestmark = pytest.mark.gpu
GOLD = json.loads((Path(__file__).resolve().parent / "golden" / "sampler_ref.json").read_text())


class Dev:
    """One device sampler row: draw(...) -> (token, flags) with an explicit uniform."""

    def __init__(self, v):
        self.work = torch.empty(int(_lib.lib().ssmoe_sample_workspace_bytes(v)), dtype=torch.uint8, device="cuda")
        self.out = torch.empty(2, dtype=torch.int32, device="cuda")
        self.u = torch.empty(1, dtype=torch.float32, device="cuda")

    def draw(self, x, gen, t, tp, tk, mp, pp, u):
        g = sorted(set(int(a) for a in gen))
        gt = torch.tensor(g, dtype=torch.int32, device="cuda") if g else None
        self.u.fill_(float(u))
        _lib.check(_lib.lib().ssmoe_sample(x.data_ptr(), x.numel(), _lib.ptr(gt), len(g), float(t), float(tp), int(tk),
                                           float(mp), float(pp), self.u.data_ptr(), self.work.data_ptr(),
                                           self.work.numel(), self.out.data_ptr(), 0))
        o = self.out.cpu().numpy()
        return int(o[0]), int(o[1])


@pytest.mark.parametrize("vocab", [256, 4096, 151936])
def test_fixture_grid_bitwise_and_reference(vocab):
    print(f"[sampler] fixture grid vocab={vocab}", flush=True)
    x = sampler_logits(vocab, 99)
    xd = torch.from_numpy(x).cuda()
    dev = Dev(vocab)
    ok = tot = 0
    for case in [c for c in GOLD["cases"] if c["vocab"] == vocab]:
        got = replay_sampler_case(case, xd, lambda l, g, *a: dev.draw(l, g, *a)[0])
        want = replay_sampler_case(case, x, lambda l, g, *a: O.sample(l, g, *a)[0])
        assert got == want, case
        ok += sum(a == b for a, b in zip(got, case["tokens"]))
        tot += len(got)
    assert ok >= tot - 2  # the reference's own draws (see tests/test_sampler_oracle.py)


EDGE_PARAMS = [(0.0, 1.0, 0, 0.0, 0.0), (0.7, 1.0, 0, 0.0, 0.0), (1.0, 0.9, 0, 0.0, 0.0), (0.6, 0.5, 40, 0.05, 1.5),
               (1.3, 1.0, 1, 0.0, 0.0), (0.9, 0.95, 0, 0.2, -0.7), (0.8, 1e-6, 0, 0.0, 0.0), (1.0, 1.0, 0, 1.0, 0.0),
               (2.0, 0.3, 7, 0.0, 3.0)]


@pytest.mark.parametrize("v,seed", [(1, 0), (7, 1), (1023, 2), (1024, 3), (1025, 4), (5000, 5), (248320, 6)])
def test_random_rows_bitwise(v, seed):
    print(f"[sampler] random rows v={v}", flush=True)
    rng = np.random.default_rng(seed)
    dev = Dev(v)
    for r in range(4):
        x = (rng.standard_normal(v) * (1 + 3 * r)).astype(np.float32)
        if r == 1 and v > 4:
            x[rng.integers(0, v, 3)] = -np.inf
        if r == 2 and v > 4:
            x[: v // 2] = np.float32(1.25)  # large tie groups
        xd = torch.from_numpy(x).cuda()
        gen = set(rng.integers(0, v, min(v, 20)).tolist())
        for (t, tp, tk, mp, pp) in EDGE_PARAMS:
            u = np.float32(rng.random())
            assert dev.draw(xd, gen, t, tp, tk, mp, pp, u) == O.sample(x, gen, t, tp, tk, mp, pp, u), (r, t, tp, tk)
        for u in (np.float32(0.0), np.float32(1.0)):
            assert dev.draw(xd, (), 1.0, 0.8, 0, 0.0, 0.0, u) == O.sample(x, (), 1.0, 0.8, 0, 0.0, 0.0, u)


def test_nonfinite_rows_fall_back_to_argmax():
    x = np.random.default_rng(9).standard_normal(3000).astype(np.float32)
    x[1234] = np.nan
    xd = torch.from_numpy(x).cuda()
    dev = Dev(3000)
    for params in [(1.0, 1.0, 0, 0.0, 0.0), (0.7, 0.9, 10, 0.1, 0.0), (0.0, 1.0, 0, 0.0, 0.0)]:
        assert dev.draw(xd, (), *params, np.float32(0.3)) == O.sample(x, (), *params, 0.3)
    assert O.sample(x, (), 1.0, 1.0, 0, 0.0, 0.0, 0.3) == (1234, 1)  # numpy's max propagates NaN: argmax fallback


def test_sampler_api_advances_like_the_reference():
    v = 4096
    x = sampler_logits(v, 99)
    case = [c for c in GOLD["cases"] if c["vocab"] == v and c["temperature"] > 0][0]
    s = Sampler(case["seed"])
    p = SampleParams(temperature=case["temperature"], top_p=case["top_p"], top_k=case["top_k"], min_p=case["min_p"],
                     presence_penalty=case["presence_penalty"])
    xd = torch.from_numpy(x).cuda()
    gen, toks = set(), []
    for _ in range(16):
        t = s.next(xd, p, gen)
        toks.append(t)
        if case["accumulate"]:
            gen.add(t)
    want = replay_sampler_case(case, x, lambda l, g, *a: O.sample(l, g, *a)[0])
    assert toks == want


# ---- the sampled verify round on the device (ssmoe_accept_sampled) against oracle.accept_sampled

def _self_drafts(t, seen, params, u):
    """Drafts equal to the round's own draws, so every row is reached (the penalty set grows through the round)."""
    d = t.shape[0] - 1
    drafts = np.full(d, -1, np.int32)
    for i in range(d):
        out = O.accept_sampled(t, drafts, seen, *params, u)
        drafts[i] = out[4 + i]
    return drafts


ROUND_PARAMS = [(0.7, 1.0, 0, 0.0, 0.0), (0.8, 0.95, 40, 0.0, 0.0), (0.7, 0.9, 0, 0.05, 1.2), (0.0, 1.0, 0, 0.0, 2.0),
                (1.1, 0.5, 5, 0.0, -0.5)]


@pytest.mark.parametrize("v", [3000, 151936])
def test_accept_sampled_bitwise(v):
    from slotstream_spark_amd.engine.accept import Acceptor, AcceptResult
    print(f"[sampler] accept_sampled v={v}", flush=True)
    rng = np.random.default_rng(v)
    D = 3
    acc = Acceptor(D, v)
    for k, params in enumerate(ROUND_PARAMS):
        t = (rng.standard_normal((D + 1, v)) * 3).astype(np.float32)
        u = rng.random(D + 1).astype(np.float32)
        seen = set(rng.integers(0, v, 12).tolist())
        for drafts in (_self_drafts(t, seen, params, u), rng.integers(0, v, D).astype(np.int32)):
            want = O.accept_sampled(t, drafts, seen, *params, u)
            sp = SampleParams(temperature=params[0], top_p=params[1], top_k=params[2], min_p=params[3],
                              presence_penalty=params[4])
            got = acc.sampled_async(torch.from_numpy(t).cuda(), torch.from_numpy(drafts).cuda(), sp, seen,
                                    torch.from_numpy(u).cuda()).cpu().numpy()
            assert got[:4].tolist() == want[:4].tolist(), (k, got, want)
            assert got[4: 4 + got[1]].tolist() == want[4: 4 + want[1]].tolist(), (k, got, want)
        if k == 0:
            assert want[0] >= 0 and AcceptResult.from_out(got).n_emit == want[1]
    # a non-finite row ends the round before its draw
    t = (rng.standard_normal((D + 1, v)) * 3).astype(np.float32)
    u = rng.random(D + 1).astype(np.float32)
    drafts = _self_drafts(t, (), ROUND_PARAMS[1], u)
    t[2, v // 3] = np.nan
    want = O.accept_sampled(t, drafts, (), *ROUND_PARAMS[1], u)
    got = acc.sampled_async(torch.from_numpy(t).cuda(), torch.from_numpy(drafts).cuda(), SampleParams(), (),
                            torch.from_numpy(u).cuda()).cpu().numpy()
    assert want[:4].tolist() == [2, 2, 2, 1] and got[:6].tolist() == want[:6].tolist()


def test_accept_sampled_stream_and_seen_follow_the_reference_loop():
    """Acceptor.sampled advances the sampler's stream by the draws made and adds the emitted tokens to seen, so two
    rounds in a row equal the oracle rounds fed from the same stream."""
    from slotstream_spark_amd.engine.accept import Acceptor, UniformStream
    v, D = 4096, 3
    rng = np.random.default_rng(5)
    acc = Acceptor(D, v)
    params = SampleParams(temperature=0.7, top_p=0.95, top_k=40, presence_penalty=0.8)
    dev_stream, ref_stream = UniformStream(77), UniformStream(77)
    dev_seen, ref_seen = {1, 2, 3}, {1, 2, 3}
    for _ in range(3):
        t = (rng.standard_normal((D + 1, v)) * 3).astype(np.float32)
        u = ref_stream.peek(D + 1)
        p = params.sanitized()
        drafts = _self_drafts(t, ref_seen, (p.temperature, p.top_p, p.top_k, p.min_p, p.presence_penalty), u)
        drafts[2] = (drafts[2] + 1) % v
        want = O.accept_sampled(t, drafts, ref_seen, p.temperature, p.top_p, p.top_k, p.min_p, p.presence_penalty, u)
        ref_stream.advance(int(want[2]))
        ref_seen.update(want[4: 4 + want[1]].tolist())
        res = acc.sampled(torch.from_numpy(t).cuda(), torch.from_numpy(drafts).cuda(), params, dev_seen, dev_stream)
        assert (res.n_accept, res.n_emit, res.n_uniform) == (2, 3, 3)
        assert res.tokens == want[4: 4 + want[1]].tolist()
        assert dev_stream.state == ref_stream.state and dev_seen == ref_seen


@pytest.mark.parametrize("v", [5000, 151936])
def test_compact_top_p_and_its_fallback_bitwise(v):
    """Top-k rows find the top-p threshold from their survivors (up to 512) instead of the 13 radix rounds; rows with
    more survivors (a large top-k, or ties at the k-th value) run the rounds. Both equal or_sample bit for bit."""
    print(f"[sampler] compact top-p v={v}", flush=True)
    rng = np.random.default_rng(v + 17)
    dev = Dev(v)
    rows = [(rng.standard_normal(v) * 4).astype(np.float32), np.full(v, 1.25, np.float32)]
    tied = (rng.standard_normal(v) * 2).astype(np.float32)
    tied[rng.permutation(v)[:700]] = np.float32(9.0)  # 700 ties at the top: k = 40 keeps all 700
    rows.append(tied)
    for ri, x in enumerate(rows):
        xd = torch.from_numpy(x).cuda()
        for (t, tp, tk, mp, pp) in [(0.7, 0.95, 40, 0.0, 0.0), (1.0, 0.9, 300, 0.0, 0.0), (1.0, 0.99, 512, 0.02, 0.0),
                                    (0.9, 0.8, 600, 0.0, 0.0), (1.2, 0.5, 2, 0.0, 0.0), (0.5, 0.999, 100, 0.0, 1.0)]:
            for u in (np.float32(0.0), np.float32(rng.random()), np.float32(0.9999)):
                gen = set(rng.integers(0, v, 8).tolist())
                assert dev.draw(xd, gen, t, tp, tk, mp, pp, u) == O.sample(x, gen, t, tp, tk, mp, pp, u), (ri, tk, u)
