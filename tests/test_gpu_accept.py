"""Greedy and p/q acceptance on the GPU at BASELINE config 2 (depth 3, vocab 151936), bit for bit against the
CPU restatement, including non-finite rows and out-of-range drafts."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd import _lib
from slotstream_spark_amd.engine.accept import Acceptor, UniformStream
from slotstream_spark_amd.memory.synth import verify_logits

pytestmark = pytest.mark.gpu

D, V = 3, 151936


@pytest.fixture(scope="module")
def acc():
    return Acceptor(D, V)


def _drafts(target, seed, force):
    """Drafts that match the target argmax for the first `force` rows, random after."""
    g = np.random.default_rng(seed)
    am = target.argmax(axis=1)
    d = g.integers(0, V, D).astype(np.int32)
    d[:force] = am[:force]
    return d


@pytest.mark.parametrize("seed", range(6))
def test_greedy_bitexact(acc, seed):
    tgt, _ = verify_logits(D, V, 5000 + seed)
    t = tgt.cpu().numpy()
    d = _drafts(t, seed, seed % (D + 1))
    out = acc.greedy_async(tgt, torch.from_numpy(d).cuda()).cpu().numpy()
    ref = O.accept_greedy(t, d)
    assert np.array_equal(out, ref), (out, ref)
    assert out[0] == seed % (D + 1)


@pytest.mark.parametrize("d,v,seed", [(3, 307200, 1), (0, 151936, 2), (5, 100003, 3), (5, 100003, 4)])
def test_greedy_launch_forms(d, v, seed):
    """Both forms of the greedy round: (3, 307200) has 1,200 (row, chunk) units, more than the one-launch round's
    1,024 waves (the per-chunk launch with an arrival count); D = 0 emits the argmax of one row; V = 100,003 ends in
    a partial chunk of rows that are not 16-byte aligned. Two calls on one workspace each."""
    small = Acceptor(d, v)
    tgt, _ = verify_logits(d, v, 9000 + seed)
    t = tgt.cpu().numpy()
    g = np.random.default_rng(seed)
    am = t.argmax(axis=1)
    dr = g.integers(0, v, d).astype(np.int32)
    dr[:seed % (d + 1)] = am[:seed % (d + 1)]
    for _ in range(2):
        out = small.greedy_async(tgt, torch.from_numpy(dr).cuda()).cpu().numpy()
        assert np.array_equal(out, O.accept_greedy(t, dr)), out


def test_greedy_nonfinite_stops(acc):
    tgt, _ = verify_logits(D, V, 77)
    t = tgt.cpu().numpy()
    d = _drafts(t, 1, 3)
    t[2, 1234] = np.nan
    out = acc.greedy_async(torch.from_numpy(t).cuda(), torch.from_numpy(d).cuda()).cpu().numpy()
    ref = O.accept_greedy(t, d)
    assert np.array_equal(out, ref)
    assert out[1] == 2 and out[3] == 1


@pytest.mark.parametrize("seed", range(12))
def test_pq_bitexact(acc, seed):
    tgt, drf = verify_logits(D, V, 6000 + seed)
    t, q = tgt.cpu().numpy(), drf.cpu().numpy()
    # Drafts sampled from q's argmax neighbourhood so that decisions go both ways.
    g = np.random.default_rng(seed)
    d = np.where(g.random(D) < 0.7, q.argmax(axis=1), g.integers(0, V, D)).astype(np.int32)
    u = UniformStream(seed).peek(D + 1)
    out = acc.pq_async(tgt, drf, torch.from_numpy(d).cuda(), torch.from_numpy(u).cuda(), 0.7).cpu().numpy()
    ref = O.accept_pq(t, q, d, u, 0.7)
    assert np.array_equal(out, ref), (out, ref)


def test_pq_equal_distributions_accept_all(acc):
    tgt, _ = verify_logits(D, V, 11)
    d = np.array([1, 2, 3], np.int32)
    u = np.array([0.999, 0.5, 0.9999, 0.25], np.float32)
    out = acc.pq_async(tgt, tgt[:D].contiguous(), torch.from_numpy(d).cuda(), torch.from_numpy(u).cuda(),
                       0.7).cpu().numpy()
    ref = O.accept_pq(tgt.cpu().numpy(), tgt[:D].cpu().numpy(), d, u, 0.7)
    assert np.array_equal(out, ref)
    assert out[0] == D and out[1] == D + 1 and out[2] == D + 1


def test_pq_bad_draft_token_flags(acc):
    _lib.device_error(clear=True)
    tgt, drf = verify_logits(D, V, 12)
    d = np.array([5, V + 3, 7], np.int32)
    u = np.full(D + 1, 0.0, np.float32)
    out = acc.pq_async(tgt, drf, torch.from_numpy(d).cuda(), torch.from_numpy(u).cuda(), 0.7).cpu().numpy()
    ref = O.accept_pq(tgt.cpu().numpy(), drf.cpu().numpy(), d, u, 0.7)
    assert np.array_equal(out, ref)
    assert out[3] & 2
    assert _lib.device_error(clear=True) & 4


def test_pq_small_vocab_edge(acc):
    small = Acceptor(2, 37)
    g = np.random.default_rng(3)
    for i in range(20):
        t = (g.standard_normal((3, 37)) * 3).astype(np.float32)
        q = (g.standard_normal((2, 37)) * 3).astype(np.float32)
        d = g.integers(0, 37, 2).astype(np.int32)
        u = g.random(3).astype(np.float32)
        out = small.pq_async(torch.from_numpy(t).cuda(), torch.from_numpy(q).cuda(), torch.from_numpy(d).cuda(),
                             torch.from_numpy(u).cuda(), 0.7).cpu().numpy()
        assert np.array_equal(out, O.accept_pq(t, q, d, u, 0.7)), i


@pytest.mark.parametrize("d,v,seed", [(3, 307200, 1), (3, 307200, 2), (0, 151936, 3), (5, 100003, 4), (5, 100003, 5),
                                      (2, 200000, 6), (1, 400000, 7)])
def test_pq_launch_forms(d, v, seed):
    """Both forms of the round against the C definition: (3, 307200) has 1,200 (row pair, chunk) units, more than
    the one-launch round's 1,024 waves, so it runs the two-launch form; D = 0 samples the bonus row only; V = 100,003
    ends in a partial chunk and rows that are not 16-byte aligned (element loads). The chunk layout holds 1, 2, 3 or
    4 chunks per lane in builds of their own and more in a generic one: V = 200,000 (196 chunks: 4 per lane) and
    V = 400,000 (391 chunks: 7 per lane, the generic build) cover the last two."""
    small = Acceptor(d, v)
    tgt, drf = verify_logits(d, v, 8000 + seed)
    t, q = tgt.cpu().numpy(), drf.cpu().numpy()
    g = np.random.default_rng(seed)
    dr = np.where(g.random(d) < 0.7, q.argmax(axis=1), g.integers(0, v, d)).astype(np.int32) if d else \
        np.zeros(0, np.int32)
    u = UniformStream(seed).peek(d + 1)
    for _ in range(2):  # a second call on the same workspace: the counters were left at zero
        out = small.pq_async(tgt, drf, torch.from_numpy(dr).cuda(), torch.from_numpy(u).cuda(), 0.7).cpu().numpy()
        assert np.array_equal(out, O.accept_pq(t, q, dr, u, 0.7)), out
    if d:
        # q = p: every draft accepted, the bonus row sampled (its own form, without the residual pass)
        same = tgt[:d].contiguous()
        out = small.pq_async(tgt, same, torch.from_numpy(dr).cuda(), torch.from_numpy(u).cuda(), 0.7).cpu().numpy()
        assert np.array_equal(out, O.accept_pq(t, t[:d], dr, u, 0.7)), out
        assert out[0] == d and out[1] == d + 1


@pytest.mark.parametrize("seed", range(4))
def test_draw_drafts_bitexact(acc, seed):
    """The proposal draw of the p/q round (ssmoe_sample_rows): row i's token is x ~ softmax(draft_i / T) with
    uniforms[i], bit for bit against the C definition (or_draw_rows); a second call on the same workspace too."""
    _, drf = verify_logits(D, V, 7000 + seed)
    u = UniformStream(100 + seed).peek(D)
    want = O.draw_rows(drf.cpu().numpy(), 0.7, u).tolist()
    for _ in range(2):
        assert acc.draw_drafts_async(drf, torch.from_numpy(u).cuda(), 0.7).cpu().tolist() == want


@pytest.mark.parametrize("r,v,seed", [(16, 151936, 1), (64, 4096, 2), (5, 100003, 3), (2, 400000, 4), (1, 37, 5)])
def test_draw_rows_shapes(r, v, seed):
    """ssmoe_sample_rows at other shapes, bit for bit against or_draw_rows: 16 rows of 149 chunks run as three launches
    of at most six rows (every (row, chunk) unit a wave of a resident grid), 64 rows of four chunks in one; V = 100,003
    ends in a partial chunk of rows that are not 16-byte aligned; V = 400,000 has 391 chunks (seven per lane of the
    chunk layout, the generic build); V = 37 has one partial chunk."""
    x = torch.randn((r, v), generator=torch.Generator(device="cuda").manual_seed(seed), device="cuda") * 3.0
    u = np.random.default_rng(seed).random(r).astype(np.float32)
    ws = torch.zeros(int(_lib.lib().ssmoe_sample_rows_workspace_bytes(r, v)), dtype=torch.uint8, device="cuda")
    out = torch.empty(r, dtype=torch.int32, device="cuda")
    want = O.draw_rows(x.cpu().numpy(), 0.7, u).tolist()
    for _ in range(2):
        _lib.check(_lib.lib().ssmoe_sample_rows(x.data_ptr(), r, v, 0.7, torch.from_numpy(u).cuda().data_ptr(),
                                                ws.data_ptr(), ws.numel(), out.data_ptr(), _lib.stream_of(x)))
        assert out.cpu().tolist() == want


def _chi2(counts, probs):
    n = counts.sum()
    e = probs * n
    return float(((counts - e) ** 2 / e).sum())


def test_pq_round_preserves_the_target_distribution():
    """The p/q path as wired (drafts drawn from q = softmax(draft / T) by ssmoe_sample_rows, then ssmoe_accept_pq):
    the first emitted token is distributed as p_0 = softmax(target_0 / T), and the token after an accepted first
    draft as p_1 (Leviathan et al. 2023, Theorem 1), by chi-square over 8000 seeded rounds on a 6-token vocabulary.
    Critical value 25.7 = the 1e-4 tail of chi-square with 5 degrees of freedom; the argmax-draft procedure this
    replaces fails the same check on the CPU (tests/test_oracle.py)."""
    Dd, Vs, N, T = 2, 6, 8000, 0.7
    t = np.array([[1.2, 0.9, 0.2, -0.1, -0.8, 0.4], [0.1, 1.0, -0.5, 0.6, 0.3, -1.2], [0.0, 0.2, 0.4, 0.6, 0.8, 1.0]],
                 np.float32)
    q = np.array([[0.2, 1.6, 0.1, 0.3, -0.6, 0.9], [1.1, 0.2, 0.0, -0.4, 0.9, 0.1]], np.float32)
    small = Acceptor(Dd, Vs)
    g = torch.Generator(device="cuda").manual_seed(4242)
    ud = torch.rand((N, Dd), generator=g, device="cuda")
    ua = torch.rand((N, Dd + 1), generator=g, device="cuda")
    tt, qq = torch.from_numpy(t).cuda(), torch.from_numpy(q).cuda()
    drafts = torch.empty((N, Dd), dtype=torch.int32, device="cuda")
    res = torch.empty((N, Dd + 5), dtype=torch.int32, device="cuda")
    for i in range(N):
        small.draw_drafts_async(qq, ud[i], T, out=drafts[i])
        res[i].copy_(small.pq_async(tt, qq, drafts[i], ua[i], T))
    r = res.cpu().numpy()
    assert (r[:, 3] == 0).all() and (r[:, 1] >= 1).all()

    def p_of(row):
        z = np.exp((row.astype(np.float64) / T) - (row.astype(np.float64) / T).max())
        return z / z.sum()

    c0 = np.bincount(r[:, 4], minlength=Vs).astype(np.float64)
    x0 = _chi2(c0, p_of(t[0]))
    sel = r[:, 0] >= 1
    c1 = np.bincount(r[sel, 5], minlength=Vs).astype(np.float64)
    x1 = _chi2(c1, p_of(t[1]))
    # the drafts themselves follow q (the proposal is what Alg. 1 divides by)
    cq = np.bincount(drafts[:, 0].cpu().numpy(), minlength=Vs).astype(np.float64)
    xq = _chi2(cq, p_of(q[0]))
    print(f"chi2 first token {x0:.2f}, second token ({int(sel.sum())} rounds) {x1:.2f}, drafts vs q {xq:.2f}; "
          f"mean accepted {r[:, 0].mean():.3f}")
    assert x0 < 25.7 and x1 < 25.7 and xq < 25.7
