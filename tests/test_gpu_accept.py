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
