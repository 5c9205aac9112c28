"""Pins of or_draw_rows, the C definition of the p/q round's proposal draw (ssmoe_sample_rows): x_r ~ softmax(x_r / T),
chunk by chunk mass, then the entry inside the chunk. Checked against what the mathematics fixes: chi-square of the
draws against softmax on small and multi-chunk vocabularies, the inverse-CDF endpoints, the temperature, and a
planted mistake (the chunk masses left unscaled by a_c) that the multi-chunk check must reject."""
import numpy as np
import pytest

from oracle import oracle as O


def _softmax(x, t):
    z = np.exp((x.astype(np.float64) - x.max()) / t)
    return z / z.sum()


def _chi2(counts, p):
    e = p * counts.sum()
    keep = e > 0
    return float((((counts - e) ** 2)[keep] / e[keep]).sum())


def test_small_vocabulary_chi_square():
    """6 tokens, 12,000 stratified uniforms (u = (k + 0.5) / N): the counts follow softmax within chi-square 20.5
    (the 1e-3 tail at 5 degrees of freedom)."""
    x = np.array([1.2, 0.9, 0.2, -0.1, -0.8, 0.4], np.float32)
    n = 12000
    u = ((np.arange(n) + 0.5) / n).astype(np.float32)
    toks = O.draw_rows(np.tile(x, (n, 1)), 0.7, u)
    c = np.bincount(toks, minlength=6).astype(np.float64)
    assert _chi2(c, _softmax(x, 0.7)) < 20.5


def test_multi_chunk_vocabulary_masses():
    """3,000 tokens over three chunks: stratified draws land in each 64-token band in proportion to its softmax mass
    (chi-square over 47 bands, 1e-3 tail 82.7), the endpoints u -> 0 and u -> 1 give the first and the last token of
    nonzero mass, and draws move with the temperature as softmax(x / T) does."""
    g = np.random.default_rng(5)
    x = (g.standard_normal(3000) * 1.5).astype(np.float32)
    n = 20000
    u = ((np.arange(n) + 0.5) / n).astype(np.float32)
    for t in (0.7, 1.3):
        toks = O.draw_rows(np.tile(x, (n, 1)), t, u)
        p = _softmax(x, t)
        band = np.arange(3000) // 64
        c = np.bincount(band[toks], minlength=band.max() + 1).astype(np.float64)
        pb = np.bincount(band, weights=p)
        assert _chi2(c, pb) < 82.7, t
    ends = O.draw_rows(np.tile(x, (2, 1)), 0.7, np.array([0.0, np.nextafter(np.float32(1), np.float32(0))],
                                                           np.float32))
    assert ends[0] == 0 and ends[1] > 2900  # u -> 1 lands in the top tokens (their mass is ~3 %)


def test_planted_mistake_fails_the_mass_check():
    """The same band check on a restatement that picks the chunk by its unscaled total s_c (dropping a_c, a plausible
    slip) fails: the chunks' maxima differ, so their masses are not proportional to s_c."""
    g = np.random.default_rng(6)
    x = (g.standard_normal(3072) * 1.5).astype(np.float32)
    x[1024:2048] += 2.0  # chunk 1 carries most of the mass
    p = _softmax(x, 0.7)
    s = []
    for c in range(3):
        y = x[c * 1024:(c + 1) * 1024].astype(np.float64) / 0.7
        s.append(np.exp(y - y.max()).sum())
    wrong = np.array(s) / np.sum(s)
    right = np.array([p[c * 1024:(c + 1) * 1024].sum() for c in range(3)])
    n = 20000
    u = ((np.arange(n) + 0.5) / n).astype(np.float32)
    toks = O.draw_rows(np.tile(x, (n, 1)), 0.7, u)
    cc = np.bincount(toks // 1024, minlength=3).astype(np.float64)
    assert _chi2(cc, right) < 13.8  # 1e-3 tail, 2 degrees of freedom
    assert _chi2(cc, wrong) > 1000.0


@pytest.mark.parametrize("v", [1, 37, 1024, 1025, 100003])
def test_tokens_in_range_and_deterministic(v):
    x = np.random.default_rng(v).standard_normal((4, v)).astype(np.float32) * 3
    u = np.array([0.0, 0.25, 0.5, 0.999], np.float32)
    a = O.draw_rows(x, 0.9, u)
    assert np.all((a >= 0) & (a < v))
    assert np.array_equal(a, O.draw_rows(x, 0.9, u))
