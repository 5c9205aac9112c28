"""Pins the CPU oracle (oracle/) before anything is compared against it.

Every check here comes from outside the oracle's own formulas: fp64 arithmetic, torch's bf16 conversion,
brute-force restatements of the reference's specs (tests/t0/test_topk_stable.py:14-31, engine/sampler.py:83-84),
known answers (tests/t0/test_affine_kernels.py:35-38, the SplitMix64 published first output), or a
distributional invariant (p/q acceptance emits tokens distributed as p). CPU only.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as orc


def _ulp_diff(a, b):
    """Signed distance in units in the last place between fp32 arrays of one sign."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return ia - ib


# ---------------------------------------------------------------- exp
def test_expf_within_one_ulp_of_fp64():
    x = np.concatenate([
        np.linspace(-103.9, 88.7, 2_000_003, dtype=np.float32),
        np.random.default_rng(3).uniform(-30, 30, 500_000).astype(np.float32),
    ])
    got = orc.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)  # correctly rounded except at rare double-rounding ties
    d = np.abs(_ulp_diff(got, ref))
    assert d.max() <= 1, f"max ulp distance {d.max()} at x={x[d.argmax()]}"
    # The result never strays more than one ulp from the exact value, so it is faithfully rounded.
    exact = np.exp(x.astype(np.float64))
    up = np.nextafter(got, np.float32(np.inf)).astype(np.float64)
    dn = np.nextafter(got, np.float32(-np.inf)).astype(np.float64)
    fin = np.isfinite(got) & (got > 0)
    assert np.all((exact[fin] <= up[fin]) & (exact[fin] >= dn[fin]))


def test_expf_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 89.0, 1000.0, -104.0, -1000.0, 1.0], np.float32)
    y = orc.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
    assert y[5] == np.inf and y[6] == np.inf
    assert y[7] == 0.0 and y[8] == 0.0
    assert abs(int(_ulp_diff(y[9:10], np.float32(np.e))[0])) <= 1


def test_expf_subnormal_results():
    x = np.linspace(-103.0, -87.0, 100_001, dtype=np.float32)
    got = orc.expf(x).astype(np.float64)
    exact = np.exp(x.astype(np.float64))
    tiny = np.float64(2.0 ** -149)  # one subnormal ulp
    assert np.max(np.abs(got - exact)) <= tiny


# ---------------------------------------------------------------- bf16
def test_bf16_every_pattern_round_trips():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.bf16_to_f32(bits)
    back = orc.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(np.isnan(orc.bf16_to_f32(back[nan])))


def test_bf16_rounding_matches_torch_and_c():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    u = rng.integers(0, 2 ** 32, 400_000, dtype=np.uint64).astype(np.uint32)
    u[:50_000] = (u[:50_000] & 0xFFFF0000) | 0x8000  # exact ties: round half to even
    u[50_000:60_000] = (u[50_000:60_000] & 0xFFFF0000) | 0x7FFF
    f = u.view(np.float32)
    fin = np.isfinite(f)
    ours = orc.f32_to_bf16(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours[fin], ref[fin])
    L = orc.lib()
    L.or_f32_to_bf16.argtypes, L.or_f32_to_bf16.restype = [ctypes.c_float], ctypes.c_uint16
    sample = np.flatnonzero(fin)[::97]
    c = np.array([L.or_f32_to_bf16(float(f[i])) for i in sample], np.uint16)
    assert np.array_equal(c, ours[sample])


# ---------------------------------------------------------------- affine 4-bit
def test_unpack_known_answer():
    # tests/t0/test_affine_kernels.py:35-38: 0x76543210 unpacks low nibble first to 0..7.
    q = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert orc.unpack4(q).tolist() == [list(range(16))]


def test_dequant_closed_form():
    q = np.array([[0x76543210] * 8], dtype=np.uint32)  # 64 nibbles, one group
    s = orc.f32_to_bf16(np.array([[0.5]], np.float32))
    b = orc.f32_to_bf16(np.array([[-1.0]], np.float32))
    w = orc.dequant(q, s, b)
    assert w.tolist() == [[0.5 * (i % 8) - 1.0 for i in range(64)]]
    with pytest.raises(ValueError):
        orc.dequant(q, s, np.zeros((1, 2), np.uint16))


def test_record_offsets_match_baseline_table():
    offs, total = orc.record_offsets(2048, 512)
    assert offs == [0, 524288, 557056, 589824, 1114112, 1146880, 1179648, 1703936, 1736704]
    assert total == 1769472
    # The reference's own model shape (H 2560, I 640) has 2,764,800-byte records.
    assert orc.record_offsets(2560, 640)[1] == 2764800


def test_unpack_record_reads_every_piece():
    H, I = 128, 64
    offs, total = orc.record_offsets(H, I)
    rec = np.zeros(total, np.uint8)
    ends = offs[1:] + [total]
    for p, (a, e) in enumerate(zip(offs, ends)):
        rec[a:e] = p + 1  # each piece filled with its own byte
    pieces = orc.unpack_record(rec, H, I)
    for p, arr in enumerate(x for trio in pieces for x in trio):
        assert np.all(arr.view(np.uint8) == p + 1)


def test_nibble_swap_control_exceeds_tolerance():
    """Negative control: reading the nibbles high-first moves the routed output far beyond 2e-2."""
    rng = np.random.default_rng(9)
    H, I, E, K = 256, 128, 4, 2
    _, total = orc.record_offsets(H, I)
    recs = []
    for _ in range(E):
        rec = rng.integers(0, 256, total, dtype=np.uint8)
        for (q, s, b) in orc.unpack_record(rec, H, I):
            sv = orc.f32_to_bf16(np.abs(rng.normal(0, 0.02, s.shape)).astype(np.float32))
            s[...] = sv
            b[...] = orc.f32_to_bf16(-8 * orc.bf16_to_f32(sv))
        recs.append(rec)

    def swapped(rec):
        r = rec.copy()
        for (q, _, _) in orc.unpack_record(r, H, I):
            v = q.view(np.uint8)
            v[...] = ((v & 15) << 4) | (v >> 4)
        return r

    x = orc.bf16_to_f32(orc.f32_to_bf16(rng.normal(0, 1, (2, H)).astype(np.float32)))
    ids = np.array([[0, 1], [2, 3]], np.int32)
    w = np.array([[0.6, 0.4], [0.7, 0.3]], np.float32)
    good = orc.moe_routed_fp64(x, ids, w, lambda e: orc.expert_dense(recs[e], H, I))
    bad = orc.moe_routed_fp64(x, ids, w, lambda e: orc.expert_dense(swapped(recs[e]), H, I))
    assert orc.rel_l2(bad, good) > 10 * 2e-2


# ---------------------------------------------------------------- dense rows / router
def test_dense_rows_exact_on_integers():
    rng = np.random.default_rng(1)
    T, H, N = 3, 1024, 37
    x = rng.integers(-3, 4, (T, H)).astype(np.float32)
    w = rng.integers(-3, 4, (N, H)).astype(np.float32)
    got = orc.bf16_to_f32(orc.dense_rows(orc.f32_to_bf16(x), orc.f32_to_bf16(w)))
    exact = x.astype(np.float64) @ w.astype(np.float64).T  # |dot| < 2^24: every partial sum is exact in fp32
    assert np.array_equal(got, orc.bf16_to_f32(orc.f32_to_bf16(exact.astype(np.float32))))


def test_dense_rows_close_to_fp64():
    rng = np.random.default_rng(2)
    T, H, N = 4, 2048, 300
    xb = orc.f32_to_bf16(rng.normal(0, 1, (T, H)).astype(np.float32))
    wb = orc.f32_to_bf16(rng.normal(0, 0.02, (N, H)).astype(np.float32))
    got = orc.bf16_to_f32(orc.dense_rows(xb, wb)).astype(np.float64)
    exact = orc.bf16_to_f32(xb).astype(np.float64) @ orc.bf16_to_f32(wb).astype(np.float64).T
    assert np.all(np.abs(got - exact) <= np.abs(exact) * 2.0 ** -8 + 1e-6)  # one bf16 rounding
    # rows of w permute the outputs; x rows are independent
    perm = rng.permutation(N)
    assert np.array_equal(orc.dense_rows(xb, wb[perm]), orc.dense_rows(xb, wb)[:, perm])
    assert np.array_equal(orc.dense_rows(xb[1:2], wb), orc.dense_rows(xb, wb)[1:2])


def _brute_topk_desc(v, k):
    """Indices of the k largest values, ties to the lower index (stable sort of -v)."""
    return np.argsort(-v.astype(np.float64), kind="stable")[:k]


@pytest.mark.parametrize("E,K", [(64, 4), (512, 10), (300, 16)])
def test_router_topk_spec(E, K):
    rng = np.random.default_rng(E + K)
    T = 6
    logits = orc.f32_to_bf16(rng.normal(0, 1.5, (T, E)).astype(np.float32))
    logits[0, :] = logits[0, 0]  # all equal: ids 0..K-1
    logits[1, 5::7] = orc.f32_to_bf16(np.float32(9.0))  # ties among the top
    bias = rng.normal(0, 1, E).astype(np.float32)
    for b in (None, bias):
        probs, ids, w = orc.router_topk(logits, K, b)
        s = orc.bf16_to_f32(logits).astype(np.float64) + (0 if b is None else b.astype(np.float64))
        ref = np.exp(s - s.max(1, keepdims=True))
        ref /= ref.sum(1, keepdims=True)
        assert np.allclose(probs, ref, rtol=2e-6, atol=1e-12)
        for t in range(T):
            assert ids[t].tolist() == _brute_topk_desc(probs[t], K).tolist()
        assert np.allclose(w.sum(1), 1.0, atol=2e-6)
        assert np.allclose(w, probs[np.arange(T)[:, None], ids] / probs[np.arange(T)[:, None], ids].sum(1, keepdims=True),
                           rtol=1e-6)
    assert orc.router_topk(logits, K)[1][0].tolist() == list(range(K))
    big = np.zeros(E, np.float32)
    big[E - 1] = 50.0  # a large bias puts the last expert first on every row
    assert np.all(orc.router_topk(logits, K, big)[1][:, 0] == E - 1)


# ---------------------------------------------------------------- topk_stable (tests/t0/test_topk_stable.py:14-31)
def _keys(x):
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.int64)
    key = np.where(b >= 0x80000000, (~b) & 0xFFFFFFFF, b ^ 0x80000000)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, 0, key)


def _ref_row(x, k, nv):
    key = _keys(x[:nv])
    order = np.argsort(-key, kind="stable")[:k]
    sel = order if k <= 16 else np.sort(order)
    idx = np.full(k, -1, np.int64)
    idx[: sel.size] = sel
    return idx


def _check_topk(x, k, nv=None):
    idx, val = orc.topk_stable(x, k, nv)
    for r in range(x.shape[0]):
        n = x.shape[1] if nv is None else nv[r]
        ref = _ref_row(x[r], k, n)
        assert idx[r].tolist() == ref.tolist(), f"row {r}"
        ok = ref >= 0
        assert np.array_equal(val[r][ok].view(np.uint32), x[r][ref[ok]].view(np.uint32))
        assert np.all(np.isneginf(val[r][~ok]))
    return idx


@pytest.mark.parametrize("k", [1, 10, 16, 17, 100])
def test_topk_stable_random_with_ties(k):
    rng = np.random.default_rng(k)
    x = rng.integers(0, 5, (4, 700)).astype(np.float32)  # heavy ties
    _check_topk(x, k)
    _check_topk(rng.normal(size=(3, 513)).astype(np.float32), k)


def test_topk_stable_special_values():
    rng = np.random.default_rng(7)
    n = 512
    x = rng.normal(size=(4, n)).astype(np.float32)
    x[0, :20] = np.nan
    x[1, 5:15] = -np.inf
    x[1, 100:104] = np.inf
    x[2, ::2] = 0.0
    x[2, 1::2] = -0.0
    x[3, :] = np.nan
    for k in (10, 512):
        _check_topk(x, k)
    idx = orc.topk_stable(x, 10)[0]
    assert not set(idx[0].tolist()) & set(range(20))
    assert idx[1, :4].tolist() == [100, 101, 102, 103]
    assert idx[3].tolist() == list(range(10))
    assert idx[2].tolist() == list(range(0, 20, 2))


def test_topk_stable_n_valid():
    rng = np.random.default_rng(11)
    x = rng.integers(0, 4, (5, 2048)).astype(np.float32)
    x[:, 700:] = 1e9
    for k in (10, 40):
        nv = np.array([700, 700, 513, k, 3], np.int32)
        _check_topk(x, k, nv)


# ---------------------------------------------------------------- greedy acceptance (engine/generate.py:208-229)
def _greedy_brute(target, drafts):
    D = len(drafts)
    toks, good, flags = [], 0, 0
    for i in range(D + 1):
        row = target[i]
        if not np.all(np.isfinite(row)):
            flags = 1
            break
        t = int(np.argmax(row))
        toks.append(t)
        if i < D and t == drafts[i]:
            good += 1
            continue
        break
    return good, toks, flags


@pytest.mark.parametrize("seed", range(12))
def test_accept_greedy_brute_force(seed):
    rng = np.random.default_rng(seed)
    D, V = int(rng.integers(0, 6)), int(rng.integers(2, 50))
    target = rng.integers(0, 4, (D + 1, V)).astype(np.float32)  # ties: the first maximum wins
    drafts = np.array([int(np.argmax(target[i])) if rng.random() < 0.7 else int(rng.integers(0, V))
                       for i in range(D)], np.int32)
    if seed % 4 == 3 and D > 0:
        target[int(rng.integers(0, D + 1)), int(rng.integers(0, V))] = [np.nan, np.inf, -np.inf][seed % 3]
    out = orc.accept_greedy(target, drafts)
    good, toks, flags = _greedy_brute(target, drafts)
    assert out[0] == good and out[1] == len(toks) and out[2] == 0 and out[3] == flags
    assert out[4:4 + len(toks)].tolist() == toks
    assert np.all(out[4 + len(toks):] == -1)


# ---------------------------------------------------------------- p/q acceptance (Leviathan et al. 2023, Alg. 1)
def _softmax64(x, temp):
    a = x.astype(np.float64) / temp
    e = np.exp(a - a.max())
    return e / e.sum()


def test_accept_pq_emits_target_distribution():
    """Draft tokens x ~ q, accept with min(1, p/q), else resample from norm(max(0, p - q)): first token ~ p."""
    V, temp, n = 6, 0.7, 30_000
    tl = np.array([[1.0, 0.2, -0.5, 2.0, 0.0, -3.0], [0.3, 0.1, 0.0, -1.0, 1.0, 0.5]], np.float32)
    dl = np.array([[0.1, 1.5, 0.0, 0.5, -1.0, 0.0]], np.float32)
    p, q = _softmax64(tl[0], temp), _softmax64(dl[0], temp)
    u = orc.uniforms(2024, 3 * n).reshape(n, 3)
    xs = np.searchsorted(np.cumsum(q), np.random.default_rng(1).random(n), side="right").clip(0, V - 1)
    counts = np.zeros(V)
    acc = 0
    for i in range(n):
        out = orc.accept_pq(tl, dl, np.array([xs[i]], np.int32), u[i], temp)
        assert out[3] == 0
        counts[out[4]] += 1
        acc += out[0]
    chi2 = float(((counts - n * p) ** 2 / (n * p)).sum())
    assert chi2 < 25.0, (chi2, counts / n, p)  # 5 degrees of freedom: p-value ~1e-4
    expect_acc = float(np.minimum(p, q).sum())  # acceptance rate of Alg. 1
    assert abs(acc / n - expect_acc) < 0.015


def test_accept_pq_with_sampled_drafts_and_the_argmax_control():
    """The p/q path as wired, on the CPU: the draft drawn by the sampler's definition (orc.sample at the round's
    temperature, no filter, its own uniform), then accept_pq: the first token is distributed as p. The argmax draft
    (the greedy proposal) fed to the same rule over the same uniforms is biased towards the draft token, and the same
    chi-square check rejects it by far: the check can see that wiring mistake."""
    V, temp, n = 6, 0.7, 12_000
    tl = np.array([[1.2, 0.9, 0.2, -0.1, -0.8, 0.4], [0.1, 1.0, -0.5, 0.6, 0.3, -1.2]], np.float32)
    dl = np.array([[0.2, 1.6, 0.1, 0.3, -0.6, 0.9]], np.float32)
    p = _softmax64(tl[0], temp)
    u = orc.uniforms(77, 3 * n).reshape(n, 3)
    c_s, c_a = np.zeros(V), np.zeros(V)
    am = np.array([int(np.argmax(dl[0]))], np.int32)
    for i in range(n):
        x = orc.sample(dl[0], [], temp, 1.0, 0, 0.0, 0.0, u[i, 2])[0]
        c_s[orc.accept_pq(tl, dl, np.array([x], np.int32), u[i, :2], temp)[4]] += 1
        c_a[orc.accept_pq(tl, dl, am, u[i, :2], temp)[4]] += 1
    chi_s = float(((c_s - n * p) ** 2 / (n * p)).sum())
    chi_a = float(((c_a - n * p) ** 2 / (n * p)).sum())
    assert chi_s < 25.0, (chi_s, c_s / n, p)
    assert chi_a > 500.0, (chi_a, c_a / n, p)


def test_accept_pq_equal_distributions_always_accept():
    rng = np.random.default_rng(4)
    V, D = 50, 3
    t = rng.normal(0, 3, (D + 1, V)).astype(np.float32)
    d = t[:D].copy()
    for s in range(20):
        u = orc.uniforms(s, D + 1) * np.float32(0.999)
        drafts = rng.integers(0, V, D).astype(np.int32)
        out = orc.accept_pq(t, d, drafts, u, 0.7)
        assert out[0] == D and out[1] == D + 1 and out[2] == D + 1
        assert out[4:4 + D].tolist() == drafts.tolist()


def test_accept_pq_edge_cases():
    V = 8
    t = np.zeros((2, V), np.float32)
    d = np.zeros((1, V), np.float32)
    t[0, 3] = -200.0  # p(3) underflows to 0: a draft of 3 is always rejected and never resampled
    u = np.array([0.0, 0.5], np.float32)
    out = orc.accept_pq(t, d, np.array([3], np.int32), u, 1.0)
    assert out[0] == 0 and out[1] == 1 and out[4] != 3 and out[2] == 2 and out[3] == 0
    d2 = np.zeros((1, V), np.float32)
    d2[0, 5] = -200.0  # q(5) = 0 with p(5) > 0: always accepted
    out = orc.accept_pq(t, d2, np.array([5], np.int32), np.array([0.999, 0.1], np.float32), 1.0)
    assert out[0] == 1 and out[4] == 5
    out = orc.accept_pq(t, d, np.array([9], np.int32), u, 1.0)  # draft out of range
    assert out[3] & 2 and out[0] == 0
    tn = t.copy()
    tn[0, 0] = np.nan
    out = orc.accept_pq(tn, d, np.array([1], np.int32), u, 1.0)
    assert out[3] & 1 and out[1] == 0


def test_row_total_close_to_fp64():
    rng = np.random.default_rng(6)
    x = rng.normal(0, 3, 151936).astype(np.float32)
    temp = np.float32(0.7)
    a = (x / temp).astype(np.float64)
    ref = np.exp(a - a.max()).sum()
    assert abs(orc.row_z(x, temp) - ref) / ref < 1e-5


# ---------------------------------------------------------------- uniform stream (engine/sampler.py:20-24, :101-102)
def test_splitmix_known_answer():
    # First output of SplitMix64 (Steele, Lea, Flood 2014) from state 0.
    assert orc.splitmix(0) == 0xE220A8397B1DCDAF
    u = orc.uniforms(0, 2)  # seed 0 means 0xDEADBEEF (engine/sampler.py:73)
    st = orc.splitmix(0xDEADBEEF + 1)
    assert u[0] == np.float32((st >> 11) / 2.0 ** 53)
    assert np.all((orc.uniforms(5, 1000) >= 0) & (orc.uniforms(5, 1000) < 1))
