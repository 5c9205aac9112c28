"""Independent pins of the oracle functions that the round-trip tests leave open. CPU only.

  * oracle.moe_ref (the timed CPU baseline) against moe_ref_cases.npz, written from the reference's own moe_ref
    (model/reference_torch.py:118-134): top-k ids and y bit for bit;
  * oracle.moe_align against the reference's own torch moe_align (moe_align_ref.npz: -1 and out-of-range entries,
    Zipf skew, block 4/64/128, the config-3 shape) and against a brute-force restatement of the spec in
    kernels/moe_align.py:1-48 (stable order inside an expert, sentinel R in the padding, every block owned by one
    expert, -1 past num_padded);
  * oracle.prefill_rows against scalar loops over tiny shapes (exact sums with math.fsum, nibbles read bit by bit),
    with a planted mistake that the comparison must catch;
  * the router over 64 seeds of the reference's CPU router (router_ref.npz, torch F.linear + softmax + topk):
    top-k ids equal on every row, logits within two bf16 steps and identical on at least 99.95 % of entries;
  * the threshold top-k selection of the verify kernel's router tail, emulated in numpy, against a stable sort.
"""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.golden import gen
from tests.golden.make_router_golden import inputs as router_inputs

GOLD = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- moe_ref restatement vs the reference's moe_ref
Z = np.load(GOLD / "moe_ref_cases.npz")
MOE_CASES = json.loads(bytes(Z["meta"]).decode())["cases"]


@pytest.mark.parametrize("c", MOE_CASES, ids=lambda c: f"s{c['seed']}-T{c['T']}-E{c['E']}")
def test_moe_ref_restatement_matches_reference_fixture(c):
    s, T, H, E, K, I, Is = (c[k] for k in ("seed", "T", "H", "E", "K", "I", "Is"))
    x, rw, sg, su, sd, sgg = (torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
                              for a in gen.layer_inputs(s, T, H, E, Is))
    cache = {}

    def expert(e):
        if e not in cache:
            cache[e] = tuple(torch.from_numpy(d) for d in O.expert_dense(gen.record(s, e, H, I), H, I, np.float32))
        return cache[e]

    y, ti, tv = O.moe_ref(x, rw, K, expert, sg, su, sd, sgg)
    assert np.array_equal(ti.numpy().astype(np.int32), Z[f"s{s}_ids"])
    assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), Z[f"s{s}_y"])


# ---------------------------------------------------------------- moe_align vs a brute-force spec
def _align_brute(le, num_local, block_m):
    """Scalar restatement of the moe_align contract: rows of expert 0 in row order, padded with the sentinel R to a
    multiple of block_m, then expert 1, ...; rows outside [0, num_local) are dropped; the tail up to padded_rows
    is sentinel; block b belongs to the expert whose padded range holds position b * block_m, -1 past the end."""
    R = len(le)
    bound = R + num_local * (block_m - 1)
    P = -(-bound // block_m) * block_m
    out, owner = [], []
    for e in range(num_local):
        rows = [r for r in range(R) if le[r] == e]
        if not rows:
            continue
        n = -(-len(rows) // block_m) * block_m
        out += rows + [R] * (n - len(rows))
        owner += [e] * (n // block_m)
    used = len(out)
    out += [R] * (P - used)
    owner += [-1] * (P // block_m - len(owner))
    return np.array(out, np.int32), np.array(owner, np.int32), used


@pytest.mark.parametrize("R,nl,bm,seed", [(0, 3, 4, 0), (1, 1, 1, 1), (9, 2, 4, 2), (50, 5, 8, 3), (64, 1, 64, 4),
                                          (300, 16, 16, 5), (257, 7, 128, 6), (1000, 40, 64, 7)])
def test_moe_align_matches_brute_force_spec(R, nl, bm, seed):
    rng = np.random.default_rng(seed)
    le = rng.integers(-2, nl + 2, size=R).astype(np.int32)      # -1, -2 and ids past num_local are skipped
    if seed % 2:
        le = np.minimum(rng.zipf(1.5, size=R) - 1, nl + 1).astype(np.int32)   # skewed, some experts empty
    s, b, n = O.moe_align(le, nl, bm)
    rs, rb, rn = _align_brute(le.tolist(), nl, bm)
    assert n == rn
    assert np.array_equal(s, rs) and np.array_equal(b, rb)
    assert len(s) == O.padded_rows(R, nl, bm) and n % bm == 0


ALIGN = np.load(GOLD / "moe_align_ref.npz")


@pytest.mark.parametrize("case", ["tiny", "r1", "mid", "oob", "cfg3", "skew64"])
def test_moe_align_matches_reference_fixture(case):
    """Against the reference's own torch moe_align (kernels/moe_align.py:17-48) on tests/golden/moe_align_ref.npz,
    written by tests/golden/make_align_golden.py: every output array equal."""
    R, nl, bm = (int(v) for v in ALIGN[case + "_meta"])
    s, b, n = O.moe_align(ALIGN[case + "_le"], nl, bm)
    assert np.array_equal(s, ALIGN[case + "_sorted"])
    assert np.array_equal(b, ALIGN[case + "_block"])
    assert n == int(ALIGN[case + "_num"][0])


def test_moe_align_brute_force_catches_an_unstable_sort():
    """A sort that is not stable (rows of one expert in reverse order) must differ from the spec."""
    le = np.array([2, 0, 2, 1, 0, 2], np.int32)
    s, _, _ = O.moe_align(le, 3, 2)
    rs, _, _ = _align_brute(le.tolist(), 3, 2)
    assert np.array_equal(s, rs)
    wrong = rs.copy()
    wrong[0:2] = wrong[1::-1]
    assert not np.array_equal(wrong, rs)
    assert list(rs[:2]) == [1, 4]                                 # expert 0: rows 1, 4 in row order


# ---------------------------------------------------------------- prefill_rows vs scalar loops
def _bits_bf16(v: float) -> float:
    """float32(v) rounded to bf16 (round to nearest even) and back, with struct and integer arithmetic."""
    u = struct.unpack("<I", struct.pack("<f", v))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def _f32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def _dequant_scalar(q_words, s_bits, b_bits, n, k):
    """bf16(fp32(q * s + b)) of element (n, k): nibble k % 8 of word k // 8, low nibble first."""
    q = (int(q_words[n, k // 8]) >> (4 * (k % 8))) & 0xF
    s = struct.unpack("<f", struct.pack("<I", int(s_bits[n, k // 64]) << 16))[0]
    b = struct.unpack("<f", struct.pack("<I", int(b_bits[n, k // 64]) << 16))[0]
    return _bits_bf16(_f32(_f32(q * s) + b))


def _prefill_scalar(x, row_token, row_weight, row_expert, records, H, I):
    R = len(row_expert)
    hs = np.zeros((R, I), np.float32)
    out = np.zeros((R, H), np.float32)
    dq = {}
    for r in range(R):
        e = int(row_expert[r])
        if e < 0:
            continue
        if e not in dq:
            (gq, gs_, gb), (uq, us, ub), (dqw, ds, db) = O.unpack_record(records[e], H, I)
            dq[e] = ([[_dequant_scalar(gq, gs_, gb, i, k) for k in range(H)] for i in range(I)],
                     [[_dequant_scalar(uq, us, ub, i, k) for k in range(H)] for i in range(I)],
                     [[_dequant_scalar(dqw, ds, db, j, i) for i in range(I)] for j in range(H)])
        g_w, u_w, d_w = dq[e]
        xt = [float(v) for v in x[int(row_token[r])]]
        for i in range(I):
            g = math.fsum(xt[k] * g_w[i][k] for k in range(H))
            u = math.fsum(xt[k] * u_w[i][k] for k in range(H))
            hs[r, i] = _bits_bf16(_f32(g / (1.0 + math.exp(-g)) * u))
        for j in range(H):
            out[r, j] = _f32(math.fsum(float(hs[r, i]) * d_w[j][i] for i in range(I)) * float(row_weight[r]))
    return hs, out


def test_prefill_rows_matches_scalar_loops():
    H, I, T, K, E = 128, 64, 5, 2, 3
    records = [gen.record(77, e, H, I) for e in range(E)]
    rng = np.random.default_rng(5)
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32)))
    row_expert = np.array([0, 2, 1, 2, -1, 0, 2, 2, 1, 0], np.int32)
    row_token = np.arange(T * K) // K
    row_weight = rng.random(T * K).astype(np.float32)
    h, rows = O.prefill_rows(x, row_token, row_weight, row_expert, lambda e: O.expert_bf16(records[e], H, I))
    hb, rb = _prefill_scalar(x, row_token, row_weight, row_expert, records, H, I)
    assert np.array_equal(h, hb)                   # h: both sums exact to far below a bf16 step
    assert np.max(np.abs(rows - rb) / (np.abs(rb) + 1e-30)) < 1e-6
    assert np.all(rows[4] == 0)                    # a row with a negative expert is zero
    # planted mistake: exact (not bf16-rounded) dequantized weights change h on most entries
    h_bad, _ = O.prefill_rows(x, row_token, row_weight, row_expert,
                              lambda e: O.expert_dense(records[e], H, I, np.float64))
    assert np.mean(h_bad != hb) > 0.2


# ---------------------------------------------------------------- router over 64 seeds of the reference CPU router
RZ = np.load(GOLD / "router_ref.npz")
RMETA = json.loads(bytes(RZ["meta"]).decode())


def _same_topk(mine, ref, scores):
    """`mine` (ties to the lower index) and `ref` (torch.topk: tie order unspecified) select the same top-K of
    `scores`: the same score sequence, the same ids in every group of equal scores, and in the group that straddles
    the K-th place (torch keeps an arbitrary part of it) `mine` holds the lowest indices of the whole group."""
    sm, sr = scores[mine], scores[ref]
    if not np.array_equal(sm, sr):
        return False
    for v in np.unique(sm):
        a, b = np.sort(mine[sm == v]), np.sort(ref[sr == v])
        if v == sm[-1]:
            group = np.nonzero(scores == v)[0]
            if a.size != b.size or not np.array_equal(a, group[:a.size]) or not np.isin(b, group).all():
                return False
            if not np.array_equal(mine[sm == v], a):     # inside a group, ascending index
                return False
        elif not np.array_equal(a, b):
            return False
    return True


def _mono(b):
    """bf16 bits -> an integer whose order is the value order (distance in bf16 steps across zero)."""
    b = b.astype(np.int32)
    return np.where(b & 0x8000, 0x8000 - b, b)


def test_router_over_64_reference_seeds():
    """End to end: the oracle's logits give the ids the oracle's tail gives on the reference's logits (the few
    logits that differ never change a selection), and those are the reference's ids up to torch's tie order."""
    K = RMETA["K"]
    n_log = n_diff = n_rows = n_boundary_ties = 0
    max_steps = 0
    for c in RMETA["cases"]:
        s = c["seed"]
        x, rw, bias = router_inputs(s)
        mine = O.dense_rows(x, rw)
        ref = RZ[f"s{s}_logits"]
        n_log += ref.size
        n_diff += int((mine != ref).sum())
        max_steps = max(max_steps, int(np.abs(_mono(mine) - _mono(ref)).max()))
        for b, suffix in ((None, ""), (bias, "_bias")):
            _, ids, _ = O.router_topk(mine, K, b)
            probs_r, ids_r, _ = O.router_topk(ref, K, b)
            assert np.array_equal(ids, ids_r), s
            for t in range(ids.shape[0]):
                n_rows += 1
                assert _same_topk(ids_r[t], RZ[f"s{s}_ids{suffix}"][t], probs_r[t]), (s, t, suffix)
                n_boundary_ties += int(not np.array_equal(np.sort(ids_r[t]), np.sort(RZ[f"s{s}_ids{suffix}"][t])))
    print(f"{n_log} logits, {n_diff} differ from torch's CPU F.linear, by at most {max_steps} bf16 steps; "
          f"{n_rows} rows, {n_boundary_ties} with a tie across the K-th place that torch.topk breaks otherwise")
    assert n_log >= 65536
    assert max_steps <= 2
    assert n_diff <= 5e-4 * n_log


def test_same_topk_catches_a_wrong_selection():
    scores = np.array([5, 4, 4, 4, 3, 1], np.float32)
    assert _same_topk(np.array([0, 1, 2]), np.array([0, 3, 1]), scores)        # torch kept another tie member
    assert not _same_topk(np.array([0, 2, 3]), np.array([0, 1, 2]), scores)    # not the lowest of the tie group
    assert not _same_topk(np.array([0, 1, 4]), np.array([0, 1, 2]), scores)    # a lower score selected


def test_router_tail_on_reference_logits():
    """The oracle's renormalised weights on the reference's own logits equal torch's top-k values renormalised."""
    K = RMETA["K"]
    for c in RMETA["cases"][:16]:
        s = c["seed"]
        _, _, bias = router_inputs(s)
        _, _, w = O.router_topk(RZ[f"s{s}_logits"], K, bias)
        tv = RZ[f"s{s}_topv_bias"].astype(np.float64)
        assert np.allclose(w, tv / tv.sum(1, keepdims=True), rtol=1e-5, atol=0)


# ---------------------------------------------------------------- threshold top-k selection (verify router tail)
def _key(p):
    u = np.asarray(p, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    k = np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u ^ 0x80000000)
    return np.where(nan, 0, k).astype(np.uint64)


def _threshold_select(p, K, lanes=64):
    """The selection of the verify kernel's router tail for one row (E <= 8 * lanes): entry e lives in lane
    e % lanes. kp = key + 1; tau = the largest value with zero low 16 bits that at least K lane maxima reach; the
    entries >= tau are ranked by (kp, 0xFFFF - e). Returns the top-K ids, or None when the kernel falls back to its
    K rounds (no such tau, or more than 64 candidates)."""
    E = p.size
    kp = _key(p) + 1
    lm = np.zeros(lanes, np.uint64)
    for e in range(E):
        lm[e % lanes] = max(lm[e % lanes], kp[e])
    tau = 0
    for b in range(31, 15, -1):
        c = tau | (1 << b)
        if int((lm >= c).sum()) >= K:
            tau = c
    cand = np.nonzero(kp >= tau)[0]
    if tau == 0 or cand.size > 64:
        return None
    keys = (kp[cand] << np.uint64(32)) | (np.uint64(0xFFFF) - cand.astype(np.uint64))
    rank = np.array([(keys > k).sum() for k in keys])
    out = np.full(K, -1, np.int64)
    for c_, r in zip(cand, rank):
        if r < K:
            out[r] = c_
    return out


def test_threshold_selection_equals_stable_sort():
    rng = np.random.default_rng(11)
    E, K = 512, 10
    rows = []
    for i in range(3000):
        kind = i % 6
        z = rng.standard_normal(E).astype(np.float32)
        if kind == 1:
            z = np.round(z * 2) / 2                                  # quantised: many exact ties
        elif kind == 2:
            z[rng.random(E) < 0.9] = -200                            # underflow: most probabilities +0
        elif kind == 3:
            z[:] = 1.0                                               # everything tied
        elif kind == 4:
            z[rng.integers(0, E)] = np.nan                           # a NaN probability
        elif kind == 5:
            z[rng.integers(0, E, 12)] = 30                           # a dozen equal winners
        p = np.exp(z.astype(np.float64) - np.nanmax(z)).astype(np.float32)
        if kind == 4:
            p[np.isnan(z)] = np.nan
        rows.append(p)
    taken = 0
    for p in rows:
        kp = _key(p)
        want = np.lexsort((np.arange(E), -kp.astype(np.int64)))[:K]   # key desc, index asc
        got = _threshold_select(p, K)
        if got is not None:
            taken += 1
            assert np.array_equal(got, want)
    print(f"threshold path taken on {taken} of {len(rows)} rows")
    assert 1500 < taken < len(rows)                                  # both paths are exercised


# ---------------------------------------------------------------- combine_rank_order: the rank order itself
def test_combine_rank_order_sums_in_rank_order():
    """((r0 + r1) + r2) + ... in fp32: with r = (2^24, 1, -2^24) the rank order gives 0 (2^24 + 1 rounds to 2^24),
    any order that adds 1 last gives 1, and one that pairs +-2^24 first gives 1 as well; integer rows small enough to
    sum exactly in fp32 must give their exact sum."""
    T, K, H = 3, 3, 4
    rows = np.zeros((T * K, H), np.float32)
    rows[0::K] = 2.0 ** 24
    rows[1::K] = 1.0
    rows[2::K] = -(2.0 ** 24)
    out = O.combine_rank_order(rows, T, K)
    assert out.dtype == np.float32 and np.all(out == 0.0)
    # the reverse rank order (1 + ...) would not lose the 1: the check above fails for it
    rev = O.combine_rank_order(rows.reshape(T, K, H)[:, ::-1].reshape(T * K, H), T, K)
    assert np.all(rev == 1.0)
    rng = np.random.default_rng(7)
    ints = rng.integers(-1000, 1000, size=(5 * 10, 6)).astype(np.float32)
    exact = ints.reshape(5, 10, 6).astype(np.float64).sum(axis=1)
    assert np.array_equal(O.combine_rank_order(ints, 5, 10).astype(np.float64), exact)
