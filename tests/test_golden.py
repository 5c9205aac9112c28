"""The oracle against the golden fixtures written from the reference's own CPU path (tests/golden/make_golden.py:
model/reference_torch.py:118-134 moe_ref). CPU only.

What the fixtures show and this file pins:
  * router logits: the oracle's fixed-order fp32 dot + one bf16 rounding equals torch's CPU F.linear bit for bit
    on every fixture entry;
  * top-k ids: equal to moe_ref's torch.topk, except that torch.topk's CPU order inside a group of exactly equal
    probabilities is unspecified (case seed 5 returns 417 before 307 at equal logits); the path follows the
    reference kernel's rule (kernels/topk_stable.py:1-13, ties -> lower index), so ids are compared after putting
    each tie group of the fixture in index order;
  * y: the oracle's layer (fp64 exact-dequant routed experts, bf16 shared-expert chain) within 2e-2 relative.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc
from tests.golden import gen

FIX = Path(__file__).resolve().parent / "golden" / "moe_ref_cases.npz"
Z = np.load(FIX)  # allow_pickle stays False
META = json.loads(bytes(Z["meta"]).decode())
CASES = META["cases"]


def canonical_ids(ids, probs):
    """Each run of equal probabilities in a top-k row put in ascending index order."""
    out = ids.copy()
    for t in range(ids.shape[0]):
        row = list(ids[t])
        i = 0
        while i < len(row):
            j = i
            while j + 1 < len(row) and probs[t, row[j + 1]] == probs[t, row[i]]:
                j += 1
            row[i:j + 1] = sorted(row[i:j + 1])
            i = j + 1
        out[t] = row
    return out


@pytest.fixture(params=CASES, ids=lambda c: f"s{c['seed']}-T{c['T']}-E{c['E']}-K{c['K']}")
def case(request):
    c = request.param
    return c, gen.layer_inputs(c["seed"], c["T"], c["H"], c["E"], c["Is"])


def test_router_logits_bit_exact(case):
    c, (x, rw, *_) = case
    assert np.array_equal(orc.dense_rows(x, rw), Z[f"s{c['seed']}_logits"])


def test_topk_ids_match(case):
    c, (x, rw, *_) = case
    s = c["seed"]
    _, ids, _ = orc.router_topk(orc.dense_rows(x, rw), c["K"])
    ref = canonical_ids(Z[f"s{s}_ids"], Z[f"s{s}_probs"])
    assert np.array_equal(ids, ref)


def test_layer_output_within_tolerance(case):
    c, (x, rw, sg, su, sd, sgg) = case
    s, H, I = c["seed"], c["H"], c["I"]
    _, _, ids, w = orc.router(x, rw, c["K"])
    recs = {}
    routed = orc.moe_routed_fp64(orc.bf16_to_f32(x), ids, w,
                                 lambda e: recs.setdefault(e, orc.expert_dense(gen.record(s, e, H, I), H, I)))
    sh, sgl = orc.shared_expert(x, sg, su, sd, sgg)
    y = orc.bf16_to_f32(orc.combine_shared(routed.astype(np.float32), sh, sgl))
    ref = orc.bf16_to_f32(Z[f"s{s}_y"])
    err = orc.rel_l2(y, ref)
    assert err < 2e-2
    assert err < 1e-3  # observed <= 4e-5, with >99.9 % of the bf16 outputs bit-identical
    assert np.mean(orc.f32_to_bf16(y) == Z[f"s{s}_y"]) > 0.99


def test_fixture_metadata():
    assert META["source"].startswith("model/reference_torch.py")
    assert {c["E"] for c in CASES} == {64, 512}
