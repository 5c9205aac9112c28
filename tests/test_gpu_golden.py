"""The HIP path against the golden fixtures written from the reference's CPU moe_ref
(model/reference_torch.py:118-134, tests/golden/make_golden.py): router logits bit for bit, top-k ids equal (tie
groups of the fixture in index order, the reference kernel's rule, kernels/topk_stable.py:1-13), y within the
north-star bound of 2e-2 relative."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.engine.verify import MoEVerifyLayer
from slotstream_spark_amd.kernels.router import route
from slotstream_spark_amd.memory.slot_pool import SlotPool
from tests.golden import gen
from tests.gpu_util import bits
from tests.test_golden import canonical_ids

pytestmark = pytest.mark.gpu

Z = np.load(Path(__file__).resolve().parent / "golden" / "moe_ref_cases.npz")
CASES = json.loads(bytes(Z["meta"]).decode())["cases"]


def _bf16(a):
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()


@pytest.mark.parametrize("c", CASES, ids=lambda c: f"s{c['seed']}-T{c['T']}-E{c['E']}-K{c['K']}")
def test_hip_layer_matches_moe_ref_fixture(c):
    s, T, H, E, K, I, Is = (c[k] for k in ("seed", "T", "H", "E", "K", "I", "Is"))
    print(f"[golden] seed {s} T={T} E={E} K={K}", flush=True)
    x, rw, sg, su, sd, sgg = (_bf16(a) for a in gen.layer_inputs(s, T, H, E, Is))
    ref_ids = canonical_ids(Z[f"s{s}_ids"], Z[f"s{s}_probs"])
    pool = SlotPool(1, E, H, I)
    pool.storage.zero_()
    pool.place_permuted(s + 1732)
    slots = pool.map.cpu().numpy()
    for e in np.unique(ref_ids):  # only the selected experts are ever read
        pool.write_record(int(slots[e]), torch.from_numpy(gen.record(s, int(e), H, I)).cuda())
    logits = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
    ids_r, _ = route(x, rw, K, logits=logits)
    layer = MoEVerifyLayer(pool, 0, rw, sg, su, sd, sgg, top_k=K)
    y, ids, _ = layer(x)
    torch.cuda.synchronize()
    assert np.array_equal(bits(logits), Z[f"s{s}_logits"])
    assert np.array_equal(ids_r.cpu().numpy(), ref_ids)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    ref_y = O.bf16_to_f32(Z[f"s{s}_y"])
    err = O.rel_l2(O.bf16_to_f32(bits(y)), ref_y)
    same = float(np.mean(bits(y) == Z[f"s{s}_y"]))
    print(f"y rel_l2 {err:.3e}; bf16 bits equal {same:.4f}")
    assert err <= 2e-2


RZ = np.load(Path(__file__).resolve().parent / "golden" / "router_ref.npz")
RCASES = json.loads(bytes(RZ["meta"]).decode())["cases"]


@pytest.fixture(scope="module")
def zero_pool():
    pool = SlotPool(1, 512, 2048, 512)
    pool.storage.zero_()                     # zero records: the experts contribute nothing, routing is unchanged
    pool.place_permuted(9)
    return pool


def test_router_64_reference_seeds_on_gpu(zero_pool):
    """ssmoe_router and the verify kernel's router phase against the oracle on the 64 seeds of router_ref.npz, with
    and without the Zipf bias: logits bit for bit, ids and weights bit for bit (the oracle's ids are pinned to the
    reference's torch CPU router, up to torch's tie order, by tests/test_oracle_pins.py)."""
    from tests.golden.make_router_golden import inputs

    K = 10
    for c in RCASES:
        s = c["seed"]
        xb, rwb, bias = inputs(s)
        x, rw, b = _bf16(xb), _bf16(rwb), torch.from_numpy(bias).cuda()
        want_logits = O.dense_rows(xb, rwb)
        for bb in (None, b):
            logits = torch.empty((xb.shape[0], 512), dtype=torch.bfloat16, device="cuda")
            ids, w = route(x, rw, K, bb, logits=logits)
            zs = torch.zeros((512, 2048), dtype=torch.bfloat16, device="cuda")
            layer = MoEVerifyLayer(zero_pool, 0, rw, zs, zs, torch.zeros((2048, 512), dtype=torch.bfloat16,
                                                                          device="cuda"),
                                   torch.zeros((1, 2048), dtype=torch.bfloat16, device="cuda"), top_k=K,
                                   router_bias=bb)
            _, vids, vw = layer(x)
            torch.cuda.synchronize()
            _, rids, rwt = O.router_topk(want_logits, K, None if bb is None else bias)
            assert np.array_equal(bits(logits), want_logits), s
            for got_i, got_w in ((ids, w), (vids, vw)):
                assert np.array_equal(got_i.cpu().numpy(), rids), s
                assert np.array_equal(got_w.cpu().numpy().view(np.uint32), rwt.view(np.uint32)), s
