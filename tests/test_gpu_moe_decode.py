"""moe_decode on the GPU against the fp64 exact-dequant oracle, plus the reference's bitwise invariances
(tests/t0/test_moe_gemv_affine.py:91-166 of the reference, at BASELINE and reference shapes)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd import _lib
from slotstream_spark_amd.kernels.moe_gemv_affine import moe_decode
from tests.gpu_util import DenseCache, make_pool, rand_ids, rand_weights, rand_x

pytestmark = pytest.mark.gpu

REL_FP64 = 1e-4          # the reference kernel's own bound vs fp64 (test_moe_gemv_affine.py:100)
CONTROL_RATIO = 10.0     # negative control must exceed 10x the limit (numeric_contract.toml:70)


def _run(pool, x, ids, w, layer=0):
    r, k = ids.shape
    dev = pool.device
    h = torch.full((r, k, pool.inter), float("nan"), device=dev)
    o = torch.full((r, k, pool.hidden), float("nan"), device=dev)
    out = torch.full((r, pool.hidden), float("nan"), device=dev)
    moe_decode(x.to(dev), ids.to(dev), w.to(dev), layer, pool.map, pool.slot_ptr, h, o, out,
               experts_per_layer=pool.experts)
    torch.cuda.synchronize()
    return h, o, out


@pytest.fixture(scope="module")
def pool_b():
    print("[moe_decode] BASELINE shape pool H=2048 I=512 E=64", flush=True)
    return make_pool(64, 2048, 512, seed=1729)


@pytest.fixture(scope="module")
def pool_ref():
    print("[moe_decode] reference shape pool H=2560 I=640 E=32", flush=True)
    return make_pool(32, 2560, 640, seed=77)


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("r,k", [(2, 10), (4, 10), (1, 4), (3, 16)])
def test_matches_fp64(pool_b, xdtype, r, k):
    x, ids, w = rand_x(r, 2048, 11 + r, xdtype), rand_ids(r, k, 64, 12 + r), rand_weights(r, k, 13 + r)
    h, o, out = _run(pool_b, x, ids, w)
    dense = DenseCache(pool_b)
    ref = O.moe_routed_fp64(x.float().numpy(), ids.numpy(), w.numpy(), dense)
    err = O.rel_l2(out.cpu().numpy(), ref)
    print(f"r={r} k={k} x={xdtype} rel_l2 vs fp64 {err:.3e}")
    assert err <= REL_FP64
    # h and o buffers hold the per-(row, rank) intermediates of the reference.
    xd = x.double().numpy()
    for t in range(r):
        for kk in range(k):
            g, u, d = dense(int(ids[t, kk]))
            hh = O.silu64(g @ xd[t]) * (u @ xd[t])
            assert O.rel_l2(h[t, kk].cpu().numpy(), hh) <= REL_FP64
            assert O.rel_l2(o[t, kk].cpu().numpy(), float(w[t, kk]) * (d @ hh)) <= REL_FP64
    # out is the sequential rank-order fp32 sum of o (kernels/fused_moe_affine.py:164-172), bit for bit.
    on = o.cpu().numpy()
    seq = on[:, 0].copy()
    for kk in range(1, k):
        seq = (seq + on[:, kk]).astype(np.float32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), seq.view(np.uint32))


def test_negative_control_nibble_swap(pool_b):
    x, ids, w = rand_x(2, 2048, 5), rand_ids(2, 10, 64, 6), rand_weights(2, 10, 7)
    _, _, out = _run(pool_b, x, ids, w)
    dense = DenseCache(pool_b)

    def swapped(e):
        pieces = O.unpack_record(dense.record(e), 2048, 512)
        res = []
        for q, s, b in pieces:
            by = q.view(np.uint8)
            qs = ((by >> 4) | ((by & 15) << 4)).astype(np.uint8).view(np.uint32).reshape(q.shape)
            res.append(O.dequant(qs, s, b, 64, np.float64))
        return tuple(res)

    ctrl = O.rel_l2(out.cpu().numpy(), O.moe_routed_fp64(x.float().numpy(), ids.numpy(), w.numpy(), swapped))
    print(f"nibble-swap control rel {ctrl:.3f}")
    assert ctrl > CONTROL_RATIO * REL_FP64


def test_reference_shape(pool_ref):
    x, ids, w = rand_x(3, 2560, 21), rand_ids(3, 10, 32, 22), rand_weights(3, 10, 23)
    _, _, out = _run(pool_ref, x, ids, w)
    ref = O.moe_routed_fp64(x.float().numpy(), ids.numpy(), w.numpy(), DenseCache(pool_ref))
    err = O.rel_l2(out.cpu().numpy(), ref)
    print(f"reference shape rel_l2 {err:.3e}")
    assert err <= REL_FP64


@pytest.mark.parametrize("r", [3, 6])
def test_row_invariance_and_duplicates(pool_b, r):
    x, ids, w = rand_x(r, 2048, 31), rand_ids(r, 10, 64, 32), rand_weights(r, 10, 33)
    ids[1] = ids[0]            # same experts in two rows
    ids[2, :5] = ids[0, :5]    # partial overlap
    _, o, out = _run(pool_b, x, ids, w)
    for t in range(r):
        _, o1, one = _run(pool_b, x[t:t + 1].contiguous(), ids[t:t + 1].contiguous(), w[t:t + 1].contiguous())
        assert torch.equal(one[0], out[t])
        assert torch.equal(o1[0], o[t])


def test_placement_bitwise(pool_b):
    """Moving records between slots changes no bit (test_moe_gemv_affine.py:103-116)."""
    x, ids, w = rand_x(2, 2048, 41), rand_ids(2, 10, 64, 42), rand_weights(2, 10, 43)
    _, _, ref = _run(pool_b, x, ids, w)
    moved = make_pool(64, 2048, 512, seed=1729, permute=False, layers=2)
    # Copy pool_b's records into layer 1 of another pool at a different placement.
    src_map = pool_b.map.cpu().tolist()
    perm = torch.randperm(64, generator=torch.Generator().manual_seed(9)).tolist()
    for e in range(64):
        moved.write_record(64 + perm[e], pool_b.record(src_map[e]))
    moved.assign(1, [64 + perm[e] for e in range(64)])
    _, _, out = _run(moved, x, ids, w, layer=1)
    assert torch.equal(out, ref)


def test_two_runs_identical(pool_b):
    x, ids, w = rand_x(4, 2048, 51), rand_ids(4, 10, 64, 52), rand_weights(4, 10, 53)
    assert torch.equal(_run(pool_b, x, ids, w)[2], _run(pool_b, x, ids, w)[2])


def test_bad_ids_raise_status_not_fault(pool_b):
    _lib.device_error(clear=True)
    x, ids, w = rand_x(2, 2048, 61), rand_ids(2, 10, 64, 62), rand_weights(2, 10, 63)
    ids[0, 3] = 64 + 7          # outside [0, E)
    _, o, out = _run(pool_b, x, ids, w)
    flags = _lib.device_error(clear=True)
    assert flags & 1
    assert float(o[0, 3].abs().max()) == 0.0
    assert torch.isfinite(out).all()


def test_validation_errors(pool_b):
    x, ids, w = rand_x(2, 2048, 1).cuda(), rand_ids(2, 10, 64, 2).cuda(), rand_weights(2, 10, 3).cuda()
    h = torch.empty(2, 10, 512, device="cuda")
    o = torch.empty(2, 10, 2048, device="cuda")
    out = torch.empty(2, 2048, device="cuda")
    with pytest.raises(ValueError):
        moe_decode(x, ids.long(), w, 0, pool_b.map, pool_b.slot_ptr, h, o, out)
    with pytest.raises(ValueError):
        moe_decode(x, ids, w, 0, pool_b.map, pool_b.slot_ptr, h, o[:, :9], out)
    with pytest.raises(ValueError):
        moe_decode(x, ids, w, 0, pool_b.map, pool_b.slot_ptr, h, o, out, cfg={"bk": 96})


def test_two_streams_overlap(pool_b):
    """Calls on two streams at once (each stream has its own slot of the static scratch): every result equals the
    same call run alone, bit for bit."""
    print("[moe_decode] two streams", flush=True)
    dev = pool_b.device
    cases = [(rand_x(4, 2048, seed), rand_ids(4, 8, pool_b.experts, seed + 1), rand_weights(4, 8, seed + 2))
             for seed in (11, 21)]
    alone = [_run(pool_b, *c)[2] for c in cases]
    cases = [tuple(t.to(dev) for t in c) for c in cases]
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    torch.cuda.synchronize()
    outs = []
    for _ in range(20):
        for st, (x, ids, w) in zip(streams, cases):
            with torch.cuda.stream(st):
                h = torch.empty((4, 8, pool_b.inter), device=dev)
                o = torch.empty((4, 8, pool_b.hidden), device=dev)
                out = torch.empty((4, pool_b.hidden), device=dev)
                moe_decode(x, ids, w, 0, pool_b.map, pool_b.slot_ptr, h, o, out, experts_per_layer=pool_b.experts)
                outs.append(out)
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        assert torch.equal(out, alone[i % 2]), i
