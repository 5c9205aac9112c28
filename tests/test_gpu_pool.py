"""The HBM expert slot pool fed from experts.bin (ssmoe_pool_*, ExpertPool) on the GPU: the reference's slotio
binding tests (tests/t0/test_slotio_bindings.py:69-199 of the reference: record bytes, duplicates, eviction after
progress, overwrite, Exhausted changes nothing, resize keeps survivors), an I/O error past the end of the file, the
pool against the bookkeeping model on a long seeded sequence, and moe_decode through the pool's tables bitwise
equal to the fully resident pool."""
import json

import numpy as np
import pytest
import torch

from oracle.pool_model import Exhausted as ModelExhausted, PoolModel
from slotstream_spark_amd import _lib
from slotstream_spark_amd.kernels.moe_gemv_affine import moe_decode
from slotstream_spark_amd.memory.expert_pool import ExpertPool, write_experts_bin
from tests.gpu_util import make_pool, rand_ids, rand_weights, rand_x

pytestmark = pytest.mark.gpu

REC = 65536   # synthetic record size (the reference test's)
NREC = 64     # records in the file: layer 0, experts 0..63; the manifest says 48 x 512
LAYERS = 48


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    print("[pool] experts.bin 64 x 64 KiB, manifest 48 x 512", flush=True)
    d = tmp_path_factory.mktemp("pool")
    data = np.random.default_rng(1234).integers(0, 256, size=NREC * REC, dtype=np.uint8)
    (d / "experts.bin").write_bytes(data.tobytes())
    (d / "experts.manifest.json").write_text(json.dumps(
        {"record_bytes": REC, "layers": LAYERS, "experts": 512, "alignment": 4096}))
    return d, data


def _rec(data, i):
    return data[i * REC:(i + 1) * REC]


def _device_records(ep, idxs):
    """The bytes of the slot each map entry names, copied back from HBM (moe_decode reads them on the device in
    the last test)."""
    m = ep.map.cpu().numpy()
    out = []
    for idx in idxs:
        s = int(m[idx])
        assert s >= 0, idx
        out.append(ep.pool.slot_view(s))
    return out


@pytest.mark.parametrize("lanes", [1, 4, 8])
def test_pool_bytes_duplicates_and_eviction(packed, lanes):
    d, data = packed
    ep = ExpertPool(d, 16, chunk_bytes=1 << 26, lanes=lanes)
    try:
        assert ep.stats()["lanes"] == lanes
        assert ep.layers == 49 and ep.map.numel() == 49 * 512    # the MTP layer shares the table
        ids = np.array([3, 9, 40, 9], dtype=np.int32)
        slots = ep.ensure(0, ids)
        assert slots[1] == slots[3]
        for e, s in zip(ids, slots):
            assert ep.pool.slot_view(int(s)).tobytes() == _rec(data, int(e)).tobytes(), (e, s)
        m = ep.map.cpu().numpy()
        assert [m[e] for e in (3, 9, 40)] == [slots[0], slots[1], slots[2]]
        ptr = ep.slot_ptr.cpu().numpy()
        assert len(set(ptr[:16].tolist())) == 16 and (ptr[16:] == 0).all()
        assert ep.last_timing["misses"] == 3 and ep.last_timing["hits"] == 0
        # progress passes the pins: every slot can be replaced
        prog = torch.zeros(1, dtype=torch.int64).pin_memory()
        prog[0] = 1000
        ep.set_progress_ptr(prog.data_ptr())
        more = np.arange(10, 26, dtype=np.int32)
        slots2 = ep.ensure(0, more, gen=2000)
        assert sorted(slots2.tolist()) == list(range(16))
        for e, b in zip(more, _device_records(ep, more.tolist())):
            assert b.tobytes() == _rec(data, int(e)).tobytes()
        assert ep.pool.map_numpy()[3] == -1     # evicted, not left stale
        assert ep.owned_bytes() == (1 << 26)
        assert ep.stats()["misses"] == 19 and ep.stats()["bytes"] == 19 * REC
    finally:
        ep.close()


def test_direct_reads(packed):
    """O_DIRECT reads (File.open_direct) give the same records; skipped where the file system refuses O_DIRECT."""
    d, data = packed
    ep = ExpertPool(d, 16, chunk_bytes=1 << 26, lanes=1)
    try:
        ep.set_reader(4, direct=True)
    except _lib.IoError as e:
        ep.close()
        pytest.skip(f"file system refuses O_DIRECT: {e}")
    ids = np.array([0, 17, 63, 5, 17], dtype=np.int32)
    slots = ep.ensure(0, ids, gen=1)
    for e, s in zip(ids, slots):
        assert ep.pool.slot_view(int(s)).tobytes() == _rec(data, int(e)).tobytes()
    assert ep.stats()["direct"] == 1
    ep.close()


def test_overwrite_slot(packed):
    d, data = packed
    ep = ExpertPool(d, 4, chunk_bytes=1 << 26)
    first = ep.ensure(0, np.array([1, 2, 3, 4], dtype=np.int32), gen=1)
    prog = torch.zeros(1, dtype=torch.int64).pin_memory()
    prog[0] = 2
    ep.set_progress_ptr(prog.data_ptr())
    second = ep.ensure(0, np.array([11, 12, 13, 14], dtype=np.int32), gen=2)
    assert set(second.tolist()) == set(first.tolist())
    for e, b in zip((11, 12, 13, 14), _device_records(ep, [11, 12, 13, 14])):
        assert b.tobytes() == _rec(data, e).tobytes()
    assert ep.pool.map_numpy()[1] == -1
    ep.close()


def test_exhausted_changes_nothing(packed):
    d, _ = packed
    ep = ExpertPool(d, 4, chunk_bytes=1 << 26)
    ep.ensure(0, np.array([1, 2, 3, 4], dtype=np.int32), gen=1)
    before = ep.pool.map_numpy().copy()
    with pytest.raises(_lib.Exhausted):
        ep.ensure(0, np.array([7], dtype=np.int32), gen=2)
    assert (ep.pool.map_numpy() == before).all()
    assert ep.stats()["pinned"] == 4
    ep.close()


def test_read_past_end_is_io_error_and_publishes_nothing(packed):
    d, data = packed
    ep = ExpertPool(d, 4, chunk_bytes=1 << 26)
    ep.ensure(0, np.array([1, 2], dtype=np.int32), gen=1)
    ep.retire_below(2)
    with pytest.raises(_lib.IoError):
        ep.ensure(0, np.array([5, 200], dtype=np.int32), gen=2)    # record 200 lies past the end of the file
    m = ep.pool.map_numpy()
    assert m[5] == -1 and m[200] == -1                            # nothing published
    assert ep.stats()["pinned"] == 0                              # pins restored
    s = ep.ensure(0, np.array([5, 6, 7, 8], dtype=np.int32), gen=3)
    for e, b in zip((5, 6, 7, 8), _device_records(ep, [5, 6, 7, 8])):
        assert b.tobytes() == _rec(data, e).tobytes()
    assert sorted(s.tolist()) == [0, 1, 2, 3]
    ep.close()


def test_resize_keeps_surviving_slots(packed):
    d, data = packed
    ep = ExpertPool(d, 8, chunk_bytes=1 << 26)
    slots = ep.ensure(0, np.array([5, 6], dtype=np.int32), gen=1)
    assert slots.tolist() == [0, 1]
    ep.resize_slots(20000 // 8)           # 2500 slots: three chunks of 1024
    assert ep.pool.chunks == 3
    assert ep.pool.slot_view(int(slots[0])).tobytes() == _rec(data, 5).tobytes()
    ep.resize_slots(8)
    assert ep.pool.slots == 8 and ep.pool.chunks == 1
    assert ep.pool.slot_view(int(slots[1])).tobytes() == _rec(data, 6).tobytes()
    ep.resize_slots(1)                    # shrinking below an owner unmaps it
    m = ep.pool.map_numpy()
    assert m[5] == 0 and m[6] == -1 and (m >= 0).sum() == 1
    ep.close()


def test_pool_follows_the_model_on_a_seeded_sequence(packed):
    """Slots, map and pins of the native pool equal the bookkeeping model's over 400 random operations: ensures
    with duplicates, hits and misses, capacity and CLOCK exhaustion, reads past the end, retires and resizes."""
    d, data = packed
    rng = np.random.default_rng(99)
    ep = ExpertPool(d, 12, chunk_bytes=1 << 20, max_slots=40)      # 16 slots per chunk
    model = PoolModel(49, 512, 40)
    model.resize(12)
    gen = 0
    outcomes = {"ok": 0, "exhausted": 0, "io": 0}
    for step in range(400):
        op = rng.random()
        if op < 0.08:
            n = int(rng.integers(1, 40))
            ep.resize_slots(n)
            model.resize(n)
        elif op < 0.25:
            prog = int(rng.integers(max(0, gen - 3), gen + 2))
            ep.retire_below(prog)
            model.retire_below(prog)
        else:
            gen += 1
            k = int(rng.integers(1, 9))
            hi = NREC + 4 if rng.random() < 0.1 else NREC        # now and then a record past the end of the file
            ids = rng.integers(0, hi, k).astype(np.int32)
            fail = bool((ids >= NREC).any())
            want = err = None
            try:
                want = model.ensure(0, ids.tolist(), gen, fail_read=fail)
            except ModelExhausted:
                err = _lib.Exhausted
            except IOError:
                err = _lib.IoError
            if err is None:
                got = ep.ensure(0, ids, gen=gen)
                assert got.tolist() == want, (step, ids)
                outcomes["ok"] += 1
            else:
                with pytest.raises(err):
                    ep.ensure(0, ids, gen=gen)
                outcomes["exhausted" if err is _lib.Exhausted else "io"] += 1
        assert ep.pool.map_numpy()[:512].tolist() == model.map[:512], step
        assert ep.stats()["pinned"] == model.pin_count, step
    assert min(outcomes.values()) > 0, outcomes
    m = ep.pool.map_numpy()[:512]
    for e in np.nonzero(m >= 0)[0][:8]:
        assert ep.pool.slot_view(int(m[e])).tobytes() == _rec(data, int(e)).tobytes()
    ep.close()


def test_moe_decode_through_pool_tables_is_bitwise_resident(tmp_path):
    """Experts loaded on demand into 24 slots feed moe_decode exactly as the fully resident pool does, also after
    eviction and reload."""
    print("[pool] moe_decode via ExpertPool H=2048 I=512 E=64", flush=True)
    H, I, E = 2048, 512, 64
    resident = make_pool(E, H, I, seed=31)
    m = resident.map.cpu().numpy()
    records = np.stack([resident.record(int(m[e])).cpu().numpy() for e in range(E)])[None]
    write_experts_bin(tmp_path, records)
    ep = ExpertPool(tmp_path, 24)
    assert (ep.hidden, ep.inter) == (H, I)
    dev = resident.device
    for batch in range(3):
        x, ids, w = rand_x(2, H, 70 + batch), rand_ids(2, 10, E, 80 + batch), rand_weights(2, 10, 90 + batch)
        ep.ensure(0, np.unique(ids.numpy()), gen=batch + 1)
        outs = []
        for pool in (resident, ep):
            h = torch.empty(2, 10, I, device=dev)
            o = torch.empty(2, 10, H, device=dev)
            out = torch.empty(2, H, device=dev)
            moe_decode(x.to(dev), ids.to(dev), w.to(dev), 0, pool.map, pool.slot_ptr, h, o, out, experts_per_layer=E)
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), batch
        ep.retire_below(batch + 2)
    assert ep.stats()["misses"] > 24    # later batches evicted and reloaded
    ep.close()
