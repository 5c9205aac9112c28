"""The slot-pool model (oracle.pool_model, slotio clock.cpp / ensure.cpp restated) against sequences derived by
hand from the reference's rules, and the experts.bin manifest reader / writer (the fields of
tests/t0/test_repack_experts.py)."""
import ctypes
import json

import numpy as np
import pytest

from oracle.pool_model import Exhausted, PoolModel
from slotstream_spark_amd.memory.expert_pool import LAYOUT, PIECE_NAMES, read_manifest, write_experts_bin


def test_fill_then_clock_takes_slot_zero_after_clearing_every_reference_bit():
    m = PoolModel(2, 16, 8)
    m.resize(4)
    assert m.ensure(0, [1, 2, 3, 4], gen=1) == [0, 1, 2, 3]  # empty pool: the hand walks 0..3
    m.retire_below(2)
    # every slot has its reference bit (set at publish): one pass clears them, the hand comes back to slot 0
    assert m.ensure(0, [5], gen=2) == [0]
    assert m.map[1] == -1 and m.map[5] == 0 and m.hand == 1


def test_hit_sets_reference_bit_and_is_skipped_once():
    m = PoolModel(1, 16, 4)
    m.resize(4)
    m.ensure(0, [1, 2, 3, 4], gen=1)
    m.retire_below(2)
    m.ensure(0, [5], gen=2)          # takes slot 0, hand -> 1, refs of 1..3 cleared
    m.retire_below(3)
    m.ensure(0, [2], gen=3)          # hit on slot 1: reference bit set again
    m.retire_below(4)
    assert m.ensure(0, [6], gen=4) == [2]   # slot 1 is skipped once (bit cleared), slot 2 has no bit
    assert m.map[3] == -1 and m.map[2] == 1


def test_duplicates_pins_and_exhausted_change_nothing():
    m = PoolModel(1, 16, 4)
    m.resize(4)
    assert m.ensure(0, [7, 3, 7], gen=1) == [0, 1, 0]
    before = (list(m.map), list(m.pin_gen), m.pin_count, m.hand)
    with pytest.raises(Exhausted):
        m.ensure(0, [8, 9, 10], gen=2)   # 2 free slots, 2 pinned: 3 misses do not fit
    assert (list(m.map), list(m.pin_gen), m.pin_count, m.hand) == before
    assert m.ensure(0, [8, 9], gen=2) == [2, 3]
    assert m.pin_count == 4


def test_read_error_restores_pins_and_unmaps_victims():
    m = PoolModel(1, 16, 2)
    m.resize(2)
    m.ensure(0, [1, 2], gen=1)
    m.retire_below(2)
    with pytest.raises(IOError):
        m.ensure(0, [5], gen=2, fail_read=True)
    assert m.map[5] == -1 and m.map[1] == -1 and m.pin_count == 0   # victim unmapped, nothing published


def test_shrink_unmaps_and_unpins():
    m = PoolModel(1, 16, 8)
    m.resize(8)
    m.ensure(0, list(range(8)), gen=1)
    m.resize(3)
    assert [m.map[e] for e in range(8)] == [0, 1, 2, -1, -1, -1, -1, -1] and m.pin_count == 3


def test_manifest_writer_has_the_reference_fields(tmp_path):
    rec = np.random.default_rng(0).integers(0, 256, (3, 2, 1000), dtype=np.uint8)
    offs = [0, 100, 200, 300, 400, 500, 600, 700, 800]
    man = write_experts_bin(tmp_path, rec, piece_offsets=offs)
    data = (tmp_path / "experts.bin").read_bytes()
    assert len(data) == man["total_bytes"] == 3 * 2 * 1000
    assert man["layout"] == LAYOUT and man["version"] == 1 and man["alignment"] == 4096
    assert man["piece_names"] == PIECE_NAMES
    assert man["pieces"] == [int(x) for x in np.diff(man["piece_offsets"] + [1000])]
    assert data[(2 * 2 + 1) * 1000:(2 * 2 + 2) * 1000] == rec[2, 1].tobytes()
    assert read_manifest(tmp_path)["record_bytes"] == 1000


def test_manifest_reader_rejects_foreign_layouts(tmp_path):
    (tmp_path / "experts.manifest.json").write_text(json.dumps(
        {"record_bytes": 10, "layers": 1, "experts": 1, "layout": "something-else"}))
    with pytest.raises(ValueError, match="layout"):
        read_manifest(tmp_path)
    (tmp_path / "experts.manifest.json").write_text(json.dumps({"record_bytes": 10, "layers": 1}))
    with pytest.raises(ValueError, match="experts"):
        read_manifest(tmp_path)
    (tmp_path / "experts.manifest.json").write_text(json.dumps(
        {"record_bytes": 10, "layers": 1, "experts": 1, "piece_offsets": [0, 5, 20]}))
    with pytest.raises(ValueError, match="piece offsets"):
        read_manifest(tmp_path)


def test_pool_capi_rejects_bad_arguments(tmp_path):
    from slotstream_spark_amd import _lib
    L = _lib.lib()
    h = ctypes.c_void_p()
    p = ctypes.c_void_p(4096)
    assert L.ssmoe_pool_open(None, 1, 1, 10, 4, 100, p, p, ctypes.byref(h)) == 1
    assert L.ssmoe_pool_open(b"/x", 0, 1, 10, 4, 100, p, p, ctypes.byref(h)) == 1
    assert L.ssmoe_pool_open(b"/x", 1, 1, 10, 4, 5, p, p, ctypes.byref(h)) == 1   # chunk smaller than a record
    assert L.ssmoe_pool_open(str(tmp_path / "missing.bin").encode(), 1, 1, 10, 4, 100, p, p,
                             ctypes.byref(h)) == 4 and b"cannot open" in L.ssmoe_last_error()
    assert L.ssmoe_pool_resize(None, 3) == 1
    assert L.ssmoe_pool_set_reader(None, 4, 0) == 1
    assert L.ssmoe_pool_ensure(None, 0, None, 0, 1, None, None) == 1
