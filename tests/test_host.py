"""Host-side logic on the CPU: the uniform stream, the acceptance bookkeeping, the slot-pool tables and record
packing, and the synthetic generators' shapes."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from slotstream_spark_amd import _lib
from slotstream_spark_amd.engine.accept import AcceptResult, RoundStats, UniformStream
from slotstream_spark_amd.memory import synth
from slotstream_spark_amd.memory.slot_pool import SlotPool, pack_record

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="libssmoe.so not built")


def test_uniform_stream_matches_sampler_stream():
    s = UniformStream(0)
    assert s.state == 0xDEADBEEF  # engine/sampler.py:73 (seed 0 -> 0xDEADBEEF)
    assert np.array_equal(s.peek(50), orc.uniforms(0, 50))
    s7 = UniformStream(7)
    first = s7.peek(10)
    s7.advance(3)
    assert np.array_equal(s7.peek(7), first[3:])


def test_accept_result_and_round_stats():
    r = AcceptResult.from_out([2, 3, 3, 0, 11, 12, 13, -1])
    assert (r.n_accept, r.n_emit, r.tokens) == (2, 3, [11, 12, 13])
    st = RoundStats()
    st.add(3, r)                                   # accepted 2 of 3: depth 3 was attempted and rejected
    st.add(3, AcceptResult(0, 1, 1, 0, [5]))       # rejected at depth 1
    st.add(3, AcceptResult(3, 4, 4, 0, [1, 2, 3, 4]))
    assert st.rounds == 3 and st.drafted == 9 and st.accepted == 5
    assert st.attempts_by_depth == [3, 2, 2] and st.accepted_by_depth == [2, 2, 1]
    assert st.acceptance_length == pytest.approx(8 / 3)


@needs_lib
def test_slot_pool_tables_and_placement():
    pool = SlotPool(layers=2, experts=8, hidden=128, inter=128, device="cpu")
    assert pool.stride % 256 == 0 and pool.stride >= pool.record_bytes
    base = pool.storage.data_ptr()
    assert pool.slot_ptr.tolist() == [base + s * pool.stride for s in range(16)]
    assert torch.all(pool.map == -1)
    pool.place_permuted(1732)
    for layer in range(2):
        blk = pool.map[layer * 8:(layer + 1) * 8].tolist()
        assert sorted(blk) == list(range(layer * 8, layer * 8 + 8))
    with pytest.raises(ValueError):
        pool.assign(0, [0, 1, 2])


@needs_lib
def test_pack_record_matches_oracle_reading():
    H, I = 128, 64
    g = torch.Generator().manual_seed(3)
    def piece(n, k):
        q = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), generator=g, dtype=torch.int64).to(torch.int32)
        s = torch.rand(n, k // 64, generator=g).to(torch.bfloat16)
        b = -torch.rand(n, k // 64, generator=g).to(torch.bfloat16)
        return q, s, b
    gate, up, down = piece(I, H), piece(I, H), piece(H, I)
    rec = pack_record(gate, up, down, H, I)
    got = orc.unpack_record(rec.numpy(), H, I)
    for (q, s, b), (oq, os_, ob) in zip((gate, up, down), got):
        assert np.array_equal(q.numpy().view(np.uint32), oq)
        assert np.array_equal(s.view(torch.int16).numpy().view(np.uint16), os_)
        assert np.array_equal(b.view(torch.int16).numpy().view(np.uint16), ob)


@needs_lib
def test_fill_random_statistics():
    pool = SlotPool(layers=1, experts=4, hidden=256, inter=128, device="cpu")
    pool.fill_random(1729)
    for slot in range(4):
        (gq, gs, gb), _, _ = orc.unpack_record(pool.record(slot).numpy(), 256, 128)
        s = orc.bf16_to_f32(gs)
        assert np.all(s >= 0) and 0.005 < s.mean() < 0.03
        assert np.array_equal(orc.bf16_to_f32(gb), -8 * s)  # b = -8 s exactly in bf16
        nib = orc.unpack4(gq)
        assert nib.min() == 0 and nib.max() == 15 and abs(nib.mean() - 7.5) < 0.2


def test_zipf_bias_shape_and_order():
    b = synth.zipf_bias(512, 1.1, seed=1731, device="cpu")
    assert b.shape == (512,) and b.dtype == torch.float32
    p = torch.softmax(b.double(), 0)
    srt = torch.sort(p, descending=True).values
    ranks = torch.arange(1, 513, dtype=torch.float64)
    ref = ranks ** -1.1
    assert torch.allclose(srt, ref / ref.sum(), rtol=1e-5)


def test_verify_logits_correlation():
    t, d = synth.verify_logits(3, 20000, seed=5, device="cpu")
    assert t.shape == (4, 20000) and d.shape == (3, 20000)
    c = np.corrcoef(t[:3].flatten().numpy(), d.flatten().numpy())[0, 1]
    assert abs(c - 0.8) < 0.02 and abs(float(t.std()) - 3.0) < 0.1
