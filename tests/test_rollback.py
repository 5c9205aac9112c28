"""Rollback bookkeeping (engine/rollback.py) on the CPU: the reference's checks and cuts (engine/rollback.py:26-41)
and the StepRecord ring (kernels/gdn_step_record.py:19-56) over host tensors."""
import pytest
import torch

from slotstream_spark_amd.engine import rollback as rb


class _Cache:
    def __init__(self):
        self.pos, self.last = 0, "something"


class _Model:
    def __init__(self, **state):
        self.st = rb.SeqState(state={k: v.clone() for k, v in state.items()})


def _round(m, rec, rows, tokens, writes):
    """A verify round: the pass writes the state after each row into the ring and advances the live state."""
    ck = rb.checkpoint(m)
    rec.begin()
    for i in range(rows):
        for name, v in writes(i).items():
            rec.ring[name][i].copy_(v)
            m.st.state[name].copy_(v)
    m.st.pos += rows
    m.st.tokens += tokens
    return ck


def test_checkpoint_rollback_cuts_position_tokens_and_caches():
    m = _Model(S=torch.zeros(2, 3))
    m.st.attn = {3: _Cache(), 7: _Cache()}
    m.st.pos, m.st.tokens = 10, list(range(10))
    rec = rb.StepRecord(m.st, rows=3)
    ck = _round(m, rec, 3, [100, 101, 102], lambda i: {"S": torch.full((2, 3), float(i + 1))})
    assert ck == rb.Checkpoint(10, 10) and rec.outstanding == 1 and rec.rounds == 1
    rb.rollback(m, rec, ck, keep=2)
    assert m.st.pos == 12 and m.st.tokens == list(range(10)) + [100, 101]
    assert torch.equal(m.st.state["S"], torch.full((2, 3), 2.0))   # the state after row 2 of the round
    assert all(c.pos == 12 and c.last is None for c in m.st.attn.values())
    assert rec.outstanding == 0


def test_keep_all_releases_without_restore():
    m = _Model(S=torch.zeros(4))
    rec = rb.StepRecord(m.st, rows=3)
    ck = _round(m, rec, 3, [1, 2, 3], lambda i: {"S": torch.full((4,), float(10 + i))})
    rb.rollback(m, rec, ck, keep=3)
    assert m.st.pos == 3 and m.st.tokens == [1, 2, 3] and rec.outstanding == 0
    assert torch.equal(m.st.state["S"], torch.full((4,), 12.0))


def test_rollback_errors():
    m = _Model()
    rec = rb.StepRecord(m.st, rows=3)
    assert rec.nbytes == 0 and rec.ring == {}
    ck = _round(m, rec, 3, [1, 2, 3], lambda i: {})
    for bad in (0, 4):
        with pytest.raises(ValueError, match="keep must be in 1..3"):
            rb.rollback(m, rec, ck, keep=bad)
    with pytest.raises(RuntimeError, match="expected the checkpoint"):
        rb.rollback(m, rec, rb.Checkpoint(1, 0), keep=1)
    rb.rollback(m, rec, ck, keep=1)
    assert m.st.pos == 1 and m.st.tokens == [1]
    with pytest.raises(RuntimeError, match="release without a matching begin"):
        rec.release()
    with pytest.raises(ValueError):
        rec.restore(m.st, 5)


def test_rows_parameter_and_ring_shapes():
    m = _Model(S=torch.zeros(2, 5, dtype=torch.float16), conv=torch.zeros(3, dtype=torch.int32))
    rec = rb.StepRecord(m.st, rows=4)
    assert rec.ring["S"].shape == (4, 2, 5) and rec.ring["S"].dtype == torch.float16
    assert rec.ring["conv"].shape == (4, 3) and rec.nbytes == 4 * 10 * 2 + 4 * 3 * 4
    ck = _round(m, rec, 4, [9, 8, 7, 6], lambda i: {"S": torch.full((2, 5), float(i), dtype=torch.float16),
                                                     "conv": torch.full((3,), i, dtype=torch.int32)})
    rb.rollback(m, rec, ck, keep=3, rows=4)
    assert m.st.tokens == [9, 8, 7] and int(m.st.state["conv"][0]) == 2 and float(m.st.state["S"][1, 4]) == 2.0
