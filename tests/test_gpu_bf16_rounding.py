"""The device fp32 -> bf16 conversion every kernel uses (round to nearest even, NaN -> quiet NaN) against the
oracle's, over every bf16 high half with the low halves that decide rounding (0, just below half, the exact tie,
just above, all ones) and a million random patterns: denormals, ties to even, overflow to infinity, infinities.
The conversion is reached through ssmoe_combine_shared with a zero shared term, y = bf16(bf16(routed) + 0)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd import _lib

pytestmark = pytest.mark.gpu


def test_f32_to_bf16_matches_oracle_everywhere():
    print("[bf16] rounding sweep", flush=True)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234], dtype=np.uint32)
    pats = np.concatenate([(hi[:, None] | lows[None, :]).reshape(-1),
                           np.random.default_rng(7).integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    H = 4096
    pats = np.concatenate([pats, np.zeros((-pats.size) % H, np.uint32)])
    T = pats.size // H
    routed = torch.from_numpy(pats.view(np.float32).reshape(T, H).copy()).cuda()
    sh = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    sgl = torch.zeros(T, dtype=torch.bfloat16, device="cuda")
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    _lib.check(_lib.lib().ssmoe_combine_shared(routed.data_ptr(), sh.data_ptr(), sgl.data_ptr(), y.data_ptr(), T, H,
                                               torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    got = y.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    want = O.f32_to_bf16(pats.view(np.float32))
    want = np.where(want == 0x8000, 0, want)          # bf16(-0) + (+0) = +0
    nan = (pats & 0x7FFFFFFF) > 0x7F800000
    assert np.array_equal(got[~nan], want[~nan]), np.nonzero(got[~nan] != want[~nan])[0][:10]
    assert ((got[nan] & 0x7FFF) > 0x7F80).all()      # NaN stays NaN
    denorm = ((pats >> 23) & 0xFF) == 0
    assert denorm.sum() > 1000 and (got[denorm & ~nan] != 0).any()   # denormals were rounded, not flushed


def test_bf16_round_export_is_the_rule_bit_for_bit():
    """ssmoe_bf16_round (the library's ss_f32_to_bf16, the hardware conversion alone) against the oracle's integer
    rule on every bf16 high half with the deciding low halves, every NaN high half with five payloads each, and a
    million random patterns: NaNs included, bit for bit."""
    print("[bf16] export sweep", flush=True)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234], dtype=np.uint32)
    nan_hi = np.concatenate([np.arange(0x7F80, 0x8000), np.arange(0xFF80, 0x10000)]).astype(np.uint32) << 16
    nan_lows = np.array([0x0001, 0x0040, 0x8000, 0xBEEF, 0xFFFF], dtype=np.uint32)
    pats = np.concatenate([(hi[:, None] | lows[None, :]).reshape(-1), (nan_hi[:, None] | nan_lows[None, :]).reshape(-1),
                           np.random.default_rng(11).integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    x = torch.from_numpy(pats.view(np.float32).copy()).cuda()
    y = torch.empty(pats.size, dtype=torch.int16, device="cuda")
    L = _lib.lib()
    _lib.check(L.ssmoe_bf16_round(x.data_ptr(), y.data_ptr(), pats.size, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.uint16)
    want = O.f32_to_bf16(pats.view(np.float32))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(int(pats[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]
    nan = (pats & 0x7FFFFFFF) > 0x7F800000
    assert nan.sum() > 1000
