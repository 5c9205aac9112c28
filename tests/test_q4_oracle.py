"""Pins of the affine 4-bit dense rows of the oracle (or_dense_rows_q4: the shared expert's projections when the
checkpoint keeps them quantized, model/layers.py:62-76 lin -> gemv on an AffineWeight, w = q * s + b of
kernels/affine_ref.py:10-30)."""
import numpy as np
import pytest

from oracle import oracle as O


def _q4(rng, n, k, scale=0.02):
    words = rng.integers(0, 2**32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    s = O.f32_to_bf16(np.abs(rng.standard_normal((n, k // 64))).astype(np.float32) * scale)
    b = O.f32_to_bf16(-8 * O.bf16_to_f32(s))
    return words, s, b


def _nibbles(words):
    w = words.astype(np.uint64)
    return np.stack([(w >> (4 * i)) & 0xF for i in range(8)], axis=-1).reshape(words.shape[0], -1).astype(np.float64)


@pytest.mark.parametrize("k", [512, 640, 2048, 2560])
def test_unit_scale_equals_the_bf16_rows_on_the_integers(k):
    """s = 1, b = 0: every weight is the integer q, exact in bf16, and the order is or_dense_rows': equal bits."""
    rng = np.random.default_rng(k)
    x = O.f32_to_bf16(rng.standard_normal((3, k)).astype(np.float32))
    words, _, _ = _q4(rng, 37, k)
    one = np.full((37, k // 64), 0x3F80, np.uint16)
    zero = np.zeros((37, k // 64), np.uint16)
    q_bf16 = O.f32_to_bf16(_nibbles(words).astype(np.float32))
    assert np.array_equal(O.dense_rows_q4(x, words, one, zero), O.dense_rows(x, q_bf16))


def test_power_of_two_scales_are_exact():
    """s = 2^-7, b = 0: q * s is exact, so the rows equal or_dense_rows on the bf16 weights q * 2^-7."""
    rng = np.random.default_rng(5)
    k = 2048
    x = O.f32_to_bf16(rng.standard_normal((2, k)).astype(np.float32))
    words, _, _ = _q4(rng, 20, k)
    s = np.full((20, k // 64), O.f32_to_bf16(np.float32(2.0 ** -7)), np.uint16)
    zero = np.zeros((20, k // 64), np.uint16)
    w_bf16 = O.f32_to_bf16((_nibbles(words) * 2.0 ** -7).astype(np.float32))
    assert np.array_equal(O.dense_rows_q4(x, words, s, zero), O.dense_rows(x, w_bf16))


@pytest.mark.parametrize("k,n", [(2048, 512), (2560, 640), (512, 2048), (640, 2560)])
def test_against_fp64_with_a_nibble_swap_control(k, n):
    """Random scales and biases (b = -8 s): within one bf16 rounding (plus fp32 accumulation) of the fp64 dot on
    the exact dequantized weights; the same weights with the two nibbles of every byte swapped miss by far more."""
    rng = np.random.default_rng(k + n)
    x = O.f32_to_bf16(rng.standard_normal((2, k)).astype(np.float32))
    words, s, b = _q4(rng, n, k)
    got = O.bf16_to_f32(O.dense_rows_q4(x, words, s, b)).astype(np.float64)
    sc = np.repeat(O.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bi = np.repeat(O.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    w = _nibbles(words) * sc + bi
    xf = O.bf16_to_f32(x).astype(np.float64)
    ref = xf @ w.T
    mag = np.abs(xf) @ np.abs(w).T
    err = np.abs(got - ref) / (np.abs(ref) * 2.0 ** -8 + mag * 1e-6)
    assert err.max() <= 1.0, err.max()
    sw = ((words & 0x0F0F0F0F) << 4) | ((words >> 4) & 0x0F0F0F0F)
    bad = O.bf16_to_f32(O.dense_rows_q4(x, sw.astype(np.uint32), s, b)).astype(np.float64)
    assert O.rel_l2(bad, ref) > 10 * max(O.rel_l2(got, ref), 1e-3)


def test_shared_expert_q4_matches_the_dequantized_chain():
    """The q4 shared-expert chain equals the bf16 chain when every q4 weight is exactly a bf16 value (s = 2^-6,
    b = -8 s, so w = (q - 8) / 64): the same projections, silu products and rounding points."""
    rng = np.random.default_rng(9)
    H, Is = 2048, 512
    x = O.f32_to_bf16(rng.standard_normal((2, H)).astype(np.float32))
    mats = []
    for n, k in ((Is, H), (Is, H), (H, Is)):
        words, _, _ = _q4(rng, n, k)
        s = np.full((n, k // 64), O.f32_to_bf16(np.float32(2.0 ** -6)), np.uint16)
        b = np.full((n, k // 64), O.f32_to_bf16(np.float32(-8 * 2.0 ** -6)), np.uint16)
        mats.append((words, s, b, O.f32_to_bf16(((_nibbles(words) - 8) * 2.0 ** -6).astype(np.float32))))
    sg = O.f32_to_bf16((rng.standard_normal((1, H)) * 0.02).astype(np.float32))
    sh_q, sgl_q = O.shared_expert_q4(x, mats[0][:3], mats[1][:3], mats[2][:3], sg)
    sh_b, sgl_b = O.shared_expert(x, mats[0][3], mats[1][3], mats[2][3], sg)
    assert np.array_equal(sh_q, sh_b) and np.array_equal(sgl_q, sgl_b)
