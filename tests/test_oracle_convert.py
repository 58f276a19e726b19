"""Pins of the oracle's conversions (the reference's utils::to_float /
to_half, dnn/utils/convert.cu:6-27, and the bf16 rounding of the outputs).

binary16 narrowing and widening are checked against numpy's float16 casts
(IEEE round-to-nearest-even with subnormals, an implementation independent of
the oracle's), bf16 narrowing against torch's bf16 cast.  numpy keeps part of
a NaN's payload when it narrows; the oracle's policy is the quiet NaN
sign|0x7E00 (binary16) / sign|0x7FC0 (bf16), checked on its own.
"""
import numpy as np
import pytest
import torch

from oracle import pyoracle as orc

F32, F16, I8, BF16 = 0, 1, 2, 4


def np_f32_to_f16_bits(x):
    with np.errstate(over="ignore"):
        return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


def finite_or_inf(bits):
    return (bits & 0x7FFFFFFF) <= 0x7F800000


def test_f16_narrowing_structured_sweep():
    """Every sign and binary32 exponent x every value of the 13 fraction bits
    that binary16 drops (the rounding decision) x four patterns of the 10
    kept bits: 16.8M inputs covering ties, carries into the exponent,
    overflow at 65520, subnormal targets and underflow to zero."""
    se = np.arange(512, dtype=np.uint32) << 23
    low = np.arange(1 << 13, dtype=np.uint32)
    for hi in (0x000, 0x001, 0x155, 0x3FF):
        bits = (se[:, None] | (np.uint32(hi) << 13) | low[None, :]).reshape(-1)
        bits = bits[finite_or_inf(bits)]
        got = orc.convert(bits.view(np.float32), F32, F16)
        exp = np_f32_to_f16_bits(bits.view(np.float32))
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, f"hi={hi:#x}: {bad.size} mismatches, first {bits[bad[0]]:#010x}"


def test_f16_narrowing_random_and_edges():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0x477FF000, 0x477FEFFF, 0x477FE000, 0x47800000, 0x38800000, 0x387FFFFF,
                      0x33800000, 0x33000000, 0x33000001, 0x337FFFFF, 0x32FFFFFF, 0x00000001,
                      0x7F800000, 0x00000000], np.uint32)
    bits = np.concatenate([bits, edges, edges | 0x80000000])
    bits = bits[finite_or_inf(bits)]
    assert np.array_equal(orc.convert(bits.view(np.float32), F32, F16), np_f32_to_f16_bits(bits.view(np.float32)))
    # closed forms: the largest finite, its overflow midpoint, the smallest
    # subnormal and the tie below it
    f = lambda v: int(orc.convert(np.array([v], np.float32), F32, F16)[0])
    assert f(65504.0) == 0x7BFF and f(65519.996) == 0x7BFF and f(65520.0) == 0x7C00
    assert f(2.0 ** -24) == 0x0001 and f(2.0 ** -25) == 0x0000 and f(1.5 * 2.0 ** -25) == 0x0001
    assert f(-0.0) == 0x8000 and f(1.0) == 0x3C00 and f(-2.0) == 0xC000


def test_f16_nan_policy():
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001, 0x7FFFFFFF, 0x7FA00000], np.uint32)
    got = orc.convert(nans.view(np.float32), F32, F16)
    assert got.tolist() == [0x7E00, 0xFE00, 0x7E00, 0xFE00, 0x7E00, 0x7E00]


def test_f16_widening_all_patterns():
    """All 2^16 binary16 patterns, NaN payloads included (numpy keeps them
    on widening, as the oracle does)."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = orc.convert(h, F16, F32).view(np.uint32)
    exp = h.view(np.float16).astype(np.float32).view(np.uint32)
    # numpy sets the quiet bit of a signalling NaN on widening; the oracle
    # keeps the payload bits as they are, like the bf16 widening
    nan = (h & 0x7C00) == 0x7C00
    nan &= (h & 0x03FF) != 0
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.array_equal(got[nan], ((h[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000
                          | ((h[nan].astype(np.uint32) & 0x3FF) << 13))


def test_round_trip_f16_exact():
    """binary16 -> binary32 -> binary16 is the identity on every non-NaN pattern."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    keep = ~(((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0))
    back = orc.convert(orc.convert(h, F16, F32), F32, F16)
    assert np.array_equal(back[keep], h[keep])


def test_bf16_narrowing_matches_torch():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    bits = bits[finite_or_inf(bits)]
    x = bits.view(np.float32)
    got = orc.convert(x, F32, BF16)
    exp = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, exp)
    assert np.array_equal(orc.narrow_bits_range(0x3F800000, 1 << 16, False),
                          orc.convert(np.arange(0x3F800000, 0x3F810000, dtype=np.uint32).view(np.float32), F32,
                                      BF16))


def test_bf16_to_f16_is_one_rounding():
    """bf16 -> binary16 widens exactly first: equal to numpy's cast of the
    exact binary32 value."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = (h.astype(np.uint32) << 16).view(np.float32)
    keep = ~np.isnan(v)
    got = orc.convert(h, BF16, F16)
    assert np.array_equal(got[keep], np_f32_to_f16_bits(v[keep]))
    assert np.all((got[~keep] & 0x7FFF) == 0x7E00)


def test_int8_widening_exact():
    i = np.arange(-128, 128, dtype=np.int8)
    assert np.array_equal(orc.convert(i, I8, F32), i.astype(np.float32))
    assert np.array_equal(orc.convert(i, I8, F16), i.astype(np.float16).view(np.uint16))


def test_unsupported_pairs_refused():
    with pytest.raises(ValueError):
        orc.convert(np.zeros(4, np.float32), F32, I8)


def test_narrow_range_helper_matches_convert():
    first = 0x38000000
    bits = np.arange(first, first + (1 << 20), dtype=np.uint64).astype(np.uint32)
    for to_f16, dt in ((True, F16), (False, BF16)):
        assert np.array_equal(orc.narrow_bits_range(first, 1 << 20, to_f16), orc.convert(bits.view(np.float32),
                                                                                            F32, dt))
