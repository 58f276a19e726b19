"""Pins the CPU oracle's fp8 codec (CPU only, no GPU).

Each check uses a method independent of the oracle's bit manipulation:
golden fixtures from the spec's closed form and torch's casts
(tests/golden/make_golden.py), an exhaustive 2^32 sweep against a
nearest-code table search, torch casts on every bf16 pattern and on random
binary32 patterns, and properties (monotonicity, sign symmetry, round trip).
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import pyoracle as orc

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "fp8_golden.json")))
FMT = {"e4m3": orc.E4M3, "e5m2": orc.E5M2}


def bits_to_f32(b):
    return np.array(b, dtype=np.uint32).view(np.float32)


@pytest.mark.parametrize("name", ["e4m3", "e5m2"])
def test_decode_matches_spec_closed_form(name):
    table = GOLDEN["formats"][name]["decode_bits"]
    for code, exp in enumerate(table):
        got = orc.decode(code, FMT[name])
        if exp == "nan":
            assert np.isnan(got)
            assert np.signbit(np.float32(got)) == bool(code & 0x80)
        elif exp in ("inf", "-inf"):
            assert got == (np.inf if exp == "inf" else -np.inf)
        else:
            assert np.float32(got).view(np.uint32) == np.uint32(exp), hex(code)


@pytest.mark.parametrize("name", ["e4m3", "e5m2"])
def test_encode_golden_vectors(name):
    g = GOLDEN["formats"][name]
    x = bits_to_f32(g["encode_inputs_bits"])
    got = orc.quantize(x, 1.0, FMT[name])
    exp = np.array(g["encode_codes"], np.uint8)
    bad = np.nonzero(got != exp)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(exp[i])) for i in bad[:5]]
    nan_got = orc.quantize(bits_to_f32(g["nan_inputs_bits"]), 1.0, FMT[name])
    assert nan_got.tolist() == g["nan_codes"]


@pytest.mark.parametrize("name", ["e4m3", "e5m2"])
def test_exhaustive_sweep_against_table_search(name):
    """All 2^32 binary32 patterns: the oracle's encoder equals an
    independent nearest-code binary search with ties to the even code."""
    bad, first = orc.sweep_compare(0, 1 << 32, FMT[name])
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}"


def torch_codes(x, name):
    fmax = orc.FMAX[FMT[name]]
    t = torch.clamp(torch.from_numpy(np.ascontiguousarray(x, np.float32)), -fmax, fmax)
    dt = torch.float8_e4m3fn if name == "e4m3" else torch.float8_e5m2
    return t.to(dt).view(torch.uint8).numpy()


@pytest.mark.parametrize("name", ["e4m3", "e5m2"])
def test_all_bf16_patterns_against_torch(name):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = orc.bf16_to_f32(bits)
    finite = ~np.isnan(x)
    got = orc.quantize(bits, 1.0, FMT[name])
    assert np.array_equal(got[finite], torch_codes(x[finite], name))
    # NaN -> sign|0x7F
    assert np.array_equal(got[~finite], np.where(np.signbit(x[~finite]), 0xFF, 0x7F).astype(np.uint8))


@pytest.mark.parametrize("name", ["e4m3", "e5m2"])
def test_random_patterns_with_scale_against_torch(name):
    """x / s in binary32 then torch's cast: the oracle's quantize composes
    IEEE division with its encoder."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1 << 20, dtype=np.float32) * np.float32(37.0)
    for s in (0.0123, 1.0 / 448.0, 3.3e-7, 250.0):
        s32 = np.float32(s)
        got = orc.quantize(x, float(s32), FMT[name])
        assert np.array_equal(got, torch_codes(x / s32, name))


def test_reference_kat_codes():
    """Known-answer codes derived from fully_connected_layer_test.cu:266-284: W
    absmax 4 -> s = 4/448, codes {0x6E,0x76,0x7A,0x7E} (336 ties to 320);
    x absmax 2 -> {0x76, 0x7E}."""
    kat = GOLDEN["fc_kat"]
    W = np.array(kat["W"], np.float32).reshape(-1)
    sW = orc.scale(orc.absmax(W), orc.E4M3)
    assert np.float32(sW) == np.float32(4.0) / np.float32(448.0)
    assert orc.quantize(W, sW, orc.E4M3).tolist() == kat["W_codes_e4m3"] == [0x6E, 0x76, 0x7A, 0x7E]
    x = np.array(kat["x"], np.float32).reshape(-1)
    sx = orc.scale(orc.absmax(x), orc.E4M3)
    assert orc.quantize(x, sx, orc.E4M3).tolist() == kat["x_codes_e4m3"] == [0x76, 0x7E]


@pytest.mark.parametrize("fmt", [orc.E4M3, orc.E5M2])
def test_properties(fmt):
    # decode -> encode identity on every finite code
    for c in range(256):
        v = orc.decode(c, fmt)
        if np.isfinite(v):
            assert orc.encode(v, fmt) == c or (v == 0 and orc.encode(v, fmt) in (0, 0x80))
    # monotone non-decreasing over sorted positive inputs, sign symmetric
    rng = np.random.default_rng(5)
    x = np.sort(np.abs(rng.standard_normal(1 << 16).astype(np.float32)) * np.float32(orc.FMAX[fmt] / 2))
    codes = orc.quantize(x, 1.0, fmt).astype(np.int32)
    assert np.all(np.diff(codes) >= 0)
    assert np.array_equal(orc.quantize(-x, 1.0, fmt), (codes | 0x80).astype(np.uint8))
    # saturation: anything at or beyond max, and infinities, give the max code
    mx = 0x7E if fmt == orc.E4M3 else 0x7B
    big = np.array([orc.FMAX[fmt], orc.FMAX[fmt] * 1.01, 1e30, np.inf], np.float32)
    assert orc.quantize(big, 1.0, fmt).tolist() == [mx] * 4
    assert orc.quantize(-big, 1.0, fmt).tolist() == [mx | 0x80] * 4


def test_absmax_and_scale_rules():
    """D2: finite values only; absmax 0 or non-finite-only gives s = 1."""
    x = np.array([1.0, -7.5, np.nan, np.inf, -np.inf, 3.0], np.float32)
    assert orc.absmax(x) == 7.5
    assert orc.scale(7.5, orc.E4M3) == np.float32(7.5) / np.float32(448.0)
    assert orc.scale(orc.absmax(np.array([np.nan, np.inf], np.float32)), orc.E4M3) == 1.0
    assert orc.scale(0.0, orc.E5M2) == 1.0
    assert orc.scale(1e-44, orc.E5M2) == 1.0  # 1e-44 / 57344 underflows to 0
    rng = np.random.default_rng(9)
    y = rng.standard_normal(10001).astype(np.float32)
    assert orc.absmax(y) == np.max(np.abs(y))
    assert orc.absmax(y[::-1].copy()) == orc.absmax(y)  # order independent
    b = orc.f32_to_bf16(y)
    assert orc.absmax(b) == np.max(np.abs(orc.bf16_to_f32(b)))


def test_bf16_rounding_against_torch():
    rng = np.random.default_rng(4)
    x = rng.integers(0, 1 << 32, size=1 << 18, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    exp = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), exp)
    assert np.array_equal([orc.lib().dfo_f32_to_bf16(float(v)) for v in x[:2000]], exp[:2000])


@pytest.mark.parametrize("fmt", [orc.E4M3, orc.E5M2])
def test_dequantize_rules(fmt):
    """D5: decode(q) * s in binary32; NaN codes -> canonical quiet NaN with
    the code's sign; bf16 output = RNE(binary32)."""
    codes = np.arange(256, dtype=np.uint8)
    s = np.float32(0.0371)
    out = orc.dequantize(codes, float(s), fmt, "f32")
    dec = np.array([orc.decode(int(c), fmt) for c in codes], np.float32)
    fin = np.isfinite(dec) | np.isinf(dec)
    assert np.array_equal(out[fin].view(np.uint32), (dec[fin] * s).view(np.uint32))
    nan = ~fin
    assert np.all(out[nan].view(np.uint32) == np.where(codes[nan] & 0x80, 0xFFC00000, 0x7FC00000))
    outb = orc.dequantize(codes, float(s), fmt, "bf16")
    assert np.array_equal(outb, orc.f32_to_bf16(out))
