#!/usr/bin/env python3
"""Writes tests/golden/fp8_golden.json: fixtures that pin the CPU oracle.

Sources, none of them the oracle itself:
  * the reference's own known-answer case (tests/layers/
    fully_connected_layer_test.cu:266-284): W = {1,2,3,4} (2x2),
    b = {0.5,-0.5}, x = {1,2}, fp32 y = {5.5, 10.5};
  * the OCP OFP8 v1.0 closed form for every code of both formats
    (value = (-1)^S * 2^(E-bias) * (1 + M/2^m), or 2^(1-bias) * M/2^m when
    E = 0; e4m3 S.1111.111 = NaN and no inf; e5m2 E = 31 is inf/NaN),
    evaluated with Python fractions;
  * torch's CPU float8 casts (torch.float8_e4m3fn / float8_e5m2, which
    round to nearest even but do not saturate), applied after clamping to
    +-max, for a curated list of binary32 inputs: every midpoint between
    adjacent codes and its two neighbouring binary32 values, the subnormal
    range, the saturation boundary, signed zeros and specials.  NaN
    expectations follow the contract (sign|0x7F) rather than torch.
Run once; the JSON is committed.  torch is only needed to regenerate.
"""
from __future__ import annotations

import json
import math
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
FORMATS = {"e4m3": dict(m=3, bias=7, max_code=0x7E, fmax=448.0),
           "e5m2": dict(m=2, bias=15, max_code=0x7B, fmax=57344.0)}


def spec_value(code: int, fmt: str):
    """Closed-form value of a code, or 'nan'/'inf'/'-inf'."""
    f = FORMATS[fmt]
    m_bits, bias = f["m"], f["bias"]
    e_bits = 7 - m_bits
    sign = -1 if code & 0x80 else 1
    e = (code >> m_bits) & ((1 << e_bits) - 1)
    mant = code & ((1 << m_bits) - 1)
    if fmt == "e4m3" and (code & 0x7F) == 0x7F:
        return "nan"
    if fmt == "e5m2" and e == 31:
        return ("inf" if sign > 0 else "-inf") if mant == 0 else "nan"
    if e == 0:
        v = Fraction(mant, 1 << m_bits) * Fraction(2) ** (1 - bias)
    else:
        v = (1 + Fraction(mant, 1 << m_bits)) * Fraction(2) ** (e - bias)
    return sign * v


def f32(v) -> float:
    return float(np.float32(v))


def f32_bits(v: float) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def neighbours(v: float):
    a = np.array([v], np.float32)
    return [float(np.nextafter(a, np.float32(-np.inf))[0]), float(a[0]),
            float(np.nextafter(a, np.float32(np.inf))[0])]


def curated_inputs(fmt: str):
    f = FORMATS[fmt]
    pos = [spec_value(c, fmt) for c in range(f["max_code"] + 1)]
    vals = set()
    for i, v in enumerate(pos):
        vals.update(neighbours(float(v)))
        if i + 1 < len(pos):
            mid = (v + pos[i + 1]) / 2  # exact midpoint; representable in binary32
            vals.update(neighbours(float(mid)))
    fm = f["fmax"]
    half_ulp_top = float(pos[-1] - pos[-2]) / 2
    vals.update(neighbours(fm + half_ulp_top))
    vals.update([fm * 2, 1e30, 3.4028234663852886e38, 1e-40, 2.0 ** -149, 2.0 ** -126, 0.0])
    out = sorted(v for v in vals if math.isfinite(v))
    return out + [-v for v in out] + [float("inf"), float("-inf")]


def torch_codes(values, fmt: str):
    import torch
    f = FORMATS[fmt]
    x = torch.tensor(values, dtype=torch.float32)
    x = torch.clamp(x, -f["fmax"], f["fmax"])
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    return x.to(dt).view(torch.uint8).tolist()


def main():
    out = {"source": "tests/golden/make_golden.py", "formats": {}}
    for fmt in FORMATS:
        table = []
        for c in range(256):
            v = spec_value(c, fmt)
            # Fractions have no signed zero: apply the sign bit to the float
            table.append(v if isinstance(v, str) else f32_bits(math.copysign(float(abs(v)), -1.0 if c & 0x80 else 1.0)))
        inputs = curated_inputs(fmt)
        codes = torch_codes(inputs, fmt)
        out["formats"][fmt] = {
            "decode_bits": table,  # binary32 bit pattern, or 'nan'/'inf'/'-inf'
            "encode_inputs_bits": [f32_bits(v) for v in inputs],
            "encode_codes": codes,
            "nan_inputs_bits": [0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFFFFFFF],
            "nan_codes": [0x7F, 0xFF, 0x7F, 0xFF],
        }
    # reference KAT (fully_connected_layer_test.cu:266-284) and its fp8 images
    out["fc_kat"] = {
        "W": [[1.0, 2.0], [3.0, 4.0]], "b": [0.5, -0.5], "x": [[1.0, 2.0]], "y_fp32": [[5.5, 10.5]],
        "W_codes_e4m3": torch_codes([1 * 112.0, 2 * 112.0, 3 * 112.0, 4 * 112.0], "e4m3"),
        "x_codes_e4m3": torch_codes([1 * 224.0, 2 * 224.0], "e4m3"),
    }
    path = os.path.join(HERE, "fp8_golden.json")
    with open(path, "w") as fh:
        json.dump(out, fh)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
