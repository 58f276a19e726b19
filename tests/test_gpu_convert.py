"""GPU parity of df_convert, the reference's utils::to_float / to_half
(dnn/utils/convert.cu:6-27) as a tensor op, against the oracle's dfo_convert.

Bar: bit-exact (integer/byte work).  Narrowing fp32 -> bf16 and fp32 -> f16
is checked on every one of the 2^32 binary32 patterns; widening bf16 / f16 ->
fp32 and bf16 -> f16 on all 2^16 patterns, int8 on all 256 values.  The
oracle's binary16 conversions are pinned against numpy's IEEE float16 casts
(tests/test_oracle_convert.py).
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import DType
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


def convert(x, in_dt, out_dt, out_torch_dtype):
    out = torch.empty(x.shape, dtype=out_torch_dtype, device=x.device)
    df.call("df_convert", int(in_dt), x.data_ptr(), int(out_dt), out.data_ptr(), x.numel(),
            torch.cuda.current_stream().cuda_stream)
    return out


def assert_same(got, exp, what):
    got = np.asarray(got).reshape(-1)
    exp = np.asarray(exp).reshape(-1)
    bad = np.nonzero(got != exp)[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: got {got[bad[0]]:#x} exp {exp[bad[0]]:#x}"


@pytest.mark.parametrize("out_dt,to_f16", [(DType.BFLOAT16, False), (DType.HALF, True)], ids=["bf16", "f16"])
def test_narrowing_every_f32_pattern(dev, out_dt, to_f16):
    """All 2^32 binary32 inputs, in 2^28 chunks: RNE, subnormals, overflow,
    NaN policy (sign|0x7FC0 / sign|0x7E00)."""
    for c in range(16):
        first = c * CHUNK
        x = torch.arange(first, first + CHUNK, dtype=torch.int64, device=dev).to(torch.int32).view(torch.float32)
        got = convert(x, DType.FLOAT32, out_dt, torch.int16).cpu().numpy().view(np.uint16)
        del x
        assert_same(got, orc.narrow_bits_range(first, CHUNK, to_f16), f"chunk {c}")


@pytest.mark.parametrize("in_dt", [DType.BFLOAT16, DType.HALF], ids=["bf16", "f16"])
def test_widening_every_pattern(dev, in_dt):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(h.view(np.int16)).to(dev)
    got = convert(x, in_dt, DType.FLOAT32, torch.float32).cpu().numpy().view(np.uint32)
    assert_same(got, orc.convert(h, int(in_dt), 0).view(np.uint32), f"{in_dt.name} -> f32")


def test_bf16_to_f16_every_pattern(dev):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(h.view(np.int16)).to(dev)
    got = convert(x, DType.BFLOAT16, DType.HALF, torch.int16).cpu().numpy().view(np.uint16)
    assert_same(got, orc.convert(h, 4, 1), "bf16 -> f16")


@pytest.mark.parametrize("out_dt,tdt", [(DType.FLOAT32, torch.float32), (DType.HALF, torch.int16)])
def test_int8_widening(dev, out_dt, tdt):
    i = np.arange(-128, 128, dtype=np.int8)
    x = torch.from_numpy(i).to(dev)
    got = convert(x, DType.INT8, out_dt, tdt).cpu().numpy()
    exp = orc.convert(i, 2, int(out_dt))
    assert_same(got.view(exp.dtype), exp, f"int8 -> {out_dt.name}")


@pytest.mark.parametrize("n", [0, 1, 3, 255, 1000003])
def test_ragged_sizes_f32_to_f16(dev, n):
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    x = torch.from_numpy(bits.view(np.int32)).to(dev).view(torch.float32)
    got = convert(x, DType.FLOAT32, DType.HALF, torch.int16).cpu().numpy().view(np.uint16)
    assert_same(got, orc.convert(bits.view(np.float32), 0, 1), f"n={n}")


def test_unsupported_pairs_refused(dev):
    x = torch.zeros(16, dtype=torch.float32, device=dev)
    y = torch.zeros(16, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    for a, b in ((DType.FLOAT32, DType.INT8), (DType.HALF, DType.BFLOAT16), (DType.FP8E4M3, DType.FLOAT32)):
        assert df.lib().df_convert(int(a), x.data_ptr(), int(b), y.data_ptr(), 16, st) == -2
