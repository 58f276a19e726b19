"""GPU parity of the binary16 (DF_DTYPE_HALF) paths behind the reference's
FP16 instantiations -- FullyConnectedLayer<__half>
(dnn/layers/fully_connected_layer.cu:405, kernels :14-106 with T = __half:
to_float on the inputs, fp32 sums, to_half on the outputs) -- against the
CPU oracle.

Bars:
  - absmax, scale and codes of f16 inputs bit-exact: binary16 widens to
    binary32 exactly, so they are the oracle's absmax / codes of the widened
    values (every one of the 2^16 patterns, and ragged lengths);
  - f16 GEMM outputs against the oracle's fp32 products rounded to nearest
    even binary16 (dfo_convert): normwise relative error within 1e-4 plus
    the binary16 unit roundoff 2^-11;
  - the grouped f16 backward bit-identical to the two separate launches.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import DType, Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

TOL16 = 1e-4 + 2.0 ** -11


def f16_dev(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).to(dev).view(torch.float16)


def widen(bits):
    return orc.convert(np.ascontiguousarray(bits, np.uint16), 1, 0).reshape(np.shape(bits))


def round16(x):
    """fp32 -> nearest even binary16 -> fp32 (the reference's to_half)."""
    x = np.ascontiguousarray(x, np.float32)
    return widen(orc.convert(x, 0, 1).reshape(x.shape))


def host16(t):
    return widen(t.view(torch.int16).cpu().numpy().view(np.uint16))


def finite_absmax(v):
    f = np.abs(v[np.isfinite(v)])
    return np.float32(f.max()) if f.size else np.float32(0.0)


@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_every_pattern_absmax_and_codes(dev, fmt):
    """All 2^16 binary16 patterns as a [256, 256] matrix (NaN, inf, zeros,
    subnormals included): absmax skips NaN/inf, the scale is D1/D2's, and
    q / qt hold the oracle's codes of the widened values."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    x = f16_dev(bits, dev)
    am, sc = df.absmax_scale(x, fmt)
    v = widen(bits)
    assert am.item() == finite_absmax(v) == np.float32(65504.0)
    s = np.float32(orc.scale(float(finite_absmax(v)), int(fmt)))
    assert sc.cpu().numpy().view(np.uint32)[0] == s.view(np.uint32)
    q, qt = df.quantize_2d(x, sc, fmt, want_q=True, want_qt=True)
    codes = orc.quantize(v, float(s), int(fmt))
    assert np.array_equal(q.cpu().numpy()[:, :256], codes)
    assert np.array_equal(qt.cpu().numpy()[:, :256], np.ascontiguousarray(codes.T))
    # a scale below one: subnormal binary16 inputs reach the fp8 normal range
    s2 = torch.tensor([2.0 ** -20], dtype=torch.float32, device=dev)
    q2, _ = df.quantize_2d(x, s2, fmt, want_q=True)
    assert np.array_equal(q2.cpu().numpy()[:, :256], orc.quantize(v, 2.0 ** -20, int(fmt)))


@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 65537, 1 << 20])
def test_absmax_ragged(dev, n):
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 1 << 16, size=n, dtype=np.uint32).astype(np.uint16)
    am, _ = df.absmax_scale(f16_dev(bits, dev), Fmt.E4M3)
    assert am.item() == finite_absmax(widen(bits))


@pytest.mark.parametrize("rows,cols", [(1, 5), (37, 100), (129, 257), (512, 1600)])
def test_quantize_2d_colsum(dev, rows, cols):
    x = synth.normal((rows, cols), 1e-3, seed=rows + cols)
    bits = orc.convert(x, 0, 1).reshape(rows, cols)
    xd, v = f16_dev(bits, dev), widen(bits)
    am, sc = df.absmax_scale(xd, Fmt.E5M2)
    q, qt, cs = df.quantize_2d(xd, sc, Fmt.E5M2, want_q=True, want_qt=True, colsum=True)
    s = orc.scale(orc.absmax(np.ascontiguousarray(v)), int(Fmt.E5M2))
    codes = orc.quantize(v, s, int(Fmt.E5M2))
    assert np.array_equal(q.cpu().numpy()[:, :cols], codes)
    assert np.array_equal(qt.cpu().numpy()[:, :rows], np.ascontiguousarray(codes.T))
    assert orc.rel_err(cs.cpu().numpy(), orc.fc_backward_bias(v)) <= 1e-5


def operands(M, K, N, seed, dev):
    """e4m3 codes of f16 X [M, K] and W [N, K] (through the f16 path), their
    dequantized values, and an f16 bias [N]."""
    out = []
    for shape, std, sd in (((M, K), 1.0, seed), ((N, K), 0.02, seed + 1)):
        bits = orc.convert(synth.normal(shape, std, seed=sd), 0, 1).reshape(shape)
        xd = f16_dev(bits, dev)
        am, sc = df.absmax_scale(xd, Fmt.E4M3)
        q, qt = df.quantize_2d(xd, sc, Fmt.E4M3, want_q=True, want_qt=True)
        v = widen(bits)
        s = orc.scale(orc.absmax(np.ascontiguousarray(v)), int(Fmt.E4M3))
        out.append((q, qt, sc, orc.dequantize(orc.quantize(v, s, int(Fmt.E4M3)), s, int(Fmt.E4M3), "f32")))
    bbits = orc.convert(synth.normal((N,), 0.1, seed=seed + 2), 0, 1)
    return out[0], out[1], bbits


def sample_rows(M, seed):
    """every row of a small output; else 96 rows including each 256-row
    band's first and last"""
    if M <= 96:
        return np.arange(M)
    bands = np.arange(0, M, 256)
    fixed = np.concatenate([bands, np.minimum(bands + 255, M - 1)])
    extra = np.random.default_rng(seed).choice(M, size=max(0, 96 - fixed.size), replace=False)
    return np.unique(np.concatenate([fixed, extra]))


@pytest.mark.parametrize("M,K,N", [(1, 4, 3), (100, 40, 50), (129, 272, 257), (512, 1600, 1600),
                                   (2048, 1600, 4800)])
def test_forward_f16_output(dev, M, K, N):
    (xq, _, sx, Xd), (wq, _, sw, Wd), bbits = operands(M, K, N, M + K + N, dev)
    rows = sample_rows(M, M + N)
    ref = orc.fc_forward(Xd[rows], Wd, widen(bbits))
    # f16 bias, f32 bias and none (f16 output each)
    Y = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=f16_dev(bbits, dev), out_dtype=torch.float16)
    assert orc.rel_err(host16(Y)[rows], round16(ref)) <= TOL16
    b32 = torch.from_numpy(widen(bbits)).to(dev)
    Y32b = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=b32, out_dtype=torch.float16)
    assert torch.equal(Y32b.view(torch.int16), Y.view(torch.int16))  # same values, same rounding
    Yn = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, out_dtype=torch.float16)
    assert orc.rel_err(host16(Yn)[rows], round16(orc.fc_forward(Xd[rows], Wd, None))) <= TOL16


def test_f16_bias_needs_f16_output(dev):
    (xq, _, sx, _), (wq, _, sw, _), bbits = operands(64, 64, 64, 3, dev)
    b = f16_dev(bbits, dev)
    for out in (torch.float32, torch.bfloat16):
        with pytest.raises(RuntimeError):
            df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, 64, sx, sw, bias=b, out_dtype=out)


@pytest.mark.parametrize("M,K,N", [(100, 40, 50), (512, 1600, 1600), (2048, 1600, 1600)])
def test_backward_f16_outputs(dev, M, K, N):
    """dX and dW in binary16: the grouped launch equals the separate ones bit
    for bit, and both are the oracle's products rounded to binary16."""
    (_, xt, sx, Xd), (_, wt, sw, Wd), _ = operands(M, K, N, 7 * M + N, dev)
    dyb = orc.convert(synth.normal((M, N), 1e-3, seed=M + 5), 0, 1).reshape(M, N)
    dyd16 = f16_dev(dyb, dev)
    am, sdy = df.absmax_scale(dyd16, Fmt.E5M2)
    dyq, dyt = df.quantize_2d(dyd16, sdy, Fmt.E5M2, want_q=True, want_qt=True)
    v = widen(dyb)
    s = orc.scale(orc.absmax(np.ascontiguousarray(v)), int(Fmt.E5M2))
    dYd = orc.dequantize(orc.quantize(v, s, int(Fmt.E5M2)), s, int(Fmt.E5M2), "f32")
    dX, dW = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, dx_dtype=torch.float16, dw_dtype=torch.float16)
    dX1 = df.gemm_nt(dyq, Fmt.E5M2, wt, Fmt.E4M3, N, sdy, sw, out_dtype=torch.float16)
    assert torch.equal(dX.view(torch.int16), dX1.view(torch.int16))
    rows = sample_rows(M, N)
    assert orc.rel_err(host16(dX)[rows], round16(orc.fc_backward_input(dYd[rows], Wd))) <= TOL16
    assert orc.rel_err(host16(dW), round16(orc.fc_backward_weights(dYd, Xd))) <= TOL16
    grouped, _ = df.gemm_bwd_plan(M, N, K)
    if grouped:  # f16 pairs take the grouped launch like the other types
        dW1 = df.gemm_nt(dyt, Fmt.E5M2, xt, Fmt.E4M3, M, sdy, sx, out_dtype=torch.float16)
        assert orc.rel_err(host16(dW1), host16(dW)) <= 2.0 ** -10


def test_mixed_f16_pair_takes_separate_launches(dev):
    """f16 dX with an fp32 dW: not grouped; each equals its own NT call."""
    M, K, N = 512, 256, 384
    (_, xt, sx, _), (_, wt, sw, _), _ = operands(M, K, N, 11, dev)
    dyb = orc.convert(synth.normal((M, N), 1e-3, seed=12), 0, 1).reshape(M, N)
    dyd16 = f16_dev(dyb, dev)
    am, sdy = df.absmax_scale(dyd16, Fmt.E5M2)
    dyq, dyt = df.quantize_2d(dyd16, sdy, Fmt.E5M2, want_q=True, want_qt=True)
    dX, dW = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, dx_dtype=torch.float16, dw_dtype=torch.float32)
    dX1 = df.gemm_nt(dyq, Fmt.E5M2, wt, Fmt.E4M3, N, sdy, sw, out_dtype=torch.float16)
    dW1 = df.gemm_nt(dyt, Fmt.E5M2, xt, Fmt.E4M3, M, sdy, sx, out_dtype=torch.float32)
    assert torch.equal(dX.view(torch.int16), dX1.view(torch.int16))
    assert orc.rel_err(dW.cpu().numpy(), dW1.cpu().numpy()) <= 1e-6
