"""GPU parity of df_fp8_gemm_fwd_absmax and df_fp8_gemm_bwd_absmax: the
forward GEMM whose Y, and the backward whose dX, also gives its absmax and
the next quantize's scale.

The reference's TransformerBlock feeds fc1's output straight into fc2
(dnn/layers/transformer_block.cu:79-81), so fc2's just-in-time scale is the
absmax of fc1's Y.  Bars:
- Y bit-identical to df_fp8_gemm_fwd's on the same codes, bias and output
  type (the fused epilogue only adds a fold);
- absmax and scale bit-identical to df_absmax_scale_bf16 / _f16 / _f32 over that Y
  (finite values only, as stored, rule D1/D2 for the next format);
- on the config-4 shapes the planner takes the unsplit 256x256 persistent
  kernel (the fused path, asserted through df_fp8_gemm_nt_plan); small,
  ragged and long-K shapes take the two-pass path, with the same results;
- the codes the next Linear quantizes from Y at that scale equal the
  oracle's codes of Y.
The backward (second half of the file): dX and dW bit-identical to
df_fp8_gemm_bwd's, on the grouped plans (dW unsplit and in K slices) and the
separate launches, and dX's absmax and scale to df_absmax_scale_* of dX.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu


DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def _codes(rows, cols, std, seed, dev):
    x = torch.from_numpy(synth.normal((rows, cols), std, seed=seed)).to(dev).to(torch.bfloat16)
    _, s = df.absmax_scale(x, Fmt.E4M3)
    q, _ = df.quantize_2d(x, s, Fmt.E4M3)
    return q, s


CASES = [
    # M, K, N, output, bias
    (16384, 1600, 6400, "bf16", "bf16"),  # config-4 fc: its Y is the next Linear's X
    (16384, 6400, 1600, "bf16", "bf16"),  # config-4 proj
    (16384, 1600, 4800, "f32", "f32"),
    (4096, 768, 3072, "bf16", None),
    (1, 4, 3, "bf16", "bf16"),
    (129, 272, 257, "f32", "bf16"),
    (1407, 53, 3584, "bf16", "f32"),
    (300, 8192, 200, "bf16", "bf16"),  # a long reduction on a small output
    (16384, 1600, 6400, "f16", "f16"),  # binary16 output (the reference's FP16 layer line)
    (4096, 768, 3072, "f16", None),
    (129, 272, 257, "f16", "f32"),
]


@pytest.mark.parametrize("M,K,N,out,bias", CASES)
def test_fwd_absmax_matches_separate_passes(dev, M, K, N, out, bias):
    seed = 7000 + M + 3 * K + 5 * N
    xq, sx = _codes(M, K, 1.0, seed, dev)
    wq, sw = _codes(N, K, 0.02, seed + 1, dev)
    b = None
    if bias is not None:
        b = torch.from_numpy(synth.normal((N,), 0.1, seed=seed + 2)).to(dev).to(DT[bias])
    dt = DT[out]
    for fmt in (Fmt.E4M3, Fmt.E5M2):
        y, am, sc = df.gemm_fwd_absmax(xq, wq, K, sx, sw, bias=b, out_dtype=dt, next_fmt=fmt)
        y_ref = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=b, out_dtype=dt)
        assert torch.equal(_bits(y), _bits(y_ref)), f"{M}x{K}x{N}: Y"
        am_ref, sc_ref = df.absmax_scale(y_ref, fmt)
        assert am.view(torch.int32).item() == am_ref.view(torch.int32).item(), f"{M}x{K}x{N} fmt={int(fmt)}: absmax"
        assert sc.view(torch.int32).item() == sc_ref.view(torch.int32).item(), f"{M}x{K}x{N} fmt={int(fmt)}: scale"


def test_config4_shapes_take_the_fused_kernel(dev):
    """The fused fold runs only on the unsplit 256x256 persistent plan; the
    config-4 forward shapes take it."""
    for M, K, N in ((16384, 1600, 6400), (16384, 6400, 1600), (16384, 1600, 4800), (16384, 1600, 1600)):
        kernel, split = df.gemm_plan(M, N, K, df.round16(K), df.round16(K), None,
                                     int(df.lib().df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K)))
        assert kernel == df.GemmKernel.PERSISTENT and split == 1, (M, K, N)


def test_next_linear_codes_from_fused_scale(dev):
    """fc1 -> fc2 as the reference block chains them: fc2's X codes, made at
    the fused scale, equal the oracle's codes of fc1's Y."""
    M, K, N = 2048, 1600, 6400
    xq, sx = _codes(M, K, 1.0, 91, dev)
    wq, sw = _codes(N, K, 0.02, 92, dev)
    y, am, sc = df.gemm_fwd_absmax(xq, wq, K, sx, sw, out_dtype=torch.bfloat16, next_fmt=Fmt.E4M3)
    q, _ = df.quantize_2d(y, sc, Fmt.E4M3)
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16)
    vals = orc.bf16_to_f32(yb).reshape(M, N)
    s = orc.scale(orc.absmax(vals), int(Fmt.E4M3))
    assert sc.item() == np.float32(s)
    assert np.array_equal(q.cpu().numpy()[:, :N], orc.quantize(vals, s, int(Fmt.E4M3)))


@pytest.mark.parametrize("out", ["bf16", "f16", "f32"])
def test_fused_fold_skips_inf_and_nan(dev, out):
    """On the fused plan, a Y with NaN rows (a NaN code in X) and overflowed
    values (+-inf from scales whose product pushes the largest outputs past
    the type's range) gives the absmax over its finite values only, as
    df_absmax_scale does; a Y with no finite value gives absmax 0."""
    M, K, N = 4096, 768, 3072
    ws = int(df.lib().df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K))
    assert df.gemm_plan(M, N, K, K, K, None, ws) == (df.GemmKernel.PERSISTENT, 1)
    dt = DT[out]
    xq, sx = _codes(M, K, 1.0, 501, dev)
    wq, sw = _codes(N, K, 0.02, 502, dev)
    top = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, out_dtype=torch.float32).abs().max().item()
    f = 2.0 * torch.finfo(dt).max / top  # the largest |Y| lands near twice the type's maximum
    f1 = 2.0 ** int(np.log2(f) / 2)
    sx2, sw2 = sx * f1, sw * (f / f1)
    xq[123, 5] = 0x7F  # e4m3 NaN
    xq[3000, 0] = 0xFF
    for xin in (xq, torch.full_like(xq, 0x7F)):
        y, am, sc = df.gemm_fwd_absmax(xin, wq, K, sx2, sw2, out_dtype=dt, next_fmt=Fmt.E4M3)
        y_ref = df.gemm_nt(xin, Fmt.E4M3, wq, Fmt.E4M3, K, sx2, sw2, out_dtype=dt)
        assert torch.equal(_bits(y), _bits(y_ref))
        assert torch.isnan(y_ref).any()
        if xin is xq:
            assert torch.isinf(y_ref).any() and torch.isfinite(y_ref).any()
        else:
            assert not torch.isfinite(y_ref).any()
        am_ref, sc_ref = df.absmax_scale(y_ref, Fmt.E4M3)
        assert am.view(torch.int32).item() == am_ref.view(torch.int32).item()
        assert sc.view(torch.int32).item() == sc_ref.view(torch.int32).item()
    assert am.item() == 0.0


# ---- the backward mirror: df_fp8_gemm_bwd_absmax.  The reference block's
# backward passes fc2's input gradient straight to fc1 as its output
# gradient (dnn/layers/transformer_block.cu:127-134), so fc1's just-in-time
# dY scale is the absmax of fc2's dX.

def _operand(dev, shape, std, seed, fmt, want_q, want_qt):
    x = torch.from_numpy(synth.normal(shape, std, seed=seed)).to(dev)
    _, s = df.absmax_scale(x, fmt)
    q, qt = df.quantize_2d(x, s, fmt, want_q=want_q, want_qt=want_qt)
    return q, qt, s


def _bwd_operands(dev, M, K, N, seed):
    dyq, dyt, sdy = _operand(dev, (M, N), 1e-3, seed, Fmt.E5M2, True, True)
    _, wt, sw = _operand(dev, (N, K), 0.02, seed + 1, Fmt.E4M3, False, True)
    _, xt, sx = _operand(dev, (M, K), 1.0, seed + 2, Fmt.E4M3, False, True)
    return dyq, wt, dyt, xt, sdy, sw, sx


BWD_CASES = [
    # M, K, N: the config-4 Linears (grouped; dW unsplit or in K slices, as the plan decides), a
    # config-3 one, small and ragged ones (grouped too), and small dX with long reductions, whose
    # dX would be cut into K slices: those take the two separate launches
    (16384, 1600, 4800), (16384, 1600, 1600), (16384, 1600, 6400), (16384, 6400, 1600),
    (8192, 768, 2304), (129, 272, 257), (1, 4, 3), (1407, 53, 3584), (300, 64, 8192),
]


@pytest.mark.parametrize("M,K,N", BWD_CASES)
def test_bwd_absmax_matches_separate_passes(dev, M, K, N):
    print(f"bwd absmax {M}x{K}x{N} plan {df.gemm_bwd_plan(M, N, K)}", flush=True)
    dyq, wt, dyt, xt, sdy, sw, sx = _bwd_operands(dev, M, K, N, seed=7100 + M + 3 * K + 5 * N)
    for dx_dt, dw_dt, fmt in ((torch.bfloat16, torch.float32, Fmt.E5M2), (torch.float32, torch.bfloat16, Fmt.E4M3),
                              (torch.float16, torch.float16, Fmt.E5M2)):
        dX, dW, am, sc = df.gemm_bwd_absmax(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, dx_dtype=dx_dt, dw_dtype=dw_dt,
                                            next_fmt=fmt)
        dX1, dW1 = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, dx_dtype=dx_dt, dw_dtype=dw_dt)
        assert torch.equal(_bits(dX), _bits(dX1)), f"{M}x{K}x{N} {dx_dt}: dX"
        assert torch.equal(_bits(dW), _bits(dW1)), f"{M}x{K}x{N} {dx_dt}: dW"
        am1, sc1 = df.absmax_scale(dX1, fmt)
        assert am.view(torch.int32).item() == am1.view(torch.int32).item(), f"{M}x{K}x{N}: absmax"
        assert sc.view(torch.int32).item() == sc1.view(torch.int32).item(), f"{M}x{K}x{N}: scale"


def test_bwd_absmax_cases_cover_every_plan(dev):
    """The cases above include a grouped launch with dW unsplit, one with dW
    in K slices (the fold runs in both kernels) and the separate launches."""
    kinds = set()
    for M, K, N in BWD_CASES:
        grouped, slices = df.gemm_bwd_plan(M, N, K)
        kinds.add("separate" if not grouped else "split" if slices > 1 else "grouped")
    assert kinds == {"separate", "grouped", "split"}, kinds


def test_fc1_dy_codes_from_fused_scale(dev):
    """fc2's backward -> fc1's dY as the reference block chains them: fc1's
    dY codes at the fused scale, with the bias gradient's column sums, equal
    the oracle's of fc2's dX."""
    M, K, N = 2048, 6400, 1600
    dyq, wt, dyt, xt, sdy, sw, sx = _bwd_operands(dev, M, K, N, seed=93)
    dX, _, am, sc = df.gemm_bwd_absmax(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, dx_dtype=torch.bfloat16,
                                       next_fmt=Fmt.E5M2)
    q, qt = df.quantize_2d(dX, sc, Fmt.E5M2, want_q=True, want_qt=True)
    vals = orc.bf16_to_f32(dX.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(M, K)
    s = orc.scale(orc.absmax(vals), int(Fmt.E5M2))
    assert sc.item() == np.float32(s)
    flat = orc.quantize(vals, s, int(Fmt.E5M2))
    assert np.array_equal(q.cpu().numpy()[:, :K], flat)
    assert np.array_equal(qt.cpu().numpy()[:, :M], np.ascontiguousarray(flat.T))


@pytest.mark.parametrize("out", ["bf16", "f16", "f32"])
def test_bwd_fold_skips_inf_and_nan(dev, out):
    """On a grouped plan: dX with NaN rows (a NaN code in dY) and overflowed
    values gives the absmax of its finite values only (an f16 dX groups with
    an f16 dW)."""
    M, K, N = 16384, 1600, 6400
    assert df.gemm_bwd_plan(M, N, K)[0]
    dt = DT[out]
    dwt = torch.float16 if out == "f16" else torch.float32
    dyq, wt, dyt, xt, sdy, sw, sx = _bwd_operands(dev, M, K, N, seed=95)
    top = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx)[0].abs().max().item()
    f = 2.0 * torch.finfo(dt).max / top
    f1 = 2.0 ** int(np.log2(f) / 2)
    sdy2, sw2 = sdy * f1, sw * (f / f1)
    dyq[77, 3] = 0x7F  # e5m2 NaN
    dX, dW, am, sc = df.gemm_bwd_absmax(dyq, wt, dyt, xt, M, N, K, sdy2, sw2, sx, dx_dtype=dt, dw_dtype=dwt,
                                        next_fmt=Fmt.E5M2)
    dX1, dW1 = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy2, sw2, sx, dx_dtype=dt, dw_dtype=dwt)
    assert torch.equal(_bits(dX), _bits(dX1))
    assert torch.equal(_bits(dW), _bits(dW1))
    assert torch.isnan(dX1).any() and torch.isinf(dX1).any() and torch.isfinite(dX1).any()
    am1, sc1 = df.absmax_scale(dX1, Fmt.E5M2)
    assert am.view(torch.int32).item() == am1.view(torch.int32).item()
    assert sc.view(torch.int32).item() == sc1.view(torch.int32).item()
