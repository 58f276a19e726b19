"""GPU parity of df_fp8_gemm_fwd_absmax: the forward GEMM whose Y also gives
its absmax and the next quantize's scale.

The reference's TransformerBlock feeds fc1's output straight into fc2
(dnn/layers/transformer_block.cu:79-81), so fc2's just-in-time scale is the
absmax of fc1's Y.  Bars:
- Y bit-identical to df_fp8_gemm_fwd's on the same codes, bias and output
  type (the fused epilogue only adds a fold);
- absmax and scale bit-identical to df_absmax_scale_bf16 / _f32 over that Y
  (finite values only, as stored, rule D1/D2 for the next format);
- on the config-4 shapes the planner takes the unsplit 256x256 persistent
  kernel (the fused path, asserted through df_fp8_gemm_nt_plan); small,
  ragged and long-K shapes take the two-pass path, with the same results;
- the codes the next Linear quantizes from Y at that scale equal the
  oracle's codes of Y.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu


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
]


@pytest.mark.parametrize("M,K,N,out,bias", CASES)
def test_fwd_absmax_matches_separate_passes(dev, M, K, N, out, bias):
    seed = 7000 + M + 3 * K + 5 * N
    xq, sx = _codes(M, K, 1.0, seed, dev)
    wq, sw = _codes(N, K, 0.02, seed + 1, dev)
    b = None
    if bias is not None:
        b = torch.from_numpy(synth.normal((N,), 0.1, seed=seed + 2)).to(dev)
        b = b.to(torch.bfloat16) if bias == "bf16" else b
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    for fmt in (Fmt.E4M3, Fmt.E5M2):
        y, am, sc = df.gemm_fwd_absmax(xq, wq, K, sx, sw, bias=b, out_dtype=dt, next_fmt=fmt)
        y_ref = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=b, out_dtype=dt)
        assert torch.equal(y.view(torch.int16 if out == "bf16" else torch.int32),
                           y_ref.view(torch.int16 if out == "bf16" else torch.int32)), f"{M}x{K}x{N}: Y"
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


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fused_fold_skips_inf_and_nan(dev, out):
    """On the fused plan, a Y with NaN rows (a NaN code in X) and overflowed
    values (+-inf from scales whose product pushes the largest outputs past
    the type's range) gives the absmax over its finite values only, as
    df_absmax_scale does; a Y with no finite value gives absmax 0."""
    M, K, N = 4096, 768, 3072
    ws = int(df.lib().df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K))
    assert df.gemm_plan(M, N, K, K, K, None, ws) == (df.GemmKernel.PERSISTENT, 1)
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    bits = torch.int16 if out == "bf16" else torch.int32
    xq, sx = _codes(M, K, 1.0, 501, dev)
    wq, sw = _codes(N, K, 0.02, 502, dev)
    top = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, out_dtype=torch.float32).abs().max().item()
    f = 2.0 * 3.4e38 / top  # the largest |Y| lands near twice the type's maximum
    f1 = 2.0 ** int(np.log2(f) / 2)
    sx2, sw2 = sx * f1, sw * (f / f1)
    xq[123, 5] = 0x7F  # e4m3 NaN
    xq[3000, 0] = 0xFF
    for xin in (xq, torch.full_like(xq, 0x7F)):
        y, am, sc = df.gemm_fwd_absmax(xin, wq, K, sx2, sw2, out_dtype=dt, next_fmt=Fmt.E4M3)
        y_ref = df.gemm_nt(xin, Fmt.E4M3, wq, Fmt.E4M3, K, sx2, sw2, out_dtype=dt)
        assert torch.equal(y.view(bits), y_ref.view(bits))
        assert torch.isnan(y_ref).any()
        if xin is xq:
            assert torch.isinf(y_ref).any() and torch.isfinite(y_ref).any()
        else:
            assert not torch.isfinite(y_ref).any()
        am_ref, sc_ref = df.absmax_scale(y_ref, Fmt.E4M3)
        assert am.view(torch.int32).item() == am_ref.view(torch.int32).item()
        assert sc.view(torch.int32).item() == sc_ref.view(torch.int32).item()
    assert am.item() == 0.0
