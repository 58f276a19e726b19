"""GPU parity of the LayerNorm producer with the fused quantize
(df_layernorm, df_layernorm_quantize, df_layernorm_quantize_delayed).

Bars:
  - y against the oracle's restatement of layer_norm_forward_kernel
    (dnn/layers/layer_norm_layer.cu:26-63): within 1e-5 of the row's unit
    scale for fp32 (different summation order), within one bf16 step for
    bf16, within one binary16 step for f16 (LayerNormLayer<__half>,
    layer_norm_layer.cu:123; the oracle's fp32 y rounded by dfo_convert);
  - the fused codes bit-identical to df_quantize_2d applied to the y that
    df_layernorm writes, at a scale bit-identical to the oracle's D1/D2
    scale of absmax(y): the fusion changes no value;
  - delayed: codes at the history scale, absmax(y) pushed.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

SHAPES = [(1, 8), (3, 7), (37, 100), (129, 257), (256, 1600), (1000, 768)]


def dev_tensor(x, kind, dev):
    if kind == "f32":
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)
    if kind == "f16":
        return torch.from_numpy(orc.convert(x, 0, 1).view(np.int16)).to(dev).view(torch.float16)
    return torch.from_numpy(synth.f32_to_bf16_bits(x).view(np.int16)).to(dev).view(torch.bfloat16)


def oracle_y(xh, gh, bh, kind):
    ref = orc.layernorm(xh, gh, bh, eps=1e-5, round_bf16=(kind == "bf16"))
    if kind == "f16":  # the fp32 result rounded to nearest even binary16
        ref = orc.convert(orc.convert(ref, 0, 1), 1, 0).reshape(ref.shape)
    return ref


def host_f32(t):
    return t.float().cpu().numpy()


def case(rows, cols, kind, affine, dev, seed):
    x = synth.normal((rows, cols), 2.0, seed=seed, mean=0.5)
    g = synth.normal((cols,), 0.2, seed=seed + 1, mean=1.0) if affine else None
    b = synth.normal((cols,), 0.5, seed=seed + 2) if affine else None
    xd = dev_tensor(x, kind, dev)
    gd = dev_tensor(g, kind, dev) if affine else None
    bd = dev_tensor(b, kind, dev) if affine else None
    # the values the kernel reads
    xh, gh, bh = host_f32(xd), (host_f32(gd) if affine else None), (host_f32(bd) if affine else None)
    return xd, gd, bd, xh, gh, bh


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("affine", [False, True])
def test_layernorm_matches_oracle(dev, kind, affine):
    for i, (rows, cols) in enumerate(SHAPES):
        xd, gd, bd, xh, gh, bh = case(rows, cols, kind, affine, dev, 500 + i)
        y = host_f32(df.layernorm(xd, gd, bd, eps=1e-5))
        ref = oracle_y(xh, gh, bh, kind)
        unit = 1.0 if not affine else np.abs(gh).max() + 1.0
        if kind == "f32":
            assert np.abs(y - ref).max() <= 1e-5 * unit, f"{rows}x{cols}"  # ~10 ulp of max|y|
        else:  # at most one step of the 2-byte type apart (plus rounding near 0)
            step = 2 ** -7 if kind == "bf16" else 2 ** -10
            assert (np.abs(y - ref) <= np.abs(ref) * step + 1e-6 * unit).all(), f"{rows}x{cols}"


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_fused_quantize_equals_layernorm_then_quantize(dev, kind, fmt):
    for i, (rows, cols) in enumerate(SHAPES):
        xd, gd, bd, xh, gh, bh = case(rows, cols, kind, True, dev, 600 + i)
        y0 = df.layernorm(xd, gd, bd)
        y, q, qt, s = df.layernorm(xd, gd, bd, fmt=fmt, want_y=True, want_q=True, want_qt=True)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16) if kind != "f32" else y,
                           y0.view(torch.int16) if kind != "f32" else y0), f"{rows}x{cols}: y"
        yh = host_f32(y0)
        s_exp = np.float32(orc.scale(orc.absmax(np.ascontiguousarray(yh)), int(fmt)))
        assert s.item() == s_exp, f"{rows}x{cols}: scale"
        q0, qt0 = df.quantize_2d(y0, s, fmt, want_q=True, want_qt=True)
        assert torch.equal(q, q0) and torch.equal(qt, qt0), f"{rows}x{cols}: codes"
        # codes only (y never written) are the same
        _, q2, qt2, s2 = df.layernorm(xd, gd, bd, fmt=fmt, want_y=False, want_q=True, want_qt=True)
        assert torch.equal(q2, q0) and torch.equal(qt2, qt0) and torch.equal(s2, s)


def test_unaligned_rows_and_no_affine(dev):
    # ldx not a multiple of 16 bytes: the scalar load path
    base = torch.from_numpy(synth.normal((50, 103), 1.0, seed=700)).to(dev)
    x = base[:, :101]
    assert x.stride(0) == 103
    y0 = df.layernorm(x.contiguous())
    y, q, qt, s = df.layernorm(x, fmt=Fmt.E4M3, want_y=True, want_q=True, want_qt=True)
    assert torch.equal(y, y0)
    q0, qt0 = df.quantize_2d(y0, s, Fmt.E4M3, want_q=True, want_qt=True)
    assert torch.equal(q, q0) and torch.equal(qt, qt0)


def test_delayed_layernorm(dev):
    st = df.DelayedScale(Fmt.E4M3, 4, dev)
    hist = np.zeros(4, np.float32)
    scale = np.float32(1.0)
    for i, mag in enumerate((1.0, 3.0, 0.5)):
        xd, gd, bd, xh, gh, bh = case(300, 640, "bf16", True, dev, 800 + i)
        gd = gd * mag
        y, q, qt, s_used = df.layernorm(xd, gd, bd, fmt=Fmt.E4M3, want_y=True, want_q=True, want_qt=True,
                                        delayed=st)
        torch.cuda.synchronize()
        assert s_used.item() == scale
        q0, qt0 = df.quantize_2d(y, s_used, Fmt.E4M3, want_q=True, want_qt=True)
        assert torch.equal(q, q0) and torch.equal(qt, qt0), f"pass {i}"
        scale = np.float32(orc.history_push(hist, orc.absmax(np.ascontiguousarray(host_f32(y))), 0))
        assert st.scale.item() == scale
        assert np.array_equal(st.history.cpu().numpy(), hist)


def test_gpt2_xl_shape(dev):
    """M = 16384 tokens x d = 1600 (the layer the reference's launch of
    norm_size threads per block cannot run: 1600 > 1024)."""
    xd, gd, bd, *_ = case(16384, 1600, "bf16", True, dev, 900)
    y0 = df.layernorm(xd, gd, bd)
    _, q, qt, s = df.layernorm(xd, gd, bd, fmt=Fmt.E4M3, want_y=False, want_q=True, want_qt=True)
    q0, qt0 = df.quantize_2d(y0, s, Fmt.E4M3, want_q=True, want_qt=True)
    torch.cuda.synchronize()
    assert torch.equal(q, q0) and torch.equal(qt, qt0)
    # every row normalised: mean ~ beta-free check on a sample without the affine map
    yp = df.layernorm(xd[:64]).float()
    assert yp.mean(dim=1).abs().max().item() < 1e-2 and (yp.var(dim=1, unbiased=False) - 1).abs().max().item() < 2e-2


def test_argument_errors(dev):
    x = torch.zeros((4, 8), dtype=torch.float32, device=dev)
    g = torch.ones(8, dtype=torch.float32, device=dev)
    with pytest.raises(df.DFError) as ei:  # gamma without beta
        df.layernorm(x, g, None)
    assert ei.value.status == -1
    with pytest.raises(df.DFError) as ei:
        df.call("df_layernorm", 0, x.data_ptr(), 4, 8, 8, None, None, 1e-5, x.data_ptr(), 8, x.data_ptr(), 0, None)
    assert ei.value.status == -5
    with pytest.raises(df.DFError) as ei:
        df.call("df_layernorm", 2, x.data_ptr(), 4, 8, 8, None, None, 1e-5, x.data_ptr(), 8, x.data_ptr(), 4096,
                None)  # int8
    assert ei.value.status == -2
