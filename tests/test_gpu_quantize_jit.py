"""GPU parity of df_quantize_2d_jit: absmax, scale and the 2-D quantize in
one call, each tile block forming the scale from the absmax partials itself.

Bars (bit-exact throughout):
- absmax and scale equal df_absmax_scale_*'s on the same x, and the
  oracle's (finite values only, rule D1/D2), on inputs with planted NaN,
  +-inf, -0 and near-overflow values, fp32, bf16 and binary16;
- q and qt equal df_quantize_2d's at that scale (and, on the smaller
  shapes, the oracle's codes), padding zero;
- with colsum, codes and column sums equal df_quantize_2d_colsum's;
- shapes: the config-4 X and dY, ragged tile grids, one row, one column,
  one element, and a 288 MB input whose absmax pass runs its block cap;
- empty inputs give absmax 0 and scale 1 (and zero column sums), an input
  with no finite value the same scale;
- calls in a row on one workspace, each smaller than the last, give each
  call's own results.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc
from test_gpu_quant2d_wide import check_codes, make

pytestmark = pytest.mark.gpu


def make_any(dev, rows, cols, kind, seed, specials=True):
    """(device tensor, host fp32 values) with planted specials."""
    if kind != "f32":
        xd, _, vals = make(dev, rows, cols, kind, seed=seed, specials=specials)
        return xd, vals
    x = synth.normal((rows, cols), 1.0, seed=seed)
    if specials and x.size:
        rng = np.random.default_rng(seed)
        idx = rng.integers(0, x.size, 48)
        flat = x.reshape(-1)
        flat[idx[:16]] = np.nan
        flat[idx[16:24]] = np.inf
        flat[idx[24:32]] = -np.inf
        flat[idx[32:40]] = -0.0
        flat[idx[40:48]] = 3e38
    return torch.from_numpy(x).to(dev), x


def two_calls(xd, fmt, colsum=False):
    """df_absmax_scale_* then df_quantize_2d(_colsum): the reference path."""
    am, sc = df.absmax_scale(xd, fmt)
    out = df.quantize_2d(xd, sc, fmt, want_q=True, want_qt=True, colsum=colsum)
    return (am, sc) + tuple(out)


def bits(t):
    return t.view(torch.int32).item()


SHAPES = [(16384, 1600), (129, 257), (1, 3000), (3000, 1), (1, 1), (4096, 4800)]


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_jit_matches_two_calls(dev, rows, cols, kind, fmt):
    print(f"jit {kind} fmt={int(fmt)} {rows}x{cols}", flush=True)
    xd, vals = make_any(dev, rows, cols, kind, seed=4100 + rows + 3 * cols)
    am, sc, q, qt = df.quantize_2d_jit(xd, fmt, want_q=True, want_qt=True)
    am1, sc1, q1, qt1 = two_calls(xd, fmt)
    assert bits(am) == bits(am1) and bits(sc) == bits(sc1)
    assert torch.equal(q, q1) and torch.equal(qt, qt1)
    if rows * cols <= 1 << 20:  # the oracle on the smaller shapes
        s = orc.scale(orc.absmax(vals), int(fmt))
        assert sc.item() == np.float32(s)
        check_codes(q, qt, orc.quantize(vals, s, int(fmt)), rows, cols, f"{kind} {rows}x{cols}")


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(16384, 4800), (16384, 1600), (129, 257), (1, 130)])
def test_jit_colsum_matches_two_calls(dev, rows, cols, kind):
    """The dY form: e5m2 codes and the bias gradient's column sums."""
    print(f"jit colsum {kind} {rows}x{cols}", flush=True)
    xd, _ = make_any(dev, rows, cols, kind, seed=4200 + rows + cols, specials=False)
    am, sc, q, qt, cs = df.quantize_2d_jit(xd, Fmt.E5M2, want_q=True, want_qt=True, colsum=True)
    am1, sc1, q1, qt1, cs1 = two_calls(xd, Fmt.E5M2, colsum=True)
    assert bits(am) == bits(am1) and bits(sc) == bits(sc1)
    assert torch.equal(q, q1) and torch.equal(qt, qt1)
    assert torch.equal(cs.view(torch.int32), cs1.view(torch.int32))


def test_jit_at_the_partials_cap(dev):
    """144 M bf16 values: the absmax pass runs its full block count (the
    cap), and each tile block folds all of their partials."""
    rows, cols = 36864, 4096
    xd = (torch.randn((rows, cols), device=dev) * 0.25).to(torch.bfloat16)
    xd[rows - 1, cols - 1] = 7.5  # the maximum sits in the last block's range
    am, sc, q, qt = df.quantize_2d_jit(xd, Fmt.E4M3, want_q=True, want_qt=False)
    am1, sc1, q1, _ = two_calls(xd, Fmt.E4M3)
    assert am.item() == 7.5
    assert bits(am) == bits(am1) and bits(sc) == bits(sc1)
    assert torch.equal(q, q1)
    del xd, q, q1
    torch.cuda.empty_cache()


@pytest.mark.parametrize("rows,cols", [(0, 5), (5, 0)])
def test_jit_empty(dev, rows, cols):
    xd = torch.empty((rows, cols), dtype=torch.bfloat16, device=dev)
    am, sc, q, qt, cs = df.quantize_2d_jit(xd, Fmt.E4M3, want_q=True, want_qt=True, colsum=True)
    assert am.item() == 0.0 and sc.item() == 1.0
    assert not cs.any()


def test_jit_no_finite_value(dev):
    x = np.full((300, 200), np.nan, np.float32)
    x[::7, ::5] = np.inf
    xd = torch.from_numpy(x).to(dev)
    am, sc, q, qt = df.quantize_2d_jit(xd, Fmt.E4M3, want_q=True, want_qt=True)
    assert am.item() == 0.0 and sc.item() == 1.0
    check_codes(q, qt, orc.quantize(x, 1.0, int(Fmt.E4M3)), 300, 200, "no finite value")


def test_jit_calls_in_a_row_share_the_workspace(dev):
    """Each call's partials overwrite the last call's; nothing carries over."""
    for i, (rows, cols) in enumerate([(8192, 2304), (2048, 768), (100, 70)]):
        xd = (torch.randn((rows, cols), device=dev) * (4.0 - i)).to(torch.bfloat16)
        am, sc, q, qt = df.quantize_2d_jit(xd, Fmt.E4M3, want_q=True, want_qt=True)
        am1, sc1, q1, qt1 = two_calls(xd, Fmt.E4M3)
        assert bits(am) == bits(am1) and bits(sc) == bits(sc1), (rows, cols)
        assert torch.equal(q, q1) and torch.equal(qt, qt1), (rows, cols)
