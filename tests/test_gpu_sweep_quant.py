"""Seeded random-shape sweep of the quantize entry points against the oracle.

The shapes are drawn once from a fixed seed: log-uniform sizes mixed with
sizes one either side of a 128-row / 128-column tile edge, so that ragged
tile grids, single rows and columns, and grids of hundreds of tiles all
occur.  Inputs are bf16 or binary16 values of N(0, 1) with planted NaN,
+-inf, -0 and near-overflow values (the helpers of test_gpu_quant2d_wide).

Per shape and input type, for both fp8 formats:
- df_absmax_scale: absmax and scale bit-exact against the oracle
  (non-finite values skipped, rule D1/D2);
- df_quantize_2d: the row copy and the transposed copy bit-exact against
  the oracle's codes at that scale, their padding zero;
- df_quantize_2d_colsum: the same codes from a row stride that is not a
  multiple of 8 elements (the element-wise load path), column sums
  bit-identical between the two layouts and within 1e-4 of the oracle's db
  (dnn/layers/fully_connected_layer.cu:91-106), on an input without
  non-finite values;
- df_quantize_2d_delayed: codes at the scale the history held, then the
  history and the next scale bit-exact against the oracle's;
- the LayerNorm producer (fp32, bf16, f16 inputs): y against the oracle and
  the fused codes equal to the 2-D quantize of that y.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt
from oracle import pyoracle as orc
from test_gpu_layernorm import case as ln_case, host_f32, oracle_y
from test_gpu_quant2d_wide import check_codes, make, strided

pytestmark = pytest.mark.gpu


def _draw_shapes(count=12, seed=20261203):
    rng = np.random.default_rng(seed)

    def one():
        if rng.random() < 0.5:
            return int(np.exp(rng.uniform(0.0, np.log(3000.0))))
        return max(1, 128 * int(rng.integers(1, 20)) + int(rng.integers(-1, 2)))

    shapes = []
    while len(shapes) < count:
        s = (one(), one())
        if s not in shapes:
            shapes.append(s)
    return shapes


SHAPES = _draw_shapes()


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_sweep_quantize_2d(dev, rows, cols, kind):
    seed = 3000 + rows * 7 + cols
    xd, _, vals = make(dev, rows, cols, kind, seed=seed)
    clean_d, _, clean = make(dev, rows, cols, kind, seed=seed + 1, std=1e-2, specials=False)
    for fmt in (Fmt.E4M3, Fmt.E5M2):
        what = f"{kind} {rows}x{cols} fmt={int(fmt)}"
        print(what, flush=True)
        am, sc = df.absmax_scale(xd, fmt)
        a_ref = orc.absmax(vals)
        s_ref = np.float32(orc.scale(a_ref, int(fmt)))
        assert am.cpu().numpy().view(np.uint32)[0] == np.float32(a_ref).view(np.uint32), f"{what}: absmax"
        assert sc.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32), f"{what}: scale"
        q, qt = df.quantize_2d(xd, sc, fmt, want_q=True, want_qt=True)
        check_codes(q, qt, orc.quantize(vals, float(s_ref), int(fmt)), rows, cols, what)

        s2 = torch.tensor([float(np.float32(orc.scale(orc.absmax(clean), int(fmt))))], device=dev)
        qa, qta, csa = df.quantize_2d(clean_d, s2, fmt, want_q=True, want_qt=True, colsum=True)
        qb, qtb, csb = df.quantize_2d(strided(clean_d, 5), s2, fmt, want_q=True, want_qt=True, colsum=True)
        check_codes(qa, qta, orc.quantize(clean, float(s2.item()), int(fmt)), rows, cols, what + " colsum")
        assert torch.equal(qa, qb) and torch.equal(qta, qtb), f"{what}: strided codes differ"
        assert torch.equal(csa.view(torch.int32), csb.view(torch.int32)), f"{what}: strided column sums differ"
        assert orc.rel_err(csa.cpu().numpy(), orc.fc_backward_bias(clean)) <= 1e-4, f"{what}: column sums"

        length = 3
        ds = df.DelayedScale(fmt, length, dev)
        hist = np.zeros(length, np.float32)
        scale = np.float32(1.0)
        for p, (xin, v) in enumerate(((xd, vals), (clean_d, clean))):
            out = ds.quantize_2d(xin, want_q=True, want_qt=True, colsum=False)
            check_codes(out[0], out[1], orc.quantize(v, float(scale), int(fmt)), rows, cols, f"{what} delayed {p}")
            scale = np.float32(orc.history_push(hist, orc.absmax(v), int(fmt)))
            torch.cuda.synchronize()
            assert np.array_equal(ds.history.cpu().numpy().view(np.uint32), hist.view(np.uint32)), \
                f"{what} delayed {p}: history"
            assert ds.scale.cpu().numpy().view(np.uint32)[0] == scale.view(np.uint32), f"{what} delayed {p}: scale"


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_sweep_layernorm_quantize(dev, rows, cols, kind):
    """The LayerNorm producer on the same shapes, with gamma and beta:
    y against the oracle's restatement of layer_norm_forward_kernel
    (dnn/layers/layer_norm_layer.cu:26-63; fp32 within 1e-5 of the unit
    scale, bf16 / f16 within one step of the type), and for both formats the
    fused codes bit-identical to the 2-D quantize of that y, at the oracle's
    scale of absmax(y)."""
    xd, gd, bd, xh, gh, bh = ln_case(rows, cols, kind, True, dev, 5000 + rows * 7 + cols)
    y0 = df.layernorm(xd, gd, bd, eps=1e-5)
    y0h = host_f32(y0)
    ref = oracle_y(xh, gh, bh, kind)
    unit = np.abs(gh).max() + 1.0
    if kind == "f32":
        assert np.abs(y0h - ref).max() <= 1e-5 * unit, f"{rows}x{cols}: y"
    else:
        step = 2 ** -7 if kind == "bf16" else 2 ** -10
        assert (np.abs(y0h - ref) <= np.abs(ref) * step + 1e-6 * unit).all(), f"{rows}x{cols}: y"
    for fmt in (Fmt.E4M3, Fmt.E5M2):
        y, q, qt, s = df.layernorm(xd, gd, bd, eps=1e-5, fmt=fmt, want_y=True, want_q=True, want_qt=True)
        torch.cuda.synchronize()
        same = torch.equal(y, y0) if kind == "f32" else torch.equal(y.view(torch.int16), y0.view(torch.int16))
        assert same, f"{rows}x{cols} fmt={int(fmt)}: fused y"
        s_exp = np.float32(orc.scale(orc.absmax(np.ascontiguousarray(y0h)), int(fmt)))
        assert s.cpu().numpy().view(np.uint32)[0] == s_exp.view(np.uint32), f"{rows}x{cols} fmt={int(fmt)}: scale"
        q0, qt0 = df.quantize_2d(y0, s, fmt, want_q=True, want_qt=True)
        assert torch.equal(q, q0) and torch.equal(qt, qt0), f"{rows}x{cols} fmt={int(fmt)}: codes"


def test_sweep_quant_covers_the_edges():
    """Both sides of a tile edge, a single row or column, and wide grids."""
    vals = [v for s in SHAPES for v in s]
    assert any(v % 128 == 1 for v in vals) and any(v % 128 == 127 for v in vals)
    assert any(v < 16 for v in vals) and any(v > 1500 for v in vals)
