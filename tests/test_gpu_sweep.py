"""Seeded random-shape sweep of the fp8 Linear path against the oracle.

The shape-specific GPU tests pin the configurations and the edges they were
written for.  This sweep draws (M, K, N) triples once from a fixed seed,
mixing log-uniform sizes with sizes one either side of the 128- and 256-wide
tile edges, so that the planner's choices (persistent 256x256 or 256x128
tiles, split-K, grouped or separate backward, the tiled fallback for small
outputs) and every kernel's edge handling (rows past M, a K tail inside a
128-byte step, a last column tile partly outside N) meet shapes nobody
picked by hand.

Per shape, on the same seeded operands (X ~ N(0, 1), W ~ N(0, 0.02),
dY ~ N(0, 1e-3), fp32 in, GPU-quantized):
- every code and scale bit-exact against the oracle (2-D quantize, row and
  transposed copies);
- forward Y with an fp32 bias, dX and dW through df_fp8_gemm_bwd, within the
  1e-4 normwise bar of the oracle's restatement of
  dnn/layers/fully_connected_layer.cu:14-89 (every row up to 2048 rows,
  else the first, last and two seeded rows of every 256-row band);
- the bf16 outputs the round-to-nearest-even image of the fp32 ones, and the
  forward from bf16 X, W and bias with bf16 or f16 bias and output as the
  layer calls it;
- the grouped backward's dX bit-identical to a separate dX launch on the
  same codes, and dW within 1e-5 of a separate dW launch (the two plans may
  cut its K range into different slices).
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt
from oracle import pyoracle as orc
from test_gpu_gemm import TOL, bf16_operands, check_bf16_image, forward_case, grouped_case

pytestmark = pytest.mark.gpu


def _draw_shapes(count=24, seed=20261202):
    rng = np.random.default_rng(seed)

    def one():
        if rng.random() < 0.5:
            return int(np.exp(rng.uniform(0.0, np.log(4096.0))))
        edge = int(rng.choice([128, 256])) * int(rng.integers(1, 17))
        return max(1, edge + int(rng.integers(-1, 2)))

    shapes = []
    while len(shapes) < count:
        M, K, N = one(), one(), one()
        if (M, K, N) not in shapes:
            shapes.append((M, K, N))
    return shapes


SHAPES = _draw_shapes()


def _rows(n):
    return None if n <= 2048 else "bands"


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_sweep_forward(dev, M, K, N):
    forward_case(dev, M, K, N, seed=1000 + M * 3 + K * 5 + N * 7, rows=_rows(M))


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_sweep_grouped_backward(dev, M, K, N):
    grouped_case(dev, M, K, N, seed=2000 + M * 3 + K * 5 + N * 7, rows=_rows(M), wrows=_rows(N),
                 wcols=_rows(K), out16=True)


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_sweep_forward_two_byte_bias_and_output(dev, M, K, N):
    """The forward as the Linear layer calls it: bf16 X, W and bias quantized
    on the GPU (codes and scales bit-exact against the oracle), then
    - a bf16 bias with bf16 output: the RNE image of the fp32 output of the
      same call, which is within 1e-4 of the oracle (this covers the bias
      whose odd length leaves its last element outside the dword DMA);
    - an f16 bias with f16 output: bit-identical to an fp32 bias of the same
      values with f16 output, and the RNE binary16 image of the fp32 output."""
    seed = 4000 + M * 3 + K * 5 + N * 7
    Xb, Wb, bb, Xd, Wd, bd = bf16_operands(dev, M, K, N, seed)
    _, sx = df.absmax_scale(Xd, Fmt.E4M3)
    _, sw = df.absmax_scale(Wd, Fmt.E4M3)
    xq, _ = df.quantize_2d(Xd, sx, Fmt.E4M3)
    wq, _ = df.quantize_2d(Wd, sw, Fmt.E4M3)
    s_x, s_w = orc.scale(orc.absmax(Xb), 0), orc.scale(orc.absmax(Wb), 0)
    assert sx.item() == np.float32(s_x) and sw.item() == np.float32(s_w)
    cx, cw = orc.quantize(Xb, s_x, 0), orc.quantize(Wb, s_w, 0)
    assert np.array_equal(xq.cpu().numpy()[:, :K], cx) and np.array_equal(wq.cpu().numpy()[:, :K], cw)
    bvals = orc.bf16_to_f32(bb)
    Y16 = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=bd, out_dtype=torch.bfloat16)
    Y32 = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=torch.from_numpy(bvals).to(dev))
    check_bf16_image(Y32, Y16)
    ref = orc.fc_forward(orc.dequantize(cx, s_x, 0), orc.dequantize(cw, s_w, 0), bvals)
    err = orc.rel_err(Y32.cpu().numpy(), ref)
    assert err <= TOL, f"bf16 forward M={M} K={K} N={N}: {err:.3e}"
    # f16: the bf16 bias rounded to binary16 (hb), and the same values widened
    # to fp32 (hb32)
    hbits = orc.convert(np.ascontiguousarray(bvals), 0, 1)
    hvals = orc.convert(hbits, 1, 0)
    hb = torch.from_numpy(np.ascontiguousarray(hbits, np.uint16).view(np.int16)).to(dev).view(torch.float16)
    Yh = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=hb, out_dtype=torch.float16)
    hb32 = torch.from_numpy(np.ascontiguousarray(hvals, np.float32)).to(dev)
    Yh32b = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=hb32, out_dtype=torch.float16)
    assert torch.equal(Yh.view(torch.int16), Yh32b.view(torch.int16))
    Y32h = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=hb32).cpu().numpy()
    img = orc.convert(np.ascontiguousarray(Y32h), 0, 1).reshape(Y32h.shape)
    assert np.array_equal(Yh.view(torch.int16).cpu().numpy().view(np.uint16), img)


def test_sweep_covers_the_edges():
    """The drawn shapes reach both sides of the tile edges and every size class."""
    vals = [v for s in SHAPES for v in s]
    assert any(v % 256 == 1 for v in vals) and any(v % 256 == 255 for v in vals)
    assert any(v < 64 for v in vals) and any(v > 2048 for v in vals)
