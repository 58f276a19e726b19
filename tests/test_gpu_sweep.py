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
- the bf16 outputs the round-to-nearest-even image of the fp32 ones;
- the grouped backward's dX bit-identical to a separate dX launch on the
  same codes, and dW within 1e-5 of a separate dW launch (the two plans may
  cut its K range into different slices).
"""
import numpy as np
import pytest

from test_gpu_gemm import forward_case, grouped_case

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


def test_sweep_covers_the_edges():
    """The drawn shapes reach both sides of the tile edges and every size class."""
    vals = [v for s in SHAPES for v in s]
    assert any(v % 256 == 1 for v in vals) and any(v % 256 == 255 for v in vals)
    assert any(v < 64 for v in vals) and any(v > 2048 for v in vals)
