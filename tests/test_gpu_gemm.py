"""GPU parity of the fp8 Linear GEMMs (forward, dX, dW) and db.

Bar (the path's GEMM contract D6): the GPU output is within
normwise relative error 1e-4 (max|y - r| / max|r|) of the reference's
fp32-accumulated product of the same dequantized operands, computed by the
oracle's restatement of dnn/layers/fully_connected_layer.cu:14-106.  Codes
feeding the GEMM are first checked bit-exact.  bf16 outputs are checked to
be the round-to-nearest-even image of the fp32 result of the same kernel.
At full configuration sizes the oracle runs on sampled rows chosen so that
every 256-row band of the output (one band of the persistent kernel's
256x256 tiles) is checked at its first and last row and at two seeded rows
between; dW samples hit every 256 x 256 tile.  A sampled output row spans
every column tile, so every output tile is compared with the oracle.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-4


def dev_f32(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)


def quant_operand(x, fmt, dev, want_q=True, want_qt=False):
    """GPU absmax/scale/2-D quantize of a host fp32 matrix; returns the
    device codes plus the oracle's scale and dequantized matrix (after
    checking the GPU codes and scale bit-exact)."""
    xd = dev_f32(x, dev)
    am, sc = df.absmax_scale(xd, fmt)
    q, qt = df.quantize_2d(xd, sc, fmt, want_q=want_q, want_qt=want_qt)
    s = orc.scale(orc.absmax(x), int(fmt))
    assert sc.cpu().numpy().view(np.uint32)[0] == np.float32(s).view(np.uint32)
    codes = orc.quantize(x, s, int(fmt))
    rows, cols = x.shape
    if q is not None:
        assert np.array_equal(q.cpu().numpy()[:, :cols], codes)
    if qt is not None:
        assert np.array_equal(qt.cpu().numpy()[:, :rows], np.ascontiguousarray(codes.T))
    deq = orc.dequantize(codes, s, int(fmt), "f32")
    return q, qt, sc, deq


def band_rows(M, seed, band=256, extra=2):
    """First and last row of every `band`-row band of an M-row output plus
    `extra` seeded rows inside each band (sorted, unique)."""
    rng = np.random.default_rng(seed)
    rows = set()
    for b0 in range(0, M, band):
        b1 = min(b0 + band, M) - 1
        rows.update((b0, b1))
        rows.update(int(r) for r in rng.integers(b0, b1 + 1, size=extra))
    return np.array(sorted(rows), dtype=np.int64)


def pick_rows(M, rows, seed):
    """None: every row; "bands": band_rows; an int: that many seeded rows."""
    if rows is None:
        return np.arange(M)
    if isinstance(rows, str):
        assert rows == "bands"
        return band_rows(M, seed)
    return np.sort(np.random.default_rng(seed).choice(M, rows, replace=False))


def check_bf16_image(c32, c16):
    exp = synth.f32_to_bf16_bits(c32.cpu().numpy())
    got = c16.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, exp)


def forward_case(dev, M, K, N, seed, bias=True, rows=None):
    X = synth.normal((M, K), 1.0, seed=seed)
    W = synth.normal((N, K), 0.02, seed=seed + 1)
    b = synth.normal((N,), 0.1, seed=seed + 2) if bias else None
    xq, _, sx, Xd = quant_operand(X, Fmt.E4M3, dev)
    wq, _, sw, Wd = quant_operand(W, Fmt.E4M3, dev)
    bd = dev_f32(b, dev) if bias else None
    Y = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=bd)
    Yh = Y.cpu().numpy()
    idx = pick_rows(M, rows, seed)
    ref = orc.fc_forward(Xd[idx], Wd, b)
    err = orc.rel_err(Yh[idx], ref)
    assert err <= TOL, f"forward M={M} K={K} N={N}: rel err {err:.3e}"
    Y16 = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=bd, out_dtype=torch.bfloat16)
    check_bf16_image(Y, Y16)
    return err


def test_reference_known_answer(dev):
    """fully_connected_layer_test.cu:266-284: W={1,2,3,4}, b={.5,-.5}, x={1,2}."""
    X = np.array([[1, 2]], np.float32)
    W = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([0.5, -0.5], np.float32)
    xq, _, sx, Xd = quant_operand(X, Fmt.E4M3, dev)
    wq, _, sw, Wd = quant_operand(W, Fmt.E4M3, dev)
    Y = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, 2, sx, sw, bias=dev_f32(b, dev)).cpu().numpy()
    ref = orc.fc_forward(Xd, Wd, b)
    assert orc.rel_err(Y, ref) <= TOL
    assert np.all(Y != 0.0)  # NonzeroInputGivesNonzeroOutput
    # fp8 e4m3 rounds W[1,0] = 3 -> 336 (tie) -> 320: y1 = 20/7 + 8 - 0.5
    np.testing.assert_allclose(Y[0], [5.5, 20.0 / 7.0 + 7.5], rtol=1e-6)


@pytest.mark.parametrize("M,K,N", [(1, 4, 3), (1, 5, 2), (3, 7, 5), (64, 768, 3072), (100, 40, 50),
                                   (129, 272, 257), (256, 128, 128), (17, 1600, 33)])
def test_forward_shapes(dev, M, K, N):
    forward_case(dev, M, K, N, seed=M * 7 + K * 3 + N)


def test_forward_no_bias(dev):
    forward_case(dev, 70, 96, 130, seed=5, bias=False)


def backward_case(dev, M, K, N, seed, rows=None, wrows=None, wcols=None):
    """dX = dY . W (e5m2 x e4m3) and dW = dY^T . X; db = column sums of dY."""
    X = synth.normal((M, K), 1.0, seed=seed)
    W = synth.normal((N, K), 0.02, seed=seed + 1)
    dY = synth.normal((M, N), 1e-3, seed=seed + 2)
    _, xt, sx, Xd = quant_operand(X, Fmt.E4M3, dev, want_q=False, want_qt=True)
    _, wt, sw, Wd = quant_operand(W, Fmt.E4M3, dev, want_q=False, want_qt=True)
    dyq, dyt, sdy, dYd = quant_operand(dY, Fmt.E5M2, dev, want_q=True, want_qt=True)
    # dX[M,K]: A = dY [M, N], B = W^T [K, N]
    dX = df.gemm_nt(dyq, Fmt.E5M2, wt, Fmt.E4M3, N, sdy, sw).cpu().numpy()
    idx = pick_rows(M, rows, seed)
    ref = orc.fc_backward_input(dYd[idx], Wd)
    err = orc.rel_err(dX[idx], ref)
    assert err <= TOL, f"dX M={M} K={K} N={N}: {err:.3e}"
    # dW[N,K]: A = dY^T [N, M], B = X^T [K, M]
    dW = df.gemm_nt(dyt, Fmt.E5M2, xt, Fmt.E4M3, M, sdy, sx).cpu().numpy()
    o_idx = pick_rows(N, wrows, seed + 9)
    i_idx = pick_rows(K, wcols, seed + 8)
    refw = orc.fc_backward_weights(np.ascontiguousarray(dYd[:, o_idx]), np.ascontiguousarray(Xd[:, i_idx]))
    errw = orc.rel_err(dW[np.ix_(o_idx, i_idx)], refw)
    assert errw <= TOL, f"dW M={M} K={K} N={N}: {errw:.3e}"
    # db from the fp32 upstream gradient (fc_backward_bias, :91-106)
    db = df.colsum(dev_f32(dY, dev)).cpu().numpy()
    assert orc.rel_err(db, orc.fc_backward_bias(dY)) <= TOL


@pytest.mark.parametrize("M,K,N", [(1, 4, 3), (1, 5, 2), (64, 768, 3072), (100, 40, 50), (129, 272, 257),
                                   (512, 1600, 64)])
def test_backward_shapes(dev, M, K, N):
    backward_case(dev, M, K, N, seed=M * 11 + K + N * 5)


def test_backward_entry_points_match_nt(dev):
    """df_fp8_gemm_bwd_dx / _bwd_dw are the NT kernel with the documented
    operand roles: their outputs equal the direct NT calls bit for bit."""
    M, K, N = 192, 160, 96
    X = synth.normal((M, K), 1.0, seed=1)
    W = synth.normal((N, K), 0.02, seed=2)
    dY = synth.normal((M, N), 1e-3, seed=3)
    _, xt, sx, _ = quant_operand(X, Fmt.E4M3, dev, want_q=False, want_qt=True)
    _, wt, sw, _ = quant_operand(W, Fmt.E4M3, dev, want_q=False, want_qt=True)
    dyq, dyt, sdy, _ = quant_operand(dY, Fmt.E5M2, dev, want_q=True, want_qt=True)
    dX_nt = df.gemm_nt(dyq, Fmt.E5M2, wt, Fmt.E4M3, N, sdy, sw)
    dW_nt = df.gemm_nt(dyt, Fmt.E5M2, xt, Fmt.E4M3, M, sdy, sx)
    dX = torch.empty((M, K), dtype=torch.float32, device=dev)
    dW = torch.empty((N, K), dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    ws = df.gemm_workspace(M, K, N, dev)
    df.call("df_fp8_gemm_bwd_dx", dyq.data_ptr(), dyq.stride(0), wt.data_ptr(), wt.stride(0), M, N, K,
            sdy.data_ptr(), sw.data_ptr(), int(df.DType.FLOAT32), dX.data_ptr(), K, ws.data_ptr(),
            ws.numel(), st)
    df.call("df_fp8_gemm_bwd_dw", dyt.data_ptr(), dyt.stride(0), xt.data_ptr(), xt.stride(0), M, N, K,
            sdy.data_ptr(), sx.data_ptr(), int(df.DType.FLOAT32), dW.data_ptr(), K, ws.data_ptr(),
            ws.numel(), st)
    assert torch.equal(dX, dX_nt)
    assert torch.equal(dW, dW_nt)


GPT2_SMALL = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
GPT2_XL = [(1600, 4800), (1600, 1600), (1600, 6400), (6400, 1600)]


@pytest.mark.parametrize("K,N", GPT2_SMALL)
def test_config3_forward_bf16(dev, K, N):
    """Config 3: M = 8192 tokens, bf16 activations and weights quantized to
    e4m3, bf16 output with fused bias; oracle on the band rows (every
    256-row band's first, last and two seeded rows)."""
    M = 8192
    seed = synth.SEED_BASE + 3 + K + N
    Xb = synth.f32_to_bf16_bits(synth.normal((M, K), 1.0, seed=seed))
    Wb = synth.f32_to_bf16_bits(synth.normal((N, K), 0.02, seed=seed + 1))
    bb = synth.f32_to_bf16_bits(synth.normal((N,), 0.1, seed=seed + 2))
    tob = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
    Xd, Wd, bd = tob(Xb), tob(Wb), tob(bb)
    _, sx = df.absmax_scale(Xd, Fmt.E4M3)
    _, sw = df.absmax_scale(Wd, Fmt.E4M3)
    xq, _ = df.quantize_2d(Xd, sx, Fmt.E4M3)
    wq, _ = df.quantize_2d(Wd, sw, Fmt.E4M3)
    # at these shapes the plan takes the persistent kernel's 256x128 tiles
    wsb = int(df.lib().df_fp8_gemm_workspace_bytes(M, N, K))
    assert df.gemm_plan(M, N, K, xq.stride(0), wq.stride(0), bd, wsb)[0] == df.GemmKernel.PERSISTENT_NARROW
    Y32 = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=bd)
    Y16 = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=bd, out_dtype=torch.bfloat16)
    check_bf16_image(Y32, Y16)
    s_x = orc.scale(orc.absmax(Xb), 0)
    s_w = orc.scale(orc.absmax(Wb), 0)
    assert sx.item() == np.float32(s_x) and sw.item() == np.float32(s_w)
    idx = band_rows(M, seed)
    cx = orc.quantize(Xb[idx], s_x, 0)
    assert np.array_equal(xq.cpu().numpy()[idx][:, :K], cx)
    cw = orc.quantize(Wb, s_w, 0)
    assert np.array_equal(wq.cpu().numpy()[:, :K], cw)
    ref = orc.fc_forward(orc.dequantize(cx, s_x, 0), orc.dequantize(cw, s_w, 0), orc.bf16_to_f32(bb))
    err = orc.rel_err(Y32.cpu().numpy()[idx], ref)
    assert err <= TOL, f"config3 {K}->{N}: {err:.3e}"


# (M, N, K) whose plan takes the persistent kernel's 256x128 tiles, with
# ragged edges: rows and columns ending inside a wave's 64x64 part, an
# odd-length bf16 bias, outputs whose row pitch is not 16-byte aligned.
NARROW_CASES = [(1000, 999, 640), (1000, 1000, 768), (300, 130, 1024), (2048, 640, 2048)]


@pytest.mark.parametrize("M,N,K", NARROW_CASES)
def test_narrow_tiles_match_oracle(dev, M, N, K):
    """256x128 tiles (fully_connected_layer.cu:14-35 restated by the
    oracle): fp32 output on every row against the oracle, bf16 output as
    its RNE image, bf16 bias."""
    seed = synth.SEED_BASE + 700 + M + N + K
    A = synth.normal((M, K), 1.0, seed=seed)
    B = synth.normal((N, K), 0.02, seed=seed + 1)
    bb = synth.f32_to_bf16_bits(synth.normal((N,), 0.1, seed=seed + 2))
    aq, _, sa, Ad = quant_operand(A, Fmt.E4M3, dev)
    bq, _, sb, Bd = quant_operand(B, Fmt.E4M3, dev)
    bd = torch.from_numpy(bb.view(np.int16)).to(dev).view(torch.bfloat16)
    for ws_bytes in (0, int(df.lib().df_fp8_gemm_workspace_bytes(M, N, K))):
        kind = df.gemm_plan(M, N, K, aq.stride(0), bq.stride(0), bd, ws_bytes)[0]
        assert kind == df.GemmKernel.PERSISTENT_NARROW, f"plan {kind!r} (workspace {ws_bytes})"
    Y = df.gemm_nt(aq, Fmt.E4M3, bq, Fmt.E4M3, K, sa, sb, bias=bd)
    Y16 = df.gemm_nt(aq, Fmt.E4M3, bq, Fmt.E4M3, K, sa, sb, bias=bd, out_dtype=torch.bfloat16)
    check_bf16_image(Y, Y16)
    ref = orc.fc_forward(Ad, Bd, orc.bf16_to_f32(bb))
    err = orc.rel_err(Y.cpu().numpy(), ref)
    assert err <= TOL, f"narrow M={M} N={N} K={K}: rel err {err:.3e}"


@pytest.mark.parametrize("K,N", GPT2_XL)
def test_config4_forward_backward(dev, K, N):
    """Config 4: M = 16384 tokens, forward e4m3 x e4m3, backward dY ~
    N(0, 1e-3) as e5m2; oracle on the band rows of Y and dX (every 256-row
    band) and on dW rows x columns hitting every 256 x 256 tile."""
    M = 16384
    backward_case(dev, M, K, N, seed=synth.SEED_BASE + 4 + K + N, rows="bands", wrows="bands", wcols="bands")
    forward_case(dev, M, K, N, seed=synth.SEED_BASE + 40 + K + N, rows="bands")


@pytest.mark.parametrize("M,N,K", [(1600, 1600, 16384), (384, 200, 8192), (4800, 1600, 16384)])
def test_split_k_matches_unsplit(dev, M, N, K):
    """Long reductions on small outputs take the split-K path when a
    workspace is given; without one the same product runs unsplit.  Both
    must meet the bar against the oracle (sampled rows) and agree closely."""
    A = synth.normal((M, K), 1e-3, seed=M + N)
    B = synth.normal((N, K), 1.0, seed=M + N + 1)
    aq, _, sa, Ad = quant_operand(A, Fmt.E5M2, dev)
    bq, _, sb, Bd = quant_operand(B, Fmt.E4M3, dev)
    with_ws = df.gemm_nt(aq, Fmt.E5M2, bq, Fmt.E4M3, K, sa, sb).cpu().numpy()
    no_ws = df.gemm_nt(aq, Fmt.E5M2, bq, Fmt.E4M3, K, sa, sb, split_k=False).cpu().numpy()
    idx = np.sort(np.random.default_rng(M).choice(M, 16, replace=False))
    ref = orc.fc_forward(Ad[idx], Bd, None)
    assert orc.rel_err(with_ws[idx], ref) <= TOL
    assert orc.rel_err(no_ws[idx], ref) <= TOL
    assert orc.rel_err(with_ws, no_ws) <= 1e-5
    if (M, N) in ((1600, 1600), (384, 200)):
        assert df.lib().df_fp8_gemm_workspace_bytes(M, N, K) > 0  # these two do take split-K


def grouped_case(dev, M, K, N, seed, rows=None, wrows=None, wcols=None, out16=False):
    """df_fp8_gemm_bwd against the two separate calls on the same codes:
    dX bit-identical, dW within 1e-5 (the launches may cut dW's K range into
    different slices) and both against the oracle at the 1e-4 bar."""
    X = synth.normal((M, K), 1.0, seed=seed)
    W = synth.normal((N, K), 0.02, seed=seed + 1)
    dY = synth.normal((M, N), 1e-3, seed=seed + 2)
    _, xt, sx, Xd = quant_operand(X, Fmt.E4M3, dev, want_q=False, want_qt=True)
    _, wt, sw, Wd = quant_operand(W, Fmt.E4M3, dev, want_q=False, want_qt=True)
    dyq, dyt, sdy, dYd = quant_operand(dY, Fmt.E5M2, dev, want_q=True, want_qt=True)
    dX, dW = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx)
    dX_sep = df.gemm_nt(dyq, Fmt.E5M2, wt, Fmt.E4M3, N, sdy, sw)
    dW_sep = df.gemm_nt(dyt, Fmt.E5M2, xt, Fmt.E4M3, M, sdy, sx)
    assert torch.equal(dX, dX_sep)
    assert orc.rel_err(dW.cpu().numpy(), dW_sep.cpu().numpy()) <= 1e-5
    idx = pick_rows(M, rows, seed)
    assert orc.rel_err(dX.cpu().numpy()[idx], orc.fc_backward_input(dYd[idx], Wd)) <= TOL
    o_idx = pick_rows(N, wrows, seed + 9)
    i_idx = pick_rows(K, wcols, seed + 8)
    refw = orc.fc_backward_weights(np.ascontiguousarray(dYd[:, o_idx]), np.ascontiguousarray(Xd[:, i_idx]))
    assert orc.rel_err(dW.cpu().numpy()[np.ix_(o_idx, i_idx)], refw) <= TOL
    if out16:
        dX16, dW16 = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, dx_dtype=torch.bfloat16,
                                 dw_dtype=torch.bfloat16)
        check_bf16_image(dX, dX16)
        check_bf16_image(dW, dW16)


@pytest.mark.parametrize("K,N", GPT2_XL)
def test_grouped_backward_config4(dev, K, N):
    """Config 4 (M = 16384): every XL Linear takes the grouped launch, fc and
    proj with dW unsplit, qkv and attn_proj as the plan decides."""
    M = 16384
    grouped, slices = df.gemm_bwd_plan(M, N, K)
    assert grouped and slices >= 1
    grouped_case(dev, M, K, N, seed=synth.SEED_BASE + 77 + K + N, rows="bands", wrows="bands", wcols="bands",
                 out16=(N == 1600))


@pytest.mark.parametrize("M,K,N", [(1, 4, 3), (64, 768, 3072), (129, 272, 257), (4096, 1600, 1600),
                                   (2048, 6400, 1600), (8192, 768, 2304)])
def test_grouped_backward_shapes(dev, M, K, N):
    """Ragged and small shapes: grouped where the plan finds it faster,
    the two separate calls otherwise; the results are the same either way."""
    grouped_case(dev, M, K, N, seed=M + 3 * K + 7 * N, out16=True)


def test_grouped_backward_without_workspace(dev):
    """No workspace: dW cannot be sliced, the plan falls back or groups
    unsplit, and the outputs still match."""
    M, K, N = 16384, 1600, 1600
    assert df.gemm_bwd_plan(M, N, K, 0)[1] in (0, 1)
    X = synth.normal((M, K), 1.0, seed=31)
    dY = synth.normal((M, N), 1e-3, seed=32)
    W = synth.normal((N, K), 0.02, seed=33)
    _, xt, sx, _ = quant_operand(X, Fmt.E4M3, dev, want_q=False, want_qt=True)
    _, wt, sw, _ = quant_operand(W, Fmt.E4M3, dev, want_q=False, want_qt=True)
    dyq, dyt, sdy, _ = quant_operand(dY, Fmt.E5M2, dev, want_q=True, want_qt=True)
    dX, dW = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx, workspace=False)
    dX2, dW2 = df.gemm_bwd(dyq, wt, dyt, xt, M, N, K, sdy, sw, sx)
    assert torch.equal(dX, dX2)
    assert orc.rel_err(dW.cpu().numpy(), dW2.cpu().numpy()) <= 1e-5


def bf16_operands(dev, M, K, N, seed):
    """bf16 X [M, K] ~ N(0, 1), W [N, K] ~ N(0, 0.02), bias [N] ~ N(0, 0.1)
    (host bf16 bits and device tensors), as the bench generates them."""
    Xb = synth.f32_to_bf16_bits(synth.normal((M, K), 1.0, seed=seed))
    Wb = synth.f32_to_bf16_bits(synth.normal((N, K), 0.02, seed=seed + 1))
    bb = synth.f32_to_bf16_bits(synth.normal((N,), 0.1, seed=seed + 2))
    tob = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
    return Xb, Wb, bb, tob(Xb), tob(Wb), tob(bb)


@pytest.mark.parametrize("K,N", GPT2_XL)
def test_config4_forward_bf16_bias_and_output(dev, K, N):
    """Config 4 forward as the bench runs it (df_fp8_gemm_fwd with bf16
    bias and bf16 output, the persistent kernel's multi-tile walk over 16384
    rows): the bf16 Y is the RNE image of the fp32 Y of the same call with
    fp32 output, which is within 1e-4 of the oracle on every 256-row band."""
    M = 16384
    seed = synth.SEED_BASE + 44 + K + N
    Xb, Wb, bb, Xd, Wd, bd = bf16_operands(dev, M, K, N, seed)
    _, sx = df.absmax_scale(Xd, Fmt.E4M3)
    _, sw = df.absmax_scale(Wd, Fmt.E4M3)
    xq, _ = df.quantize_2d(Xd, sx, Fmt.E4M3)
    wq, _ = df.quantize_2d(Wd, sw, Fmt.E4M3)
    assert df.gemm_plan(M, N, K, xq.stride(0), wq.stride(0), bd, 1 << 30)[0] == df.GemmKernel.PERSISTENT
    Y16 = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ws = df.gemm_workspace(M, N, K, dev)
    df.call("df_fp8_gemm_fwd", xq.data_ptr(), xq.stride(0), wq.data_ptr(), wq.stride(0), M, N, K, sx.data_ptr(),
            sw.data_ptr(), int(df.DType.BFLOAT16), bd.data_ptr(), int(df.DType.BFLOAT16), Y16.data_ptr(), N,
            ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    Y32 = df.gemm_nt(xq, Fmt.E4M3, wq, Fmt.E4M3, K, sx, sw, bias=bd)
    check_bf16_image(Y32, Y16)
    s_x = orc.scale(orc.absmax(Xb), 0)
    s_w = orc.scale(orc.absmax(Wb), 0)
    assert sx.item() == np.float32(s_x) and sw.item() == np.float32(s_w)
    idx = band_rows(M, seed)
    cx = orc.quantize(Xb[idx], s_x, 0)
    assert np.array_equal(xq.cpu().numpy()[idx][:, :K], cx)
    cw = orc.quantize(Wb, s_w, 0)
    assert np.array_equal(wq.cpu().numpy()[:, :K], cw)
    ref = orc.fc_forward(orc.dequantize(cx, s_x, 0), orc.dequantize(cw, s_w, 0), orc.bf16_to_f32(bb))
    err = orc.rel_err(Y32.cpu().numpy()[idx], ref)
    assert err <= TOL, f"config4 bf16 {K}->{N}: {err:.3e}"


# Calls the persistent kernel does not take (a bias that is not 4-byte
# aligned; lda of 2^23 or more; an operand of 2 GiB or more) run the tiled
# kernels: LDS-DMA operand loads while M*lda and N*ldb stay below 2^31,
# register-staged loads beyond.  Each case states the kernel and split the
# plan must pick, then checks the product against the oracle.
#   (name, M, N, K, lda, bias_offset_elems, workspace, kernel, split>1)
FALLBACK_CASES = [
    ("dma256_bias_offset", 4096, 4096, 512, None, 1, False, "TILED_DMA_256", False),
    ("dma128_bias_offset", 384, 384, 640, None, 1, False, "TILED_DMA_128", False),
    ("dma128_splitk_bias_offset", 256, 256, 8192, None, 1, True, "TILED_DMA_128", True),
    ("dma_lda_2p23", 128, 320, 512, 1 << 23, 0, False, "TILED_DMA_128", False),
    ("reg256_2gib_operand", 32768, 384, 256, 1 << 16, 1, False, "TILED_REG_256", False),
    ("reg128_2gib_operand", 256, 256, 512, 1 << 23, 0, False, "TILED_REG_128", False),
    ("reg128_splitk_2gib_operand", 256, 320, 8192, 1 << 23, 1, True, "TILED_REG_128", True),
]


@pytest.mark.parametrize("name,M,N,K,lda,boff,use_ws,kernel,split", FALLBACK_CASES,
                         ids=[c[0] for c in FALLBACK_CASES])
def test_fallback_kernels_match_oracle(dev, name, M, N, K, lda, boff, use_ws, kernel, split):
    seed = synth.SEED_BASE + 900 + M + N + K
    A = synth.normal((M, K), 1.0, seed=seed)
    B = synth.normal((N, K), 0.02, seed=seed + 1)
    bias = synth.normal((N,), 0.1, seed=seed + 2)
    bb = synth.f32_to_bf16_bits(bias)
    aq, _, sa, Ad = quant_operand(A, Fmt.E4M3, dev)
    bq, _, sb, Bd = quant_operand(B, Fmt.E4M3, dev)
    big = None
    if lda is not None:  # the same codes at a wide leading dimension
        big = torch.zeros((M, lda), dtype=torch.uint8, device=dev)
        big[:, :aq.shape[1]].copy_(aq)
        aq = big[:, :aq.shape[1]]
        assert aq.stride(0) == lda
    # bf16 bias, `boff` elements into its buffer (2 bytes: not 4-byte aligned)
    bstore = torch.zeros(N + 2, dtype=torch.int16, device=dev)
    bstore[boff:boff + N].copy_(torch.from_numpy(bb.view(np.int16)))
    bd = bstore[boff:boff + N].view(torch.bfloat16)
    ws_bytes = int(df.lib().df_fp8_gemm_workspace_bytes(M, N, K)) if use_ws else 0
    got_kernel, got_split = df.gemm_plan(M, N, K, aq.stride(0), bq.stride(0), bd, ws_bytes)
    assert got_kernel == df.GemmKernel[kernel], f"{name}: plan {got_kernel!r}"
    assert (got_split > 1) == split, f"{name}: split {got_split}"
    Y = df.gemm_nt(aq, Fmt.E4M3, bq, Fmt.E4M3, K, sa, sb, bias=bd, split_k=use_ws)
    Y16 = df.gemm_nt(aq, Fmt.E4M3, bq, Fmt.E4M3, K, sa, sb, bias=bd, out_dtype=torch.bfloat16, split_k=use_ws)
    check_bf16_image(Y, Y16)
    idx = band_rows(M, seed) if M > 1024 else np.arange(M)
    ref = orc.fc_forward(Ad[idx], Bd, orc.bf16_to_f32(bb))
    err = orc.rel_err(Y.cpu().numpy()[idx], ref)
    assert err <= TOL, f"{name}: rel err {err:.3e}"
    del big, aq, Y, Y16
    torch.cuda.empty_cache()
