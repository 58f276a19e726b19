"""GPU parity of the 2-D quantize (df_quantize_2d / _colsum / _delayed) on
two-byte inputs at sizes of hundreds to thousands of 128x128 tiles, and on
every bf16 and random fp32 bit pattern.  It makes the fp8 operands of the
Linear's GEMMs (the inputs of the reference's kernels,
dnn/layers/fully_connected_layer.cu:14-89) from activations and gradients.

The conversion takes a short form for groups of values a wave-wide ballot
finds free of NaN and the full form otherwise; both must give the oracle's
codes.  Bars:
  - q and qt bit-exact against the oracle's codes of the same values, zero
    padded, for bf16 and binary16 inputs, full and ragged tile grids, both
    division forms (scales inside and outside [2^-40, 2^40]) and planted
    NaN / inf / -0 / huge values;
  - the same values laid out with a row stride that is not a multiple of 8
    elements take the element-wise loads: codes, column sums and the
    delayed-scaling history are bit-identical between the two layouts;
  - column sums within 1e-4 of the oracle's db; the delayed-scaling absmax
    equals the oracle's.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

# (rows, cols): 288 full tiles; a ragged grid (16 x 19 tiles with the padded
# extents); the config-4 activation shape (1664 tiles)
SHAPES = [(2048, 2304), (2037, 2305), (16384, 1600)]


def make(dev, rows, cols, kind, seed, std=1.0, specials=True):
    """(device tensor, host bits, host fp32 values) of one input."""
    x = synth.normal((rows, cols), std, seed=seed)
    if specials:
        rng = np.random.default_rng(seed)
        idx = rng.integers(0, rows * cols, 64)
        flat = x.reshape(-1)
        flat[idx[:16]] = np.nan
        flat[idx[16:24]] = np.inf
        flat[idx[24:32]] = -np.inf
        flat[idx[32:40]] = -0.0
        flat[idx[40:48]] = 6e4 if kind == "f16" else 3e38
        flat[idx[48:56]] = -6e4 if kind == "f16" else -3e38
    if kind == "bf16":
        bits = synth.f32_to_bf16_bits(x)
        vals = orc.bf16_to_f32(bits).reshape(rows, cols)
        dtype = torch.bfloat16
    else:
        bits = orc.convert(np.ascontiguousarray(x, np.float32), 0, 1).reshape(rows, cols)
        vals = orc.convert(bits, 1, 0).reshape(rows, cols)
        dtype = torch.float16
    xd = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(dtype)
    return xd, bits, vals


def strided(xd, pad):
    """The same values with row stride cols + pad (a view into a wider buffer)."""
    rows, cols = xd.shape
    wide = torch.zeros((rows, cols + pad), dtype=xd.dtype, device=xd.device)
    wide[:, :cols] = xd
    return wide[:, :cols]


def check_codes(q, qt, flat, rows, cols, what):
    qh, qth = q.cpu().numpy(), qt.cpu().numpy()
    assert np.array_equal(qh[:, :cols], flat), f"{what}: q"
    assert not qh[:, cols:].any(), f"{what}: q padding"
    assert np.array_equal(qth[:, :rows], np.ascontiguousarray(flat.T)), f"{what}: qt"
    assert not qth[:, rows:].any(), f"{what}: qt padding"


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_codes_against_oracle(dev, kind, fmt):
    for i, (rows, cols) in enumerate(SHAPES):
        print(f"stream codes {kind} fmt={int(fmt)} {rows}x{cols}", flush=True)
        xd, _, vals = make(dev, rows, cols, kind, seed=synth.SEED_BASE + 900 + i)
        s = float(np.float32(orc.scale(orc.absmax(vals), int(fmt))))
        q, qt = df.quantize_2d(xd, torch.tensor([s], device=dev), fmt, want_q=True, want_qt=True)
        check_codes(q, qt, orc.quantize(vals, s, int(fmt)), rows, cols, f"{kind} {rows}x{cols}")


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("scale", [2.0 ** -45, 2.0 ** 45, 3.0e-3])
def test_division_forms(dev, kind, scale):
    """Scales outside [2^-40, 2^40] take the IEEE division, others the
    Markstein form; both bit-exact."""
    rows, cols = 2048, 2304
    xd, _, vals = make(dev, rows, cols, kind, seed=synth.SEED_BASE + 910, std=1e-3)
    for fmt in (Fmt.E4M3, Fmt.E5M2):
        q, qt = df.quantize_2d(xd, torch.tensor([scale], dtype=torch.float32, device=dev), fmt, want_q=True,
                               want_qt=True)
        check_codes(q, qt, orc.quantize(vals, float(np.float32(scale)), int(fmt)), rows, cols, f"s={scale}")


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_vector_and_element_loads_agree(dev, kind):
    """Contiguous (16-byte loads) against a stride of cols + 3 (element-wise
    loads): codes and column sums bit-identical; sums within 1e-4 of the
    oracle."""
    for i, (rows, cols) in enumerate(SHAPES):
        print(f"stream vs tile {kind} {rows}x{cols}", flush=True)
        xd, _, vals = make(dev, rows, cols, kind, seed=synth.SEED_BASE + 920 + i, std=1e-2, specials=False)
        s = torch.tensor([float(np.float32(orc.scale(orc.absmax(vals), int(Fmt.E5M2))))], device=dev)
        qa, qta, csa = df.quantize_2d(xd, s, Fmt.E5M2, want_q=True, want_qt=True, colsum=True)
        qb, qtb, csb = df.quantize_2d(strided(xd, 3), s, Fmt.E5M2, want_q=True, want_qt=True, colsum=True)
        assert torch.equal(qa, qb) and torch.equal(qta, qtb), f"{rows}x{cols}: codes differ"
        assert torch.equal(csa.view(torch.int32), csb.view(torch.int32)), f"{rows}x{cols}: column sums differ"
        assert orc.rel_err(csa.cpu().numpy(), orc.fc_backward_bias(vals)) <= 1e-4
        # row copy only and transposed copy only
        q1, _ = df.quantize_2d(xd, s, Fmt.E5M2, want_q=True, want_qt=False)
        _, qt1 = df.quantize_2d(xd, s, Fmt.E5M2, want_q=False, want_qt=True)
        assert torch.equal(q1, qa) and torch.equal(qt1, qta), f"{rows}x{cols}: single-output passes"


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_delayed_scaling(dev, kind, fmt):
    """Delayed scaling through both layouts: codes, column sums, history and
    next scale bit-identical, and the history holds the oracle's absmax."""
    length = 4
    a = df.DelayedScale(fmt, length, dev)
    b = df.DelayedScale(fmt, length, dev)
    hist = np.zeros(length, np.float32)
    scale = np.float32(1.0)
    for i, (rows, cols) in enumerate(SHAPES):
        print(f"stream delayed {kind} fmt={int(fmt)} {rows}x{cols}", flush=True)
        xd, _, vals = make(dev, rows, cols, kind, seed=synth.SEED_BASE + 930 + i, std=4.0 ** i)
        colsum = i % 2 == 0
        oa = a.quantize_2d(xd, want_q=True, want_qt=True, colsum=colsum)
        ob = b.quantize_2d(strided(xd, 3), want_q=True, want_qt=True, colsum=colsum)
        check_codes(oa[0], oa[1], orc.quantize(vals, float(scale), int(fmt)), rows, cols, f"pass {i}")
        assert torch.equal(oa[0], ob[0]) and torch.equal(oa[1], ob[1]), f"pass {i}: codes differ"
        if colsum:
            assert torch.equal(oa[2].view(torch.int32), ob[2].view(torch.int32)), f"pass {i}: column sums"
        scale = np.float32(orc.history_push(hist, orc.absmax(vals), int(fmt)))
        torch.cuda.synchronize()
        assert np.array_equal(a.history.cpu().numpy().view(np.uint32), hist.view(np.uint32)), f"pass {i}: history"
        assert torch.equal(a.history.view(torch.int32), b.history.view(torch.int32)), f"pass {i}: histories differ"
        assert a.scale.cpu().numpy().view(np.uint32)[0] == np.float32(scale).view(np.uint32), f"pass {i}: scale"


@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
@pytest.mark.parametrize("nan", ["kept", "zeroed"])
def test_every_bf16_pattern(dev, fmt, nan):
    """All 2^16 bf16 patterns as a [256, 256] matrix: with the NaN patterns
    in place (their waves take the full form) and replaced by zeros (every
    other pattern through the short form)."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    if nan == "zeroed":
        bits = np.where((bits & 0x7FFF) > 0x7F80, np.uint16(0), bits)
    xd = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    for s in (1.0, 0.0123, 1.0 / 57344.0, 5.0e3, 2.0 ** -45, 2.0 ** 41):
        s32 = float(np.float32(s))
        q, qt = df.quantize_2d(xd, torch.tensor([s32], device=dev), fmt, want_q=True, want_qt=True)
        check_codes(q, qt, orc.quantize(bits, s32, int(fmt)), 256, 256, f"s={s32}")


@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
@pytest.mark.parametrize("nan", ["kept", "as_inf"])
def test_random_f32_patterns(dev, fmt, nan):
    """Uniform random binary32 bit patterns (every exponent, subnormals,
    infinities), NaN patterns kept or turned into infinities, as a
    [2048, 2304] matrix through the 2-D pass at several scales."""
    rng = np.random.default_rng(synth.SEED_BASE + 940)
    u = rng.integers(0, 1 << 32, size=(2048, 2304), dtype=np.uint64).astype(np.uint32)
    if nan == "as_inf":
        u = np.where((u & 0x7FFFFFFF) > 0x7F800000, u & 0xFF800000, u)
    x = u.view(np.float32)
    xd = torch.from_numpy(x).to(dev)
    for s in (1.0, 3.0e-3, 2.0 ** -40, 2.0 ** 40, 0.7 * 2.0 ** 40, 2.0 ** -45):
        s32 = float(np.float32(s))
        q, qt = df.quantize_2d(xd, torch.tensor([s32], device=dev), fmt, want_q=True, want_qt=True)
        check_codes(q, qt, orc.quantize(x, s32, int(fmt)), 2048, 2304, f"s={s32}")


@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_outputs_off_line_boundaries(dev, fmt):
    """Outputs that do not start on (or whose rows do not stride by) 128
    bytes take plain stores instead of non-temporal ones: the same codes and
    values as aligned outputs, and the oracle's."""
    st = torch.cuda.current_stream().cuda_stream
    n = (1 << 20) + 40
    x = synth.normal((n,), seed=synth.SEED_BASE + 950)
    s = float(np.float32(orc.scale(orc.absmax(x), int(fmt))))
    sd = torch.tensor([s], device=dev)
    name = "e4m3" if fmt == Fmt.E4M3 else "e5m2"
    exp = orc.quantize(x, s, int(fmt))
    xd = torch.from_numpy(x).to(dev)
    xb_bits = synth.f32_to_bf16_bits(x)
    xb = torch.from_numpy(xb_bits.view(np.int16)).to(dev).view(torch.bfloat16)
    expb = orc.quantize(xb_bits, s, int(fmt))
    for off in (8, 72):  # bytes past a 128-byte boundary (q must be 8-byte aligned for bf16)
        buf = torch.zeros(n + 256, dtype=torch.uint8, device=dev)
        df.call(f"df_quantize_f32_{name}", xd.data_ptr(), n, sd.data_ptr(), buf.data_ptr() + off, st)
        assert np.array_equal(buf[off:off + n].cpu().numpy(), exp), f"f32 codes at +{off}"
        df.call(f"df_quantize_bf16_{name}", xb.data_ptr(), n, sd.data_ptr(), buf.data_ptr() + off, st)
        assert np.array_equal(buf[off:off + n].cpu().numpy(), expb), f"bf16 codes at +{off}"
    q = torch.from_numpy(exp).to(dev)
    qb = torch.zeros(n + 256, dtype=torch.uint8, device=dev)
    qb[8:8 + n] = q
    for off in (16, 48):  # outputs must be 16-byte aligned
        ref32 = df.dequantize(q, sd, fmt, torch.float32)
        ref16 = df.dequantize(q, sd, fmt, torch.bfloat16)
        o32 = torch.zeros(n + 64, dtype=torch.float32, device=dev)
        df.call(f"df_dequantize_{name}_f32", qb.data_ptr() + 8, n, sd.data_ptr(), o32.data_ptr() + off, st)
        assert torch.equal(o32[off // 4:off // 4 + n].view(torch.int32), ref32.view(torch.int32)), f"f32 at +{off}"
        o16 = torch.zeros(n + 64, dtype=torch.bfloat16, device=dev)
        df.call(f"df_dequantize_{name}_bf16", qb.data_ptr() + 8, n, sd.data_ptr(), o16.data_ptr() + off, st)
        assert torch.equal(o16[off // 2:off // 2 + n].view(torch.int16), ref16.view(torch.int16)), f"bf16 at +{off}"
    # 2-D outputs with row strides that are not multiples of 128 (delayed
    # scaling, whose codes are otherwise stored non-temporal), against the
    # aligned layout
    rows, cols = 2048, 2304
    xd2, _, vals = make(dev, rows, cols, "bf16", seed=synth.SEED_BASE + 951)
    a = df.DelayedScale(fmt, 2, dev)
    b = df.DelayedScale(fmt, 2, dev)
    qa, qta = a.quantize_2d(xd2, want_q=True, want_qt=True)
    ldq, ldqt = cols + 16, rows + 48
    qo = torch.zeros((rows, ldq), dtype=torch.uint8, device=dev)
    qto = torch.zeros((cols, ldqt), dtype=torch.uint8, device=dev)
    nbytes = df.lib().df_quantize_2d_delayed_workspace_bytes(rows, cols, ldq, ldqt, 0)
    ws = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=dev)
    df.call("df_quantize_2d_delayed", 4, xd2.data_ptr(), rows, cols, cols, int(fmt), b.scale.data_ptr(),
            b.scale.data_ptr(), b.history.data_ptr(), 2, qo.data_ptr(), ldq, qto.data_ptr(), ldqt, None,
            ws.data_ptr(), ws.numel(), st)
    assert torch.equal(qo[:, :cols], qa[:, :cols]) and torch.equal(qto[:, :rows], qta[:, :rows])
    assert torch.equal(a.history.view(torch.int32), b.history.view(torch.int32))
