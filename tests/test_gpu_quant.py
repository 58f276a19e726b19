"""GPU parity of absmax / scale / quantize / dequantize against the CPU oracle.

Bar: bit-exact codes, absmax, scales and dequantized values (integer/byte
work).  Everything is called through the C ABI (deepfuse_amd binds
libdeepfuse_amd.so); the oracle is oracle/libdf_oracle.so.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

FMTS = [Fmt.E4M3, Fmt.E5M2]


def to_dev_f32(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)


def to_dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).to(dev).view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def assert_bits_equal(got, exp, what):
    got = np.asarray(got).reshape(-1)
    exp = np.asarray(exp).reshape(-1)
    assert got.shape == exp.shape, what
    if got.dtype == np.float32:
        got, exp = got.view(np.uint32), exp.view(np.uint32)
    bad = np.nonzero(got != exp)[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: got {got[bad[0]]:#x} exp {exp[bad[0]]:#x}"


def scale_tensor(s, dev):
    return torch.tensor([s], dtype=torch.float32, device=dev)


@pytest.mark.parametrize("fmt", FMTS)
def test_reference_kat_codes(dev, fmt):
    """fully_connected_layer_test.cu:266-284 weights/inputs quantized per tensor."""
    W = np.array([1, 2, 3, 4], np.float32)
    x = np.array([1, 2], np.float32)
    for arr in (W, x):
        t = to_dev_f32(arr, dev)
        am, sc = df.absmax_scale(t, fmt)
        q = df.quantize(t, sc, fmt)
        torch.cuda.synchronize()
        s_exp = orc.scale(orc.absmax(arr), int(fmt))
        assert_bits_equal(sc.cpu().numpy(), np.float32([s_exp]), "scale")
        assert_bits_equal(q.cpu().numpy(), orc.quantize(arr, s_exp, int(fmt)), "codes")
    if fmt == Fmt.E4M3:
        t = to_dev_f32(W, dev)
        _, sc = df.absmax_scale(t, fmt)
        assert df.quantize(t, sc, fmt).cpu().numpy().tolist() == [0x6E, 0x76, 0x7A, 0x7E]


@pytest.mark.parametrize("fmt", FMTS)
def test_exhaustive_f32_patterns_unit_scale(dev, fmt):
    """Every binary32 bit pattern at s = 1 (x / 1 == x), in 2^28 chunks."""
    one = scale_tensor(1.0, dev)
    chunk = 1 << 28
    for c in range(16):
        first = c * chunk
        x = torch.arange(first, first + chunk, dtype=torch.int64, device=dev).to(torch.int32)
        q = df.quantize(x.view(torch.float32), one, fmt)
        exp = orc.encode_bits_range(first, chunk, int(fmt))
        assert_bits_equal(q.cpu().numpy(), exp, f"chunk {c}")
        del x, q


@pytest.mark.parametrize("fmt,s", [(Fmt.E4M3, 4.0 / 448.0), (Fmt.E5M2, 3.0 / 57344.0)])
def test_exhaustive_f32_patterns_nonunit_scale(dev, fmt, s):
    """Every binary32 bit pattern divided by a non-trivial scale: pins the
    kernel's correctly rounded x / s against the oracle's IEEE division."""
    s32 = float(np.float32(s))
    sd = scale_tensor(s32, dev)
    chunk = 1 << 28
    for c in range(16):
        first = c * chunk
        x = torch.arange(first, first + chunk, dtype=torch.int64, device=dev).to(torch.int32)
        q = df.quantize(x.view(torch.float32), sd, fmt).cpu().numpy()
        del x
        bits = np.arange(first, first + chunk, dtype=np.uint64).astype(np.uint32)
        assert_bits_equal(q, orc.quantize(bits.view(np.float32), s32, int(fmt)), f"chunk {c} s={s32}")


@pytest.mark.parametrize("fmt", FMTS)
def test_random_patterns_nonunit_scale(dev, fmt):
    """Random binary32 patterns (all classes) under several scales: exercises
    the IEEE division on both sides."""
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 1 << 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    xd = to_dev_f32(x, dev)
    for s in (448.0 / 3.7, 1.0 / 448.0, 3.0e-5, 2.0 ** -140, 1.7e30, 0.999999940395,
              2.0 ** -60, 2.0 ** -61, 2.0 ** 60, 2.0 ** 61, 1.0e-25, 3.0e25,
              2.0 ** -40, 2.0 ** -41, 2.0 ** 40, 2.0 ** 41, 0.7 * 2.0 ** -40, 1.3 * 2.0 ** 40):
        s32 = float(np.float32(s))
        q = df.quantize(xd, scale_tensor(s32, dev), fmt)
        assert_bits_equal(q.cpu().numpy(), orc.quantize(x, s32, int(fmt)), f"s={s32}")


@pytest.mark.parametrize("fmt", FMTS)
def test_all_bf16_patterns(dev, fmt):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    xd = to_dev_bf16(bits, dev)
    for s in (1.0, 0.0123, 1.0 / 57344.0, 5.0e3):
        s32 = float(np.float32(s))
        q = df.quantize(xd, scale_tensor(s32, dev), fmt)
        assert_bits_equal(q.cpu().numpy(), orc.quantize(bits, s32, int(fmt)), f"bf16 s={s32}")


@pytest.mark.parametrize("fmt", FMTS)
def test_dequantize_all_codes(dev, fmt):
    codes = np.arange(256, dtype=np.uint8)
    qd = torch.from_numpy(codes).to(dev)
    for s in (1.0, 0.00892857, 1.0e-30, 3.0e30, float(np.float32(2.0 ** -149) * 1)):
        s32 = float(np.float32(s))
        out = df.dequantize(qd, scale_tensor(s32, dev), fmt, torch.float32)
        assert_bits_equal(out.cpu().numpy(), orc.dequantize(codes, s32, int(fmt), "f32"), f"f32 s={s32}")
        outb = df.dequantize(qd, scale_tensor(s32, dev), fmt, torch.bfloat16)
        assert_bits_equal(host_u16(outb), orc.dequantize(codes, s32, int(fmt), "bf16"), f"bf16 s={s32}")


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 7, 8, 9, 17, 255, 1000003])
def test_ragged_sizes(dev, n):
    x = synth.conversion_input(max(n, 1), seed=100 + n)[:n]
    xd = to_dev_f32(x, dev)
    bits = synth.f32_to_bf16_bits(x)
    xb = to_dev_bf16(bits, dev)
    for fmt in FMTS:
        am, sc = df.absmax_scale(xd, fmt)
        s_exp = orc.scale(orc.absmax(x), int(fmt))
        assert_bits_equal(sc.cpu().numpy(), np.float32([s_exp]), "scale f32")
        q = df.quantize(xd, sc, fmt)
        qe = orc.quantize(x, s_exp, int(fmt))
        assert_bits_equal(q.cpu().numpy(), qe, "codes f32")
        out = df.dequantize(q, sc, fmt, torch.float32)
        assert_bits_equal(out.cpu().numpy(), orc.dequantize(qe, s_exp, int(fmt), "f32"), "deq f32")
        amb, scb = df.absmax_scale(xb, fmt)
        sb_exp = orc.scale(orc.absmax(bits), int(fmt))
        assert_bits_equal(scb.cpu().numpy(), np.float32([sb_exp]), "scale bf16")
        qb = df.quantize(xb, scb, fmt)
        qbe = orc.quantize(bits, sb_exp, int(fmt))
        assert_bits_equal(qb.cpu().numpy(), qbe, "codes bf16")
        outb = df.dequantize(qb, scb, fmt, torch.bfloat16)
        assert_bits_equal(host_u16(outb), orc.dequantize(qbe, sb_exp, int(fmt), "bf16"), "deq bf16")


def test_degenerate_scales(dev):
    """absmax 0, all non-finite, and subnormal-only tensors (contract D2)."""
    cases = [np.zeros(64, np.float32),
             np.array([np.inf, -np.inf, np.nan] * 8, np.float32),
             np.full(40, 1e-44, np.float32),
             np.full(40, -2.0 ** -126, np.float32)]
    for x in cases:
        xd = to_dev_f32(x, dev)
        for fmt in FMTS:
            am, sc = df.absmax_scale(xd, fmt)
            assert_bits_equal(am.cpu().numpy(), np.float32([orc.absmax(x)]), "absmax")
            s_exp = orc.scale(orc.absmax(x), int(fmt))
            assert_bits_equal(sc.cpu().numpy(), np.float32([s_exp]), "scale")
            assert_bits_equal(df.quantize(xd, sc, fmt).cpu().numpy(), orc.quantize(x, s_exp, int(fmt)), "codes")


@pytest.mark.parametrize("src", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", FMTS)
def test_config2_full_size(dev, src, fmt):
    """Config 2 at its full size, n = 268,435,456, outliers and specials:
    absmax, scale, codes and the dequantized round trip, all bit-exact."""
    n = 268_435_456
    x = synth.conversion_input(n)
    if src == "f32":
        host, xd = x, to_dev_f32(x, dev)
        deq_kind, out_dtype = "f32", torch.float32
    else:
        host = synth.f32_to_bf16_bits(x)
        xd = to_dev_bf16(host, dev)
        deq_kind, out_dtype = "bf16", torch.bfloat16
    del x
    am, sc = df.absmax_scale(xd, fmt)
    am_exp = orc.absmax(host)
    s_exp = orc.scale(am_exp, int(fmt))
    assert_bits_equal(am.cpu().numpy(), np.float32([am_exp]), "absmax")
    assert_bits_equal(sc.cpu().numpy(), np.float32([s_exp]), "scale")
    q = df.quantize(xd, sc, fmt)
    del xd
    qe = orc.quantize(host, s_exp, int(fmt))
    qh = q.cpu().numpy()
    assert_bits_equal(qh, qe, "codes")
    out = df.dequantize(q, sc, fmt, out_dtype)
    got = out.cpu().numpy() if src == "f32" else host_u16(out)
    del out, q
    exp = np.empty_like(got)
    step = 1 << 25
    for lo in range(0, n, step):
        exp[lo:lo + step] = orc.dequantize(qe[lo:lo + step], s_exp, int(fmt), deq_kind)
    assert_bits_equal(got, exp, "round trip")


@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_2d_colsum(dev, fmt):
    """Fused column sums of the 2-D pass (the dY pass of the backward, db)."""
    for rows, cols in [(1, 3), (100, 50), (129, 257), (1000, 1600)]:
        x = synth.normal((rows, cols), 1e-3, seed=rows + cols)
        xd = to_dev_f32(x, dev)
        s = float(np.float32(orc.scale(orc.absmax(x), int(fmt))))
        q, qt, cs = df.quantize_2d(xd, scale_tensor(s, dev), fmt, want_q=True, want_qt=True, colsum=True)
        flat = orc.quantize(x, s, int(fmt))
        assert_bits_equal(q.cpu().numpy()[:, :cols], flat, "q")
        assert_bits_equal(qt.cpu().numpy()[:, :rows], np.ascontiguousarray(flat.T), "qt")
        assert orc.rel_err(cs.cpu().numpy(), orc.fc_backward_bias(x)) <= 1e-4
        xb = synth.f32_to_bf16_bits(x)
        _, _, csb = df.quantize_2d(to_dev_bf16(xb, dev).view(rows, cols), scale_tensor(s, dev), fmt,
                                   want_q=False, want_qt=False, colsum=True)
        assert orc.rel_err(csb.cpu().numpy(), orc.fc_backward_bias(orc.bf16_to_f32(xb).reshape(rows, cols))) <= 1e-4


@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_2d_layouts(dev, fmt):
    """q and the transposed copy qt carry the flat codes, zero padded."""
    for rows, cols in [(1, 4), (3, 5), (64, 768), (100, 50), (129, 257), (16, 16)]:
        x = synth.normal((rows, cols), seed=rows * 1000 + cols)
        xd = to_dev_f32(x, dev)
        s = float(np.float32(orc.scale(orc.absmax(x), int(fmt))))
        q, qt = df.quantize_2d(xd, scale_tensor(s, dev), fmt, want_q=True, want_qt=True)
        flat = orc.quantize(x, s, int(fmt))
        qh, qth = q.cpu().numpy(), qt.cpu().numpy()
        assert_bits_equal(qh[:, :cols], flat, f"q {rows}x{cols}")
        assert not qh[:, cols:].any()
        assert_bits_equal(qth[:, :rows], np.ascontiguousarray(flat.T), f"qt {rows}x{cols}")
        assert not qth[:, rows:].any()
        xb = synth.f32_to_bf16_bits(x)
        qb, qtb = df.quantize_2d(to_dev_bf16(xb, dev).view(rows, cols), scale_tensor(s, dev), fmt,
                                 want_q=True, want_qt=True)
        flatb = orc.quantize(xb, s, int(fmt))
        assert_bits_equal(qb.cpu().numpy()[:, :cols], flatb, "q bf16")
        assert_bits_equal(qtb.cpu().numpy()[:, :rows], np.ascontiguousarray(flatb.T), "qt bf16")


BATCH_SHAPES = [(4800, 1600), (1600, 1600), (0, 5), (1, 1), (129, 257), (6400, 1600), (3, 40), (1600, 6400)]


@pytest.mark.parametrize("with_empty", [True, False], ids=["with_empty", "no_empty"])
@pytest.mark.parametrize("given_absmax", [False, True], ids=["own_absmax", "given_absmax"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_quantize_2d_batch_matches_single_calls(dev, dtype, fmt, given_absmax, with_empty):
    """df_quantize_2d_batch gives every tensor the absmax, scale, row codes
    and transposed codes that df_absmax_scale + df_quantize_2d give it alone
    (ragged shapes, a 1x1, the GPT-2 XL weights).  With the absmax given
    (df_quantize_2d_batch_absmax) the tile pass runs its non-temporal
    instantiation, for both dtypes and formats.  Without an empty tensor every
    tensor's tile blocks form its scale themselves (the folded form); an
    empty tensor, which has no tile block, keeps the separate fold launch."""
    rng = np.random.default_rng(7)
    ts = []
    for i, (r, c) in enumerate(BATCH_SHAPES):
        if r * c == 0 and not with_empty:
            continue
        x = (rng.standard_normal((r, c)) * (0.02 * (i + 1))).astype(np.float32)
        if x.size:
            x.reshape(-1)[rng.integers(0, x.size)] = 50.0 * (i + 1)  # an outlier sets each tensor's scale
        t = to_dev_f32(x, dev)
        ts.append(t if dtype == "f32" else t.to(torch.bfloat16))
    given = None
    if given_absmax:
        given = torch.stack([df.absmax_scale(t, fmt)[0][0] if t.numel() else torch.zeros((), device=dev)
                             for t in ts]).contiguous()
    am, sc, qs, qts = df.quantize_2d_batch(ts, fmt, absmax=given)
    for i, t in enumerate(ts):
        a1, s1 = df.absmax_scale(t, fmt)
        q1, qt1 = df.quantize_2d(t, s1, fmt, want_q=True, want_qt=True)
        assert am[i].item() == a1.item() and sc[i].item() == s1.item(), f"tensor {i} {tuple(t.shape)}"
        assert torch.equal(qs[i], q1), f"q of tensor {i} {tuple(t.shape)}"
        assert torch.equal(qts[i], qt1), f"qt of tensor {i} {tuple(t.shape)}"


def test_quantize_2d_batch_beyond_cache(dev):
    """A batch whose inputs exceed the 256 MB Infinity Cache (4 x 8192 x
    2304 fp32 = 302 MB) takes the non-temporal tile pass after its own
    absmax pass; every tensor still gets the single calls' scale and codes."""
    ts = [torch.randn((8192, 2304), device=dev) * (0.5 + i) for i in range(4)]
    am, sc, qs, qts = df.quantize_2d_batch(ts, Fmt.E4M3)
    for i, t in enumerate(ts):
        a1, s1 = df.absmax_scale(t, Fmt.E4M3)
        q1, qt1 = df.quantize_2d(t, s1, Fmt.E4M3, want_q=True, want_qt=True)
        assert am[i].item() == a1.item() and sc[i].item() == s1.item(), f"tensor {i}"
        assert torch.equal(qs[i], q1) and torch.equal(qts[i], qt1), f"codes of tensor {i}"
    del ts, qs, qts
    torch.cuda.empty_cache()


def test_quantize_2d_batch_many_tensors(dev):
    """More tensors than one launch holds (32); only row codes asked for."""
    rng = np.random.default_rng(8)
    ts = [to_dev_f32(rng.standard_normal((17 + 3 * i, 40 + 8 * i)).astype(np.float32), dev) for i in range(41)]
    am, sc, qs, qts = df.quantize_2d_batch(ts, Fmt.E4M3, want_qt=False)
    assert all(q is None for q in qts)
    for i, t in enumerate(ts):
        x = t.cpu().numpy()
        s = orc.scale(orc.absmax(x), int(Fmt.E4M3))
        assert sc[i].item() == np.float32(s)
        assert np.array_equal(qs[i].cpu().numpy()[:, :x.shape[1]], orc.quantize(x, s, int(Fmt.E4M3)))
        assert not qs[i].cpu().numpy()[:, x.shape[1]:].any()  # zero padding


@pytest.mark.parametrize("rb,wb", [(16, 0), (16, 4), (16, 8), (16, 16), (4, 16), (8, 16)])
def test_hbm_probe_patterns(dev, rb, wb):
    """df_hbm_probe (the bandwidth calibration behind the bench's pattern
    ceilings) reads every source vector and writes the documented fold."""
    import deepfuse_amd as dfm
    nbytes = 2048 * rb * 5
    rng = np.random.default_rng(rb * 31 + wb)
    src = rng.integers(0, 1 << 32, size=nbytes // 4, dtype=np.uint64).astype(np.uint32)
    s = torch.from_numpy(src.view(np.int32)).to(dev)
    dbytes = dfm.lib().df_hbm_probe_dst_bytes(rb, wb, nbytes)
    d = torch.zeros(dbytes // 4, dtype=torch.int32, device=dev)
    dfm.call("df_hbm_probe", rb, wb, s.data_ptr(), nbytes, d.data_ptr(), torch.cuda.current_stream().cuda_stream)
    got = d.cpu().numpy().view(np.uint32)
    v = src.reshape(-1, rb // 4)
    if wb == 0:  # one word per block; xor-folds of its chunks, max over its threads: check it is non-trivial
        assert got.size == 5 and np.all(got != 0)
        return
    if rb == 16 and wb == 4:
        exp = v[:, 0] ^ v[:, 1] ^ v[:, 2] ^ v[:, 3]
    elif rb == 16 and wb == 8:
        exp = np.stack([v[:, 0] ^ v[:, 1], v[:, 2] ^ v[:, 3]], 1)
    elif rb == 16 and wb == 16:
        exp = v.copy()
        exp[:, 0] ^= 1
    elif rb == 4:
        w = v[:, 0]
        exp = np.stack([w, w ^ 1, w ^ 2, w ^ 3], 1)
    else:
        exp = np.stack([v[:, 0], v[:, 1], v[:, 0] ^ 1, v[:, 1] ^ 1], 1)
    assert np.array_equal(got, exp.reshape(-1))
