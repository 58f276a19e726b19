"""GPU parity of the consumer side of dW through the C ABI:
df_grad_norm_f32, df_clip_grad_norm_f32 and df_adam_update_f32 against the
oracle (oracle/df_oracle.c: the float paths of
dnn/utils/clip_grad_norm.cu:13-67 and dnn/optimizers/adam_optimizer.cu:11-109).

Bar: the norm within one binary32 ulp of the oracle's (both accumulate
binary32 squares in binary64, in different orders); the clipped gradients
and every Adam output (parameters, m, v) bit-exact, given the same norm.
Lists are ragged (empty tensors, sizes around the 8192-element block chunk,
a tail that is not a multiple of 4) and longer than one launch holds (more
than 64 tensors for the norm, 48 for Adam).
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu

RAGGED = [0, 1, 3, 4, 8191, 8192, 8193, 3 * 8192 + 5, 100_003]


def rand_list(sizes, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal(n) * scale).astype(np.float32) for n in sizes]


def to_dev(arrays, dev):
    return [torch.from_numpy(a.copy()).to(dev) for a in arrays]


def ulps(a: float, b: float) -> int:
    ia = int(np.float32(a).view(np.int32))
    ib = int(np.float32(b).view(np.int32))
    return abs(ia - ib)


@pytest.mark.parametrize("sizes", [RAGGED, [5000] * 70 + [0, 17]])
def test_grad_norm_matches_oracle(dev, sizes):
    host = rand_list(sizes, seed=11)
    norm = df.grad_norm(to_dev(host, dev))
    torch.cuda.synchronize()
    assert ulps(norm.item(), orc.grad_norm(host)) <= 1


def test_grad_norm_large_and_exact_cases(dev):
    # 2^25 ones: a binary32 running sum would stop at 2^24
    ones = torch.ones(1 << 25, dtype=torch.float32, device=dev)
    assert df.grad_norm([ones]).item() == np.float32(np.sqrt(1 << 25))
    t = [torch.tensor([3.0], device=dev), torch.tensor([4.0], device=dev)]
    assert df.grad_norm(t).item() == 5.0
    z = [torch.zeros(0, dtype=torch.float32, device=dev)]
    assert df.grad_norm(z).item() == 0.0
    # GPT-2 XL fc1 weight-gradient size, deterministic across runs
    w = torch.from_numpy(rand_list([6400 * 1600], seed=12, scale=1e-3)[0]).to(dev)
    a, b = df.grad_norm([w]).item(), df.grad_norm([w]).item()
    assert a == b
    assert ulps(a, orc.grad_norm([w.cpu().numpy()])) <= 1


@pytest.mark.parametrize("max_norm", [1.0, 1e9])
def test_clip_grad_norm_in_place(dev, max_norm):
    host = rand_list(RAGGED, seed=13)
    d = to_dev(host, dev)
    norm = df.grad_norm(d, clip=max_norm)
    torch.cuda.synchronize()
    nv = norm.item()
    expect = [a.copy() for a in host]
    clipped = False
    for a in expect:
        clipped |= orc.clip_scale(a, nv, max_norm)
    assert clipped == (max_norm < nv)
    for i, (a, t) in enumerate(zip(expect, d)):
        assert np.array_equal(t.cpu().numpy(), a), f"tensor {i} (size {a.size})"


def adam_case(dev, sizes, steps, wd, max_norm, fused, seed):
    """`steps` Adam steps on the GPU and in the oracle from the same state;
    gradients are clipped at max_norm (None: no clipping) either fused into
    the update or in place beforehand."""
    rng = np.random.default_rng(seed)
    p_h = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    m_h = [np.zeros(n, np.float32) for n in sizes]
    v_h = [np.zeros(n, np.float32) for n in sizes]
    p_d, m_d, v_d = to_dev(p_h, dev), to_dev(m_h, dev), to_dev(v_h, dev)
    lr = 1e-3
    for t in range(1, steps + 1):
        g_h = [(rng.standard_normal(n) * 0.5).astype(np.float32) for n in sizes]
        g_d = to_dev(g_h, dev)
        norm = None
        if max_norm is not None:
            norm = df.grad_norm(g_d, clip=None if fused else max_norm)
            torch.cuda.synchronize()
            nv = norm.item()
        df.adam_update(p_d, g_d, m_d, v_d, t, lr=lr, weight_decay=wd,
                       clip_norm=norm if fused else None, max_norm=max_norm or 0.0)
        f = 1.0
        if max_norm is not None and nv > max_norm:
            f = float(np.float32(max_norm) / np.float32(nv))
        for i in range(len(sizes)):
            orc.adam_step(p_h[i], g_h[i], m_h[i], v_h[i], t, lr=lr, wd=wd, clip_factor=f)
    torch.cuda.synchronize()
    for i in range(len(sizes)):
        for name, d, h in (("p", p_d, p_h), ("m", m_d, m_h), ("v", v_d, v_h)):
            got = d[i].cpu().numpy()
            assert np.array_equal(got, h[i]), f"{name}[{i}] (size {sizes[i]}) differs"


def test_adam_matches_oracle(dev):
    adam_case(dev, RAGGED, steps=3, wd=0.0, max_norm=None, fused=False, seed=21)


def test_adam_weight_decay_many_tensors(dev):
    # more tensors than one launch takes
    adam_case(dev, [1000 + 37 * i for i in range(53)], steps=2, wd=0.01, max_norm=None, fused=False, seed=22)


@pytest.mark.parametrize("fused", [False, True])
def test_adam_with_clipping(dev, fused):
    # norm of these gradients is ~ sqrt(n)/2 >> 1, so every step clips
    adam_case(dev, RAGGED, steps=3, wd=0.01, max_norm=1.0, fused=fused, seed=23)


def test_fused_clip_equals_clip_then_adam_on_device(dev):
    """The fused factor gives the same bits as clipping the gradients in place
    first (the reference's order: clip_grad_norm, then Adam::step)."""
    sizes = [6400 * 1600, 1600, 4800 * 1600]
    rng = np.random.default_rng(24)
    p0 = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    g0 = [(rng.standard_normal(n) * 1e-2).astype(np.float32) for n in sizes]
    outs = []
    for fused in (False, True):
        p, g = to_dev(p0, dev), to_dev(g0, dev)
        m = [torch.zeros_like(x) for x in p]
        v = [torch.zeros_like(x) for x in p]
        norm = df.grad_norm(g, clip=None if fused else 1.0)
        df.adam_update(p, g, m, v, 1, weight_decay=0.01, clip_norm=norm if fused else None, max_norm=1.0)
        torch.cuda.synchronize()
        outs.append((p, m, v))
    for a, b in zip(outs[0], outs[1]):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


def test_argument_errors(dev):
    x = torch.zeros(64, dtype=torch.float32, device=dev)
    with pytest.raises(df.DFError) as ei:
        df.adam_update([x], [x], [x], [x], 0)  # timestep counts from 1
    assert ei.value.status == -1
    with pytest.raises(df.DFError) as ei:
        df.adam_update([x[1:]], [x[1:]], [x[1:]], [x[1:]], 1)  # 4-byte offset: not 16-byte aligned
    assert ei.value.status == -4
    with pytest.raises(df.DFError) as ei:
        df.call("df_grad_norm_f32", df._ptrs([x]), df._sizes([x]), 1, x.data_ptr(), x.data_ptr(), 0, None)
    assert ei.value.status == -5


def test_adam_absmax_output(dev):
    """df_adam_update_absmax_f32: the same parameters, m and v as
    df_adam_update_f32, plus max |p| of every updated tensor (exact; empty
    tensors 0); more tensors than one launch holds."""
    sizes = RAGGED + [7, 4096] * 25
    rng = np.random.default_rng(31)
    p0 = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    g0 = [(rng.standard_normal(n) * 0.5).astype(np.float32) for n in sizes]
    outs = []
    for with_absmax in (False, True):
        p, g = to_dev(p0, dev), to_dev(g0, dev)
        m = [torch.zeros_like(x) for x in p]
        v = [torch.zeros_like(x) for x in p]
        am = torch.full((len(sizes),), -1.0, dtype=torch.float32, device=dev) if with_absmax else None
        df.adam_update(p, g, m, v, 1, weight_decay=0.01, absmax=am)
        torch.cuda.synchronize()
        outs.append((p, m, v, am))
    for a, b in zip(outs[0][:3], outs[1][:3]):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    am = outs[1][3].cpu().numpy()
    for i, x in enumerate(outs[1][0]):
        exp = np.abs(x.cpu().numpy()).max() if x.numel() else 0.0
        assert am[i] == exp, f"tensor {i} (size {sizes[i]})"


def test_adam_absmax_then_batch_quantize(dev):
    """The optimizer step's absmax feeds df_quantize_2d_batch_absmax: the
    scales and codes equal df_quantize_2d_batch's own absmax pass."""
    shapes = [(480, 160), (160, 160), (640, 160), (160, 640)]
    rng = np.random.default_rng(32)
    p = [torch.from_numpy(rng.standard_normal(s).astype(np.float32) * 0.02).to(dev) for s in shapes]
    g = [torch.from_numpy(rng.standard_normal(s).astype(np.float32) * 1e-3).to(dev) for s in shapes]
    m = [torch.zeros_like(x) for x in p]
    v = [torch.zeros_like(x) for x in p]
    am = torch.empty(len(p), dtype=torch.float32, device=dev)
    df.adam_update(p, g, m, v, 1, absmax=am)
    a1, s1, q1, qt1 = df.quantize_2d_batch(p, Fmt.E4M3, absmax=am)
    a2, s2, q2, qt2 = df.quantize_2d_batch(p, Fmt.E4M3)
    assert torch.equal(a1, a2) and torch.equal(s1, s2)
    for i in range(len(p)):
        assert torch.equal(q1[i], q2[i]) and torch.equal(qt1[i], qt2[i])
