"""GPU parity of delayed scaling (df_amax_history_init,
df_quantize_2d_delayed) against the oracle.

Each pass quantizes with the scale the history held before it (codes from
the oracle's quantize at that scale, saturating where the data outgrew it),
measures the pass's absmax and pushes it (oracle dfo_history_push).  Bar:
codes (row and transposed copies), the history and the next scale
bit-exact after every pass; the fused column sums bit-identical to the
just-in-time pass's (same kernel order).
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import Fmt, synth
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).reshape(-1).view(np.uint32)


def to_dev(x, kind, dev):
    if kind == "f32":
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)
    return torch.from_numpy(synth.f32_to_bf16_bits(x).view(np.int16)).to(dev).view(torch.bfloat16)


def host_values(x, kind):
    """The values the pass sees: float32, or bf16 bit patterns for the oracle."""
    return np.ascontiguousarray(x, np.float32) if kind == "f32" else synth.f32_to_bf16_bits(x)


@pytest.mark.parametrize("kind", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [Fmt.E4M3, Fmt.E5M2])
def test_history_sequence(dev, kind, fmt):
    length = 3
    # magnitudes change from pass to pass; pass 3 jumps 16x above the
    # history (saturating codes), pass 5 is empty
    passes = [((200, 300), 1.0), ((129, 257), 0.5), ((64, 1600), 16.0), ((300, 17), 0.25), ((0, 40), 1.0),
              ((1000, 200), 2.0)]
    st = df.DelayedScale(fmt, length, dev)  # zero history: first scale 1
    hist = np.zeros(length, np.float32)
    scale = np.float32(1.0)
    torch.cuda.synchronize()
    assert st.scale.item() == 1.0 and not st.history.cpu().numpy().any()
    saturated = False
    for i, ((rows, cols), mag) in enumerate(passes):
        x = synth.normal((rows, cols), mag, seed=300 + i)
        xd = to_dev(x, kind, dev).view(rows, cols)
        colsum = i % 2 == 0
        out = st.quantize_2d(xd, want_q=True, want_qt=True, colsum=colsum)
        q, qt = out[0], out[1]
        xh = host_values(x, kind)
        flat = orc.quantize(xh, float(scale), int(fmt)).reshape(rows, cols)
        qh, qth = q.cpu().numpy(), qt.cpu().numpy()
        assert np.array_equal(qh[:, :cols], flat), f"pass {i}: q"
        assert np.array_equal(qth[:, :rows], np.ascontiguousarray(flat.T)), f"pass {i}: qt"
        sat_code = 0x7E if fmt == Fmt.E4M3 else 0x7B
        saturated |= bool(((flat & 0x7F) == sat_code).any())
        if colsum and rows:
            _, _, cs_jit = df.quantize_2d(xd, st.scale.new_tensor([float(scale)]), fmt, want_q=False,
                                          want_qt=False, colsum=True)
            assert torch.equal(out[2], cs_jit), f"pass {i}: column sums"
        amax = orc.absmax(xh) if rows else 0.0
        scale = np.float32(orc.history_push(hist, amax, int(fmt)))
        torch.cuda.synchronize()
        assert np.array_equal(bits(st.history.cpu().numpy()), bits(hist)), f"pass {i}: history"
        assert bits(st.scale.cpu().numpy())[0] == bits(scale)[0], f"pass {i}: next scale"
    assert saturated  # the 16x pass ran above the scale it inherited


def test_seeded_history_equals_just_in_time(dev):
    """Seeded with the tensor's own absmax, the delayed pass gives the codes
    of the just-in-time pass."""
    x = torch.from_numpy(synth.normal((333, 1600), 0.02, seed=77)).to(dev)
    am, s = df.absmax_scale(x, Fmt.E4M3)
    st = df.DelayedScale(Fmt.E4M3, 16, dev, seed_amax=am)
    q1, qt1 = st.quantize_2d(x, want_q=True, want_qt=True)
    q0, qt0 = df.quantize_2d(x, s, Fmt.E4M3, want_q=True, want_qt=True)
    torch.cuda.synchronize()
    assert torch.equal(q1, q0) and torch.equal(qt1, qt0)
    assert torch.equal(st.scale, s)  # same amax pushed: same next scale
    h = st.history.cpu().numpy()
    assert (h == am.item()).all()


def test_argument_errors(dev):
    x = torch.zeros((4, 4), dtype=torch.float32, device=dev)
    st = df.DelayedScale(Fmt.E4M3, 4, dev)
    q = torch.empty((4, 16), dtype=torch.uint8, device=dev)
    with pytest.raises(df.DFError) as ei:  # history longer than 1024
        df.call("df_quantize_2d_delayed", 0, x.data_ptr(), 4, 4, 4, 0, st.scale.data_ptr(), st.scale.data_ptr(),
                st.history.data_ptr(), 2000, q.data_ptr(), 16, None, 0, None, q.data_ptr(), 4096, None)
    assert ei.value.status == -1
    with pytest.raises(df.DFError) as ei:  # workspace too small
        df.call("df_quantize_2d_delayed", 0, x.data_ptr(), 4, 4, 4, 0, st.scale.data_ptr(), st.scale.data_ptr(),
                st.history.data_ptr(), 4, q.data_ptr(), 16, None, 0, None, q.data_ptr(), 0, None)
    assert ei.value.status == -5
    with pytest.raises(df.DFError):
        df.DelayedScale(Fmt.E4M3, 0, dev)
