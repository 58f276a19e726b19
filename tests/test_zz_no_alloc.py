"""df_quantize_2d_delayed_noalloc, the allocation-free variant of
df_quantize_2d_delayed (its workspace is a fixed device array inside the
library), against df_quantize_2d_delayed with a caller workspace.

Bar: bit-exact (codes, transposed codes, column sums, amax history, next
scale) on two calls in a row -- the second smaller than the first, so stale
scratch contents from the first call would show -- and a clear rejection of
sizes whose scratch need exceeds the fixed maximum.  Called through the C ABI.
"""
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import DType, Fmt, synth

pytestmark = pytest.mark.gpu

LIMIT = 16 << 20  # DF_QUANTIZE_2D_NOALLOC_SCRATCH_BYTES (include/df_capi.h)


def _fn():
    return df.lib().df_quantize_2d_delayed_noalloc


def run_both(dev, x, fmt, hist_a, sc_a, hist_b, sc_b, colsum):
    """One pass of each entry point on the same input and equal state."""
    rows, cols = x.shape
    r16 = df.round16
    st = torch.cuda.current_stream().cuda_stream
    out = []
    for which, (hist, sc) in (("ws", (hist_a, sc_a)), ("noalloc", (hist_b, sc_b))):
        q = torch.full((rows, r16(cols)), 0xEE, dtype=torch.uint8, device=dev)
        qt = torch.full((cols, r16(rows)), 0xEE, dtype=torch.uint8, device=dev)
        cs = torch.full((cols,), float("nan"), dtype=torch.float32, device=dev) if colsum else None
        dt = int(DType.FLOAT32) if x.dtype == torch.float32 else int(DType.BFLOAT16)
        if which == "ws":
            nbytes = df.lib().df_quantize_2d_delayed_workspace_bytes(rows, cols, q.stride(0), qt.stride(0), int(colsum))
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
            df.call("df_quantize_2d_delayed", dt, x.data_ptr(), rows, cols, x.stride(0), int(fmt), sc.data_ptr(),
                    sc.data_ptr(), hist.data_ptr(), hist.numel(), q.data_ptr(), q.stride(0), qt.data_ptr(),
                    qt.stride(0), cs.data_ptr() if colsum else None, ws.data_ptr(), ws.numel(), st)
        else:
            rc = _fn()(dt, x.data_ptr(), rows, cols, x.stride(0), int(fmt), sc.data_ptr(), sc.data_ptr(),
                       hist.data_ptr(), hist.numel(), q.data_ptr(), q.stride(0), qt.data_ptr(), qt.stride(0),
                       cs.data_ptr() if colsum else None, st)
            df.check("df_quantize_2d_delayed_noalloc", rc)
        out.append((q, qt, cs))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fmt,colsum", [(Fmt.E4M3, False), (Fmt.E5M2, True)])
def test_noalloc_matches_workspace_entry_point(dev, dtype, fmt, colsum):
    hl = 16
    seed_amax = torch.tensor([3.0], dtype=torch.float32, device=dev)
    a = df.DelayedScale(fmt, hl, dev, seed_amax=seed_amax)
    b = df.DelayedScale(fmt, hl, dev, seed_amax=seed_amax)
    # first call large (GPT-2 XL dY: 16384 x 6400 with column sums is ~3.3 MB of
    # scratch), second smaller and ragged
    for i, (rows, cols, std) in enumerate([(16384, 6400, 1.0), (1000, 1600 + 7, 5.0)]):
        x = torch.from_numpy(synth.normal((rows, cols), std, seed=synth.SEED_BASE + 70 + i)).to(dev).to(dtype)
        (qa, qta, csa), (qb, qtb, csb) = run_both(dev, x, fmt, a.history, a.scale, b.history, b.scale, colsum)
        assert torch.equal(qa, qb), f"call {i}: codes differ"
        assert torch.equal(qta, qtb), f"call {i}: transposed codes differ"
        if colsum:
            assert torch.equal(csa.view(torch.int32), csb.view(torch.int32)), f"call {i}: column sums differ"
        assert torch.equal(a.history.view(torch.int32), b.history.view(torch.int32)), f"call {i}: history"
        assert torch.equal(a.scale.view(torch.int32), b.scale.view(torch.int32)), f"call {i}: next scale"


def test_noalloc_rejects_oversized(dev):
    """A shape whose column-sum partials alone exceed the fixed scratch is
    refused before any launch, with DF_ERR_WORKSPACE and a message naming
    the limit."""
    rows, cols = 65536, 8192  # 512 tiles x 8192 columns x 4 B = 16 MiB of partials + tile maxima
    need = df.lib().df_quantize_2d_delayed_workspace_bytes(rows, cols, cols, 0, 1)
    assert need > LIMIT
    hist = torch.zeros(4, dtype=torch.float32, device=dev)
    sc = torch.ones(1, dtype=torch.float32, device=dev)
    # x and q are NULL and colsum is a real (tiny) buffer, so the size is
    # that of the column-sum partials: the size check refuses the call
    # first, and were it to pass, the NULL-pointer checks would still refuse
    # it with no launch
    cs = torch.zeros(4, dtype=torch.float32, device=dev)
    rc = _fn()(int(DType.BFLOAT16), None, rows, cols, cols, int(Fmt.E5M2), sc.data_ptr(), sc.data_ptr(),
               hist.data_ptr(), 4, None, cols, None, 0, cs.data_ptr(), None)
    assert rc == -5
    msg = df.lib().df_last_error_string().decode()
    assert str(LIMIT) in msg and "df_quantize_2d_delayed_noalloc" in msg
    torch.cuda.synchronize()
