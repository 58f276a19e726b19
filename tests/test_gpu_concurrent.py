"""Calls on different streams are independent (include/df_capi.h's
contract): two host threads, each with its own HIP stream and its own
workspaces, run one Linear's step -- the one-call quantize of X, W and dY
(dY with its column sums), the forward GEMM and the grouped dX + dW GEMM --
on different data at the same time.  Every output (codes, scales, Y, dX,
dW, db) equals the same calls made one after another on one stream, bit for
bit.  ctypes releases the GIL during the calls, so the two threads enqueue
work concurrently."""
import threading

import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import DType, Fmt, synth

pytestmark = pytest.mark.gpu

BF, F32, E4, E5 = int(DType.BFLOAT16), int(DType.FLOAT32), int(Fmt.E4M3), int(Fmt.E5M2)


class Job:
    """One Linear's operands, outputs and workspaces (nothing shared)."""

    def __init__(self, dev, M, K, N, seed):
        L = df.lib()
        bf = lambda shape, std, s: torch.from_numpy(synth.normal(shape, std, seed=s)).to(dev).to(torch.bfloat16)
        self.M, self.K, self.N = M, K, N
        self.X, self.W, self.dY = bf((M, K), 1.0, seed), bf((N, K), 0.02, seed + 1), bf((M, N), 1e-3, seed + 2)
        self.b = bf((N,), 0.1, seed + 3)
        u8 = lambda r, c: torch.empty((r, c), dtype=torch.uint8, device=dev)
        Kp, Np, Mp = df.round16(K), df.round16(N), df.round16(M)
        self.xq, self.xt, self.wq, self.wt = u8(M, Kp), u8(K, Mp), u8(N, Kp), u8(K, Np)
        self.dyq, self.dyt = u8(M, Np), u8(N, Mp)
        self.sc = torch.zeros(8, dtype=torch.float32, device=dev)  # 6 scales and absmax values used
        self.db = torch.empty(N, dtype=torch.float32, device=dev)
        self.Y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        self.dX = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        self.dW = torch.empty((N, K), dtype=torch.float32, device=dev)
        jb = max(L.df_quantize_2d_jit_workspace_bytes(r, c, 1) for r, c in ((M, K), (N, K), (M, N)))
        gb = max(L.df_fp8_gemm_workspace_bytes(M, N, K), L.df_fp8_gemm_bwd_workspace_bytes(M, N, K), 16)
        self.jws = torch.empty(jb, dtype=torch.uint8, device=dev)
        self.gws = torch.empty(gb, dtype=torch.uint8, device=dev)

    def run(self, stream):
        M, K, N, p = self.M, self.K, self.N, self.sc.data_ptr()
        st = stream.cuda_stream
        jw, jb = self.jws.data_ptr(), self.jws.numel()
        gw, gb = self.gws.data_ptr(), self.gws.numel()
        df.call("df_quantize_2d_jit", BF, self.X.data_ptr(), M, K, E4, p, p + 4, self.xq.data_ptr(),
                self.xq.stride(0), self.xt.data_ptr(), self.xt.stride(0), None, jw, jb, st)
        df.call("df_quantize_2d_jit", BF, self.W.data_ptr(), N, K, E4, p + 8, p + 12, self.wq.data_ptr(),
                self.wq.stride(0), self.wt.data_ptr(), self.wt.stride(0), None, jw, jb, st)
        df.call("df_fp8_gemm_fwd", self.xq.data_ptr(), self.xq.stride(0), self.wq.data_ptr(), self.wq.stride(0), M, N,
                K, p + 4, p + 12, BF, self.b.data_ptr(), BF, self.Y.data_ptr(), N, gw, gb, st)
        df.call("df_quantize_2d_jit", BF, self.dY.data_ptr(), M, N, E5, p + 16, p + 20, self.dyq.data_ptr(),
                self.dyq.stride(0), self.dyt.data_ptr(), self.dyt.stride(0), self.db.data_ptr(), jw, jb, st)
        df.call("df_fp8_gemm_bwd", self.dyq.data_ptr(), self.dyq.stride(0), self.wt.data_ptr(), self.wt.stride(0),
                self.dyt.data_ptr(), self.dyt.stride(0), self.xt.data_ptr(), self.xt.stride(0), M, N, K, p + 20,
                p + 12, p + 4, BF, self.dX.data_ptr(), K, F32, self.dW.data_ptr(), K, gw, gb, st)

    def outputs(self):
        return [t.clone() for t in (self.xq, self.xt, self.wq, self.wt, self.dyq, self.dyt, self.sc, self.db, self.Y,
                                    self.dX, self.dW)]


def test_two_streams_match_sequential(dev):
    jobs = [Job(dev, 4096, 1600, 1600, seed=8100), Job(dev, 2048, 768, 3072, seed=8200)]
    one = torch.cuda.Stream()
    expect = []
    for j in jobs:  # one after another on one stream
        j.run(one)
        one.synchronize()
        expect.append(j.outputs())
    for j in jobs:  # forget the results
        for t in (j.Y, j.dX, j.dW, j.db, j.sc):
            t.zero_()
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    go = threading.Barrier(2)
    errors = []

    def worker(i):
        try:
            go.wait()
            for _ in range(3):  # repeat, so the two streams' kernels overlap
                jobs[i].run(streams[i])
            streams[i].synchronize()
        except Exception as exc:  # reported below, on the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    names = ("xq", "xt", "wq", "wt", "dyq", "dyt", "scales", "db", "Y", "dX", "dW")
    for i, j in enumerate(jobs):
        for name, got, exp in zip(names, j.outputs(), expect[i]):
            assert torch.equal(got.view(torch.uint8), exp.view(torch.uint8)), f"job {i}: {name}"


def test_python_wrappers_keep_a_workspace_per_stream(dev):
    """The package's wrappers cache their workspaces per device and stream:
    two streams get different ones, and wrapper calls queued on two streams
    without synchronisation (their kernels free to overlap) give the results
    of the same calls made one after another, bit for bit."""
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        w1 = df._scratch(dev, 1 << 20, "jit")
    with torch.cuda.stream(s2):
        w2 = df._scratch(dev, 1 << 20, "jit")
    assert w1.data_ptr() != w2.data_ptr()
    bf = lambda shape, std, s: torch.from_numpy(synth.normal(shape, std, seed=s)).to(dev).to(torch.bfloat16)
    xs = [bf((4096, 1600), 1.0, 8300), bf((2048, 6400), 1.0, 8301)]
    ws_ = [bf((1600, 1600), 0.02, 8302), bf((768, 6400), 0.02, 8303)]

    def job(i):
        am, sc, q, qt, cs = df.quantize_2d_jit(xs[i], Fmt.E5M2, want_q=True, want_qt=True, colsum=True)
        _, sw, wq, _ = df.quantize_2d_jit(ws_[i], Fmt.E4M3)
        y = df.gemm_nt(q, Fmt.E5M2, wq, Fmt.E4M3, xs[i].shape[1], sc, sw, out_dtype=torch.float32)
        return [am, sc, q, qt, cs, y]

    expect = [job(0), job(1)]
    torch.cuda.synchronize()
    got = [[], []]
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream())
    for _ in range(3):  # queued back to back on both streams, no synchronisation between
        for i, s in enumerate((s1, s2)):
            with torch.cuda.stream(s):
                got[i] = job(i)
    torch.cuda.synchronize()
    names = ("absmax", "scale", "q", "qt", "colsum", "y")
    for i in range(2):
        for name, g, e in zip(names, got[i], expect[i]):
            assert torch.equal(g.view(torch.uint8), e.view(torch.uint8)), f"stream {i}: {name}"
