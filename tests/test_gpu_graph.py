"""The path under HIP-graph capture, as bench.py times it: one Linear's step
-- the one-call quantize of X, W and dY (with column sums), the forward GEMM
that also gives Y's absmax and scale, the grouped backward that also gives
dX's -- captured once and replayed three times, with new inputs written
eagerly between the replays.  Every replay's codes, scales, absmax values, Y,
dX, dW and db equal the same calls made eagerly on the same inputs, bit for
bit.  None of these entry points records a memset; partials and scales are
rewritten by every call.

The delayed-scaling form as the bench captures it: two steps per graph (the
two scale slots of each operand alternate), each quantizing the weights in
one batch call (just-in-time) and X and dY at the scale of their amax
histories (df_quantize_2d_delayed, dY with column sums).  Every replay's
histories, scales, codes and column sums equal the same two steps made
eagerly, bit for bit, so the state the histories carry evolves alike."""
import ctypes

import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import DType, Fmt

pytestmark = pytest.mark.gpu

BF, F32, E4, E5 = int(DType.BFLOAT16), int(DType.FLOAT32), int(Fmt.E4M3), int(Fmt.E5M2)


class Step:
    def __init__(self, dev, M, K, N):
        L = df.lib()
        self.M, self.K, self.N = M, K, N
        z = lambda *shape, dt=torch.bfloat16: torch.zeros(shape, dtype=dt, device=dev)
        self.X, self.W, self.dY, self.b = z(M, K), z(N, K), z(M, N), z(N)
        Kp, Np, Mp = df.round16(K), df.round16(N), df.round16(M)
        u8 = lambda r, c: z(r, c, dt=torch.uint8)
        self.xq, self.xt, self.wq, self.wt, self.dyq, self.dyt = u8(M, Kp), u8(K, Mp), u8(N, Kp), u8(K, Np), \
            u8(M, Np), u8(N, Mp)
        self.sc = z(10, dt=torch.float32)
        self.db = z(N, dt=torch.float32)
        self.Y, self.dX, self.dW = z(M, N), z(M, K), z(N, K, dt=torch.float32)
        jb = max(L.df_quantize_2d_jit_workspace_bytes(r, c, 1) for r, c in ((M, K), (N, K), (M, N)))
        gb = max(L.df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K), L.df_fp8_gemm_bwd_absmax_workspace_bytes(M, N, K))
        self.jws = z(jb, dt=torch.uint8)
        self.gws = z(gb, dt=torch.uint8)

    def run(self):
        M, K, N, p = self.M, self.K, self.N, self.sc.data_ptr()
        st = torch.cuda.current_stream().cuda_stream  # the capture stream while capturing
        jw, jb, gw, gb = self.jws.data_ptr(), self.jws.numel(), self.gws.data_ptr(), self.gws.numel()
        df.call("df_quantize_2d_jit", BF, self.X.data_ptr(), M, K, E4, p, p + 4, self.xq.data_ptr(),
                self.xq.stride(0), self.xt.data_ptr(), self.xt.stride(0), None, jw, jb, st)
        df.call("df_quantize_2d_jit", BF, self.W.data_ptr(), N, K, E4, p + 8, p + 12, self.wq.data_ptr(),
                self.wq.stride(0), self.wt.data_ptr(), self.wt.stride(0), None, jw, jb, st)
        df.call("df_fp8_gemm_fwd_absmax", self.xq.data_ptr(), self.xq.stride(0), self.wq.data_ptr(),
                self.wq.stride(0), M, N, K, p + 4, p + 12, BF, self.b.data_ptr(), BF, self.Y.data_ptr(), N, E4,
                p + 24, p + 28, gw, gb, st)
        df.call("df_quantize_2d_jit", BF, self.dY.data_ptr(), M, N, E5, p + 16, p + 20, self.dyq.data_ptr(),
                self.dyq.stride(0), self.dyt.data_ptr(), self.dyt.stride(0), self.db.data_ptr(), jw, jb, st)
        df.call("df_fp8_gemm_bwd_absmax", self.dyq.data_ptr(), self.dyq.stride(0), self.wt.data_ptr(),
                self.wt.stride(0), self.dyt.data_ptr(), self.dyt.stride(0), self.xt.data_ptr(), self.xt.stride(0), M,
                N, K, p + 20, p + 12, p + 4, BF, self.dX.data_ptr(), K, F32, self.dW.data_ptr(), K, E5, p + 32,
                p + 36, gw, gb, st)

    def load(self, seed):
        g = torch.Generator(device=self.X.device).manual_seed(seed)
        for t, std in ((self.X, 1.0), (self.W, 0.02), (self.dY, 1e-3), (self.b, 0.1)):
            t.copy_((torch.randn(t.shape, generator=g, device=t.device) * std).to(t.dtype))

    def outputs(self):
        return {n: getattr(self, n).clone() for n in ("xq", "xt", "wq", "wt", "dyq", "dyt", "sc", "db", "Y", "dX",
                                                       "dW")}


def test_graph_replays_match_eager(dev):
    M, K, N = 16384, 1600, 6400  # config 4's fc1: both GEMMs take the kernels that fold
    assert df.gemm_plan(M, N, K, K, K, None, int(df.lib().df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K)))[0] == \
        df.GemmKernel.PERSISTENT
    assert df.gemm_bwd_plan(M, N, K)[0]  # the grouped backward, which folds |dX|
    g_step, e_step = Step(dev, M, K, N), Step(dev, M, K, N)
    g_step.load(1)
    g_step.run()  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_step.run()
    torch.cuda.synchronize()
    for replay, seed in enumerate((11, 12, 13)):
        g_step.load(seed)
        e_step.load(seed)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e_step.run()
        torch.cuda.synchronize()
        got, exp = g_step.outputs(), e_step.outputs()
        for name in exp:
            assert torch.equal(got[name].view(torch.uint8), exp[name].view(torch.uint8)), f"replay {replay}: {name}"
        assert got["sc"][6:].abs().sum() > 0  # the fused GEMMs wrote their absmax and scale


class DelayedSteps:
    H = 4

    def __init__(self, dev, M, K, N, NW):
        L = df.lib()
        self.M, self.K, self.N = M, K, N
        z = lambda *shape, dt=torch.bfloat16: torch.zeros(shape, dtype=dt, device=dev)
        u8 = lambda r, c: z(r, c, dt=torch.uint8)
        self.X, self.dY = z(M, K), z(M, N)
        self.Ws = [z(N, K), z(NW, K)]
        self.xq, self.xt, self.dyq, self.dyt = u8(M, K), u8(K, M), u8(M, N), u8(N, M)
        self.wq = [u8(w.shape[0], K) for w in self.Ws]
        self.wt = [u8(K, df.round16(w.shape[0])) for w in self.Ws]
        self.db = z(N, dt=torch.float32)
        self.hx, self.hdy = z(self.H, dt=torch.float32), z(self.H, dt=torch.float32)
        self.sx, self.sdy = z(3, dt=torch.float32), z(3, dt=torch.float32)  # slots 0, 1: scales; 2: seed absmax
        self.wam, self.wsc = z(2, dt=torch.float32), z(2, dt=torch.float32)
        db_ = max(L.df_quantize_2d_delayed_workspace_bytes(M, K, K, M, 0),
                  L.df_quantize_2d_delayed_workspace_bytes(M, N, N, M, 1))
        self.dws = z(db_, dt=torch.uint8)
        self.bws = z(L.df_quantize_2d_batch_workspace_bytes(), dt=torch.uint8)
        self.aws = z(L.df_absmax_workspace_bytes(), dt=torch.uint8)

    def load(self, seed):
        g = torch.Generator(device=self.X.device).manual_seed(seed)
        for t, std in ((self.X, 1.0), (self.dY, 1e-3), (self.Ws[0], 0.02), (self.Ws[1], 0.05)):
            t.copy_((torch.randn(t.shape, generator=g, device=t.device) * std).to(t.dtype))

    def seed_histories(self):
        st = torch.cuda.current_stream().cuda_stream
        for x, h, sc, fmt in ((self.X, self.hx, self.sx, E4), (self.dY, self.hdy, self.sdy, E5)):
            df.call("df_absmax_bf16", x.data_ptr(), x.numel(), sc.data_ptr() + 8, self.aws.data_ptr(),
                    self.aws.numel(), st)
            df.call("df_amax_history_init", sc.data_ptr() + 8, fmt, h.data_ptr(), self.H, sc.data_ptr(), st)

    def step(self, parity):
        M, K, N = self.M, self.K, self.N
        st = torch.cuda.current_stream().cuda_stream
        n = len(self.Ws)
        ptrs = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])
        ints = lambda vals: (ctypes.c_int * n)(*vals)
        df.call("df_quantize_2d_batch", BF, n, ptrs(self.Ws), ints([w.shape[0] for w in self.Ws]), ints([K] * n), E4,
                self.wam.data_ptr(), self.wsc.data_ptr(), ptrs(self.wq), ints([q.stride(0) for q in self.wq]),
                ptrs(self.wt), ints([q.stride(0) for q in self.wt]), self.bws.data_ptr(), self.bws.numel(), st)
        for x, rows, cols, fmt, sc, h, q, qt, cs in ((self.X, M, K, E4, self.sx, self.hx, self.xq, self.xt, None),
                                                    (self.dY, M, N, E5, self.sdy, self.hdy, self.dyq, self.dyt,
                                                     self.db)):
            df.call("df_quantize_2d_delayed", BF, x.data_ptr(), rows, cols, cols, fmt, sc.data_ptr() + 4 * parity,
                    sc.data_ptr() + 4 * (parity ^ 1), h.data_ptr(), self.H, q.data_ptr(), q.stride(0),
                    qt.data_ptr(), qt.stride(0), None if cs is None else cs.data_ptr(), self.dws.data_ptr(),
                    self.dws.numel(), st)

    def outputs(self):
        names = ("xq", "xt", "dyq", "dyt", "db", "hx", "hdy", "sx", "sdy", "wam", "wsc")
        out = {n: getattr(self, n).clone() for n in names}
        for i in range(len(self.Ws)):
            out[f"wq{i}"], out[f"wt{i}"] = self.wq[i].clone(), self.wt[i].clone()
        return out


def test_delayed_graph_replays_match_eager(dev):
    M, K, N, NW = 4096, 1600, 1600, 800
    g_st, e_st = DelayedSteps(dev, M, K, N, NW), DelayedSteps(dev, M, K, N, NW)
    for t in (g_st, e_st):
        t.load(5)
        t.seed_histories()
    torch.cuda.synchronize()
    g_st.step(0)  # warm-up outside capture, mirrored eagerly
    g_st.step(1)
    e_st.step(0)
    e_st.step(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_st.step(0)
        g_st.step(1)
    torch.cuda.synchronize()
    for replay, seed in enumerate((21, 22, 23, 24)):
        for t in (g_st, e_st):
            t.load(seed)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e_st.step(0)
        e_st.step(1)
        torch.cuda.synchronize()
        got, exp = g_st.outputs(), e_st.outputs()
        for name in exp:
            assert torch.equal(got[name].view(torch.uint8), exp[name].view(torch.uint8)), f"replay {replay}: {name}"
    assert got["hx"].min() > 0 and got["hdy"].min() > 0  # every history slot holds a measured absmax
