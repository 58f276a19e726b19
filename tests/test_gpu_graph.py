"""The path under HIP-graph capture, as bench.py times it: one Linear's step
-- the one-call quantize of X, W and dY (with column sums), the forward GEMM
that also gives Y's absmax and scale, the grouped backward that also gives
dX's -- captured once and replayed three times, with new inputs written
eagerly between the replays.  Every replay's codes, scales, absmax values, Y,
dX, dW and db equal the same calls made eagerly on the same inputs, bit for
bit.  None of these entry points records a memset; partials and scales are
rewritten by every call."""
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
