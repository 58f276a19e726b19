"""Layer-streamed GPT-2 XL Linear stack (the config-5 workload) over the C ABI.

The reference's README describes layer-serialized execution with weights
brought in per layer (README.md:212-226); its host-side pieces live in the
NVMe loader (pinned cudaHostAlloc buffers, per-slot streams and
cudaMemcpyAsync, apps/host-multi/NVMeLoader_Linux.hpp:20-26,64-71,123-125).
Here every layer's four Linears (qkv 1600->4800, attn proj 1600->1600, fc
1600->6400, proj 6400->1600) keep their e4m3 weight codes in pinned host
memory: W [N, K] for the forward sweep and W^T [K, N] for the backward sweep
(layers in reverse), brought to the device through a df_streamer ring of
device slots on the streamer's copy streams while earlier layers compute.

Per layer and Linear, forward: absmax + 2-D quantize of the activation X
(e4m3, the row copy and the transposed copy that this layer's dW reads) and
Y = Xq . Wq^T * sx * sw + b; backward: absmax + 2-D quantize of the upstream
gradient dY (e5m2, both copies, db fused), then dX and dW in one grouped
launch (df_fp8_gemm_bwd).  Every layer has its own seeded activations and
gradients (made on the device from per-layer seeds: 183 MB of X and 236 MB
of dY per layer at 8192 tokens), so no layer finds its inputs still in the
256 MB Infinity Cache from another layer; the weights differ per layer too.

Used by bench.py's streaming leg and by tests/test_gpu_stream.py, so the
test runs exactly the launches the bench times.  torch is only the device
allocator and stream provider here.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import DType, Fmt, WeightStreamer, _in_dtype, call, lib, round16, synth

XL_LINEARS = [("qkv", 1600, 4800), ("attn_proj", 1600, 1600), ("fc", 1600, 6400), ("proj", 6400, 1600)]


class StreamedStack:
    """The stack's weights (pinned host codes), inputs and output buffers.

    keep_outputs=False (the bench): Y and dX of a Linear and the row codes
    of X and dY are overwritten by every layer; dW and the transposed X
    codes (which dW reads in the backward sweep) are kept per layer.
    keep_outputs=True (the tests): Y, dX, dW and every code buffer are kept
    per layer, so a whole step can be compared afterwards.  out_dtype is the
    dtype of Y and dX (bf16 in the bench); dW is fp32."""

    def __init__(self, torch, dev, layers=48, tokens=8192, linears=XL_LINEARS, keep_outputs=False,
                 out_dtype=None):
        self.torch = torch
        self.dev = dev
        self.layers = layers
        self.M = tokens
        self.linears = list(linears)
        self.keep = keep_outputs
        self.out_dtype = out_dtype if out_dtype is not None else torch.bfloat16
        if self.out_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"StreamedStack: out_dtype must be float32 or bfloat16, got {self.out_dtype}")
        r16 = round16
        self.fwd_off, self.bwd_off = [], []
        o1 = o2 = 0
        for _, K, N in self.linears:
            self.fwd_off.append(o1)
            o1 += N * r16(K)
            self.bwd_off.append(o2)
            o2 += K * r16(N)
        self.blob = max(o1, o2)  # bytes of one layer's codes in one direction
        self.total_host = 2 * layers * self.blob
        hp = ctypes.c_void_p()
        call("df_host_alloc", self.total_host, ctypes.byref(hp))
        self.host_ptr = hp.value
        self.host = torch.frombuffer((ctypes.c_uint8 * self.total_host).from_address(hp.value), dtype=torch.uint8)
        try:
            self._build()
        except BaseException:
            self.close()
            raise

    # ------------------------------------------------------------ set-up --
    def cur(self):
        return self.torch.cuda.current_stream().cuda_stream

    def weight_seed(self, l, i):
        return synth.SEED_BASE + 5000 + 10 * l + i

    def act_seed(self, l, i):
        return synth.SEED_BASE + 7000 + 10 * l + i

    def grad_seed(self, l, i):
        return synth.SEED_BASE + 9000 + 10 * l + i

    def _normal_bf16(self, shape, std, seed):
        """N(0, std) in bf16, generated on the device from `seed`."""
        torch = self.torch
        gen = torch.Generator(device=self.dev)
        gen.manual_seed(seed)
        return (torch.randn(shape, generator=gen, device=self.dev) * std).to(torch.bfloat16)

    def weight_bf16(self, l, i):
        """Layer l's Linear i weights W [N, K] (bf16, regenerated on the
        device from their seed)."""
        _, K, N = self.linears[i]
        return self._normal_bf16((N, K), 0.02, self.weight_seed(l, i))

    def _build(self):
        torch, dev, M = self.torch, self.dev, self.M
        r16 = round16
        L = len(self.linears)
        # weights: seeded on the device, quantized with the library's own
        # kernels, stored as codes (row and transposed) in pinned host memory
        self.sw = torch.empty((self.layers, L), dtype=torch.float32, device=dev)
        am = torch.empty(1, dtype=torch.float32, device=dev)
        self.ws = torch.empty(lib().df_absmax_workspace_bytes(), dtype=torch.uint8, device=dev)
        for l in range(self.layers):
            for i, (_, K, N) in enumerate(self.linears):
                W = self.weight_bf16(l, i)
                s_ptr = self.sw_ptr(l, i)
                call("df_absmax_scale_bf16", W.data_ptr(), W.numel(), int(Fmt.E4M3), am.data_ptr(), s_ptr,
                     self.ws.data_ptr(), self.ws.numel(), self.cur())
                wq = torch.empty((N, r16(K)), dtype=torch.uint8, device=dev)
                wt = torch.empty((K, r16(N)), dtype=torch.uint8, device=dev)
                call("df_quantize_2d", int(DType.BFLOAT16), W.data_ptr(), N, K, K, int(Fmt.E4M3), s_ptr,
                     wq.data_ptr(), wq.stride(0), wt.data_ptr(), wt.stride(0), self.cur())
                fb = self.host_offset(l, 0) + self.fwd_off[i]
                bb = self.host_offset(l, 1) + self.bwd_off[i]
                self.host[fb:fb + wq.numel()].copy_(wq.reshape(-1).cpu())
                self.host[bb:bb + wt.numel()].copy_(wt.reshape(-1).cpu())
        torch.cuda.synchronize()

        def to_bf16(a):
            return torch.from_numpy(synth.f32_to_bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)

        # per layer and Linear: its activation X ~ N(0, 1) and upstream
        # gradient dY ~ N(0, 1e-3), bf16 (the bias is one per Linear)
        self.acts = [[self._normal_bf16((M, K), 1.0, self.act_seed(l, i)) for i, (_, K, N) in enumerate(self.linears)]
                     for l in range(self.layers)]
        self.grads = [[self._normal_bf16((M, N), 1e-3, self.grad_seed(l, i))
                       for i, (_, K, N) in enumerate(self.linears)] for l in range(self.layers)]
        self.bias = [to_bf16(synth.normal((N,), 0.02, seed=self.input_seed(i) + 2))
                     for i, (_, K, N) in enumerate(self.linears)]
        Mp = r16(M)
        self.Mp = Mp
        nl = self.layers if self.keep else 1
        self.xq = [[torch.empty((M, r16(K)), dtype=torch.uint8, device=dev) for _, K, N in self.linears]
                   for _ in range(nl)]
        self.xt = [[torch.empty((K, Mp), dtype=torch.uint8, device=dev) for _, K, N in self.linears]
                   for _ in range(self.layers)]
        self.dyq = [[torch.empty((M, r16(N)), dtype=torch.uint8, device=dev) for _, K, N in self.linears]
                    for _ in range(nl)]
        self.dyt = [[torch.empty((N, Mp), dtype=torch.uint8, device=dev) for _, K, N in self.linears]
                    for _ in range(nl)]
        self.Y = [[torch.empty((M, N), dtype=self.out_dtype, device=dev) for _, K, N in self.linears]
                  for _ in range(nl)]
        self.dX = [[torch.empty((M, K), dtype=self.out_dtype, device=dev) for _, K, N in self.linears]
                   for _ in range(nl)]
        self.dW = [[torch.empty((N, K), dtype=torch.float32, device=dev) for _, K, N in self.linears]
                   for _ in range(self.layers)]
        self.db = [[torch.empty((N,), dtype=torch.float32, device=dev) for _, K, N in self.linears]
                   for _ in range(nl)]
        # per layer and Linear: absmax X, scale X, absmax dY, scale dY
        self.sc = torch.empty((self.layers, L, 4), dtype=torch.float32, device=dev)
        # one-call quantize (df_quantize_2d_jit): absmax partials, and the
        # column-sum partials of dY
        self.cws = torch.empty(max(lib().df_quantize_2d_jit_workspace_bytes(M, max(K, N), 1)
                                   for _, K, N in self.linears), dtype=torch.uint8, device=dev)
        gws_b = max(max(lib().df_fp8_gemm_workspace_bytes(M, n, k), lib().df_fp8_gemm_bwd_workspace_bytes(M, n, k))
                    for _, k, n in self.linears)
        self.gws = torch.empty(max(gws_b, 16), dtype=torch.uint8, device=dev)
        # the order of a step: forward sweep, then the backward sweep in reverse
        self.seq = [(0, l) for l in range(self.layers)] + [(1, l) for l in reversed(range(self.layers))]
        self.step_flops = 3 * 2 * M * sum(K * N for _, K, N in self.linears) * self.layers

    def new_outputs(self):
        """Fresh Y / dX / dW buffers for the next step; returns the previous
        ones (lists indexed [layer or 0][linear]) so a caller can compare
        two steps."""
        torch, dev, M = self.torch, self.dev, self.M
        old = (self.Y, self.dX, self.dW)
        nl = self.layers if self.keep else 1
        self.Y = [[torch.empty((M, N), dtype=self.out_dtype, device=dev) for _, K, N in self.linears]
                  for _ in range(nl)]
        self.dX = [[torch.empty((M, K), dtype=self.out_dtype, device=dev) for _, K, N in self.linears]
                   for _ in range(nl)]
        self.dW = [[torch.empty((N, K), dtype=torch.float32, device=dev) for _, K, N in self.linears]
                   for _ in range(self.layers)]
        return old

    def input_seed(self, i):
        return synth.SEED_BASE + 5 + 10 * i

    def sw_ptr(self, l, i):
        return self.sw.data_ptr() + 4 * (l * len(self.linears) + i)

    def sc_ptr(self, l, i):
        """Device address of layer l's Linear i scale record (absmax X,
        scale X, absmax dY, scale dY)."""
        return self.sc.data_ptr() + 16 * (l * len(self.linears) + i)

    def host_offset(self, l, direction):
        """Byte offset of layer l's codes (direction 0: W, 1: W^T) in host memory."""
        return (2 * l + direction) * self.blob

    def _dt(self, t):
        return int(_in_dtype(t))

    # ------------------------------------------------------------ layers --
    def fwd_layer(self, l, base):
        """Forward of layer l with its W codes at device address `base`."""
        M, cur = self.M, self.cur()
        BF, E4 = int(DType.BFLOAT16), int(Fmt.E4M3)
        o = l if self.keep else 0
        for i, (_, K, N) in enumerate(self.linears):
            s = self.sc_ptr(l, i)
            x, xq = self.acts[l][i], self.xq[o][i]
            call("df_quantize_2d_jit", BF, x.data_ptr(), M, K, E4, s, s + 4, xq.data_ptr(), xq.stride(0),
                 self.xt[l][i].data_ptr(), self.Mp, None, self.cws.data_ptr(), self.cws.numel(), cur)
            Y = self.Y[o][i]
            call("df_fp8_gemm_fwd", xq.data_ptr(), xq.stride(0), base + self.fwd_off[i], round16(K), M, N, K, s + 4,
                 self.sw_ptr(l, i), BF, self.bias[i].data_ptr(), self._dt(Y), Y.data_ptr(), N, self.gws.data_ptr(),
                 self.gws.numel(), cur)

    def bwd_layer(self, l, base):
        """Backward of layer l with its W^T codes at device address `base`."""
        M, cur = self.M, self.cur()
        BF, F32, E5 = int(DType.BFLOAT16), int(DType.FLOAT32), int(Fmt.E5M2)
        o = l if self.keep else 0
        for i, (_, K, N) in enumerate(self.linears):
            s = self.sc_ptr(l, i)
            g, dyq, dyt = self.grads[l][i], self.dyq[o][i], self.dyt[o][i]
            call("df_quantize_2d_jit", BF, g.data_ptr(), M, N, E5, s + 8, s + 12, dyq.data_ptr(), dyq.stride(0),
                 dyt.data_ptr(), self.Mp, self.db[o][i].data_ptr(), self.cws.data_ptr(), self.cws.numel(), cur)
            # dX and dW in one launch; dW reads the transposed X codes that
            # layer l's forward cached in xt[l], at that pass's scale s + 4
            dX = self.dX[o][i]
            call("df_fp8_gemm_bwd", dyq.data_ptr(), dyq.stride(0), base + self.bwd_off[i], round16(N), dyt.data_ptr(),
                 self.Mp, self.xt[l][i].data_ptr(), self.Mp, M, N, K, s + 12, self.sw_ptr(l, i), s + 4, self._dt(dX),
                 dX.data_ptr(), K, F32, self.dW[l][i].data_ptr(), K, self.gws.data_ptr(), self.gws.numel(), cur)

    # ------------------------------------------------------------- steps --
    def streamed_step(self, streamer: WeightStreamer, micro_batches: int = 1):
        """One fwd+bwd step with the weights streamed through `streamer`
        (slots >= 3, slot_bytes >= self.blob).  The load of entry idx +
        slots - 2 is issued right after entry idx's launches: it blocks the
        host until entry idx - 2 has finished, so entries idx - 1 and idx
        stay queued on the compute stream.

        micro_batches > 1: that many fwd+bwd passes back to back with the
        same weights (gradient accumulation: the weights change only after
        the last one), the loads running ahead across pass boundaries, so
        the next pass's first W loads overlap this pass's backward.  Each
        pass recomputes the same outputs here (same inputs)."""
        ahead = streamer.slots - 2
        assert ahead >= 1 and micro_batches >= 1
        seq = self.seq * micro_batches
        pending = [streamer.load(self.host_ptr + self.host_offset(ll, dd), self.blob) for dd, ll in seq[:ahead]]
        for idx, (d, l) in enumerate(seq):
            slot, base = pending.pop(0)
            streamer.wait(slot)
            (self.fwd_layer if d == 0 else self.bwd_layer)(l, base)
            streamer.release(slot)
            if idx + ahead < len(seq):
                dd, ll = seq[idx + ahead]
                pending.append(streamer.load(self.host_ptr + self.host_offset(ll, dd), self.blob))

    def resident_weights(self):
        """A device copy of every layer's codes (both directions)."""
        dev_w = self.torch.empty(self.total_host, dtype=self.torch.uint8, device=self.dev)
        dev_w.copy_(self.host)
        return dev_w

    def resident_entry(self, dev_w, d, l):
        base = dev_w.data_ptr() + self.host_offset(l, d)
        (self.fwd_layer if d == 0 else self.bwd_layer)(l, base)

    def resident_step(self, dev_w):
        """The same step with every layer's weights read from `dev_w`."""
        for d, l in self.seq:
            self.resident_entry(dev_w, d, l)

    def close(self):
        if self.host_ptr is not None:
            self.torch.cuda.synchronize()
            call("df_host_free", self.host_ptr)
            self.host_ptr = None
            self.host = None
