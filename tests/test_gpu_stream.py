"""GPU tests of layer weight streaming (df_streamer_*): a stack of Linear
layers whose e4m3 weight codes live in pinned host memory and reach the GEMM
through a ring of device slots filled on a copy stream.

Bar: every streamed GEMM output is bit-identical to the same GEMM reading
the weights from resident device memory (same kernel, same operands), with
few slots and many layers so every slot is refilled while earlier layers'
kernels may still be queued; misuse of the slot protocol is refused.
"""
import ctypes

import numpy as np
import pytest
import torch

import deepfuse_amd as df
from deepfuse_amd import DType, Fmt, synth

pytestmark = pytest.mark.gpu


def pinned(nbytes):
    """df_host_alloc'ed pinned buffer as (pointer, uint8 CPU tensor view)."""
    p = ctypes.c_void_p()
    df.call("df_host_alloc", nbytes, ctypes.byref(p))
    arr = (ctypes.c_uint8 * nbytes).from_address(p.value)
    return p.value, torch.frombuffer(arr, dtype=torch.uint8)


def make_stack(dev, layers, shapes, seed):
    """Per layer, the e4m3 codes [N, round16(K)] of each (K, N) Linear packed
    back to back, their scales, and one bf16 activation per shape."""
    blobs, scales, resident = [], [], []
    for l in range(layers):
        parts, sc_l, res_l = [], [], []
        for i, (K, N) in enumerate(shapes):
            W = torch.from_numpy(synth.normal((N, K), 0.02, seed=seed + 100 * l + i)).to(dev)
            _, sw = df.absmax_scale(W, Fmt.E4M3)
            wq, _ = df.quantize_2d(W, sw, Fmt.E4M3)
            parts.append(wq.reshape(-1))
            sc_l.append(sw)
            res_l.append(wq)
        blobs.append(torch.cat(parts))
        scales.append(sc_l)
        resident.append(res_l)
    return blobs, scales, resident


def run_stack(dev, slots, layers, shapes, M, prefetch):
    seed = synth.SEED_BASE + 500 + slots
    blobs, scales, resident = make_stack(dev, layers, shapes, seed)
    blob_bytes = max(b.numel() for b in blobs)
    host_ptr, host = pinned(blob_bytes * layers)
    try:
        for l, b in enumerate(blobs):
            host[l * blob_bytes:l * blob_bytes + b.numel()].copy_(b.cpu())
        xs, xq, sx = [], [], []
        for i, (K, N) in enumerate(shapes):
            X = torch.from_numpy(synth.normal((M, K), 1.0, seed=seed + 7 + i)).to(dev)
            _, s = df.absmax_scale(X, Fmt.E4M3)
            q, _ = df.quantize_2d(X, s, Fmt.E4M3)
            xs.append(X), xq.append(q), sx.append(s)
        st = torch.cuda.current_stream().cuda_stream

        def gemm(i, w_ptr, ldw, sw, out):
            K, N = shapes[i]
            df.call("df_fp8_gemm_fwd", xq[i].data_ptr(), xq[i].stride(0), w_ptr, ldw, M, N, K,
                    sx[i].data_ptr(), sw.data_ptr(), int(DType.FLOAT32), None, int(DType.FLOAT32),
                    out.data_ptr(), N, None, 0, st)

        # resident reference
        ref = [[torch.empty((M, N), dtype=torch.float32, device=dev) for (K, N) in shapes] for _ in range(layers)]
        for l in range(layers):
            for i in range(len(shapes)):
                gemm(i, resident[l][i].data_ptr(), resident[l][i].stride(0), scales[l][i], ref[l][i])
        torch.cuda.synchronize()

        # streamed: loads issued `prefetch` layers ahead
        streamer = df.WeightStreamer(slots, blob_bytes)
        out = [[torch.empty((M, N), dtype=torch.float32, device=dev) for (K, N) in shapes] for _ in range(layers)]
        pending = []
        nxt = 0
        for l in range(layers):
            while nxt < layers and nxt <= l + prefetch:
                pending.append(streamer.load(host_ptr + nxt * blob_bytes, blobs[nxt].numel()))
                nxt += 1
            slot, base = pending.pop(0)
            streamer.wait(slot)
            off = 0
            for i, (K, N) in enumerate(shapes):
                gemm(i, base + off, df.round16(K), scales[l][i], out[l][i])
                off += N * df.round16(K)
            streamer.release(slot)
        torch.cuda.synchronize()
        streamer.close()
        for l in range(layers):
            for i in range(len(shapes)):
                assert torch.equal(out[l][i], ref[l][i]), f"layer {l} linear {i} differs"
    finally:
        df.call("df_host_free", host_ptr)


@pytest.mark.parametrize("slots,prefetch", [(2, 1), (3, 2), (4, 1), (6, 3)])
def test_streamed_stack_matches_resident(dev, slots, prefetch):
    # long GEMMs keep the compute stream busy, so a refill that did not wait
    # for the release event would overwrite weights still being read;
    # prefetch = slots - 1 makes every load wait for the layer just queued,
    # prefetch = slots - 3 is the pattern that keeps two layers queued
    run_stack(dev, slots, layers=9, shapes=[(1600, 1600), (320, 4800)], M=4096, prefetch=prefetch)


def test_streamer_refuses_unreleased_slot(dev):
    nbytes = 4096
    host_ptr, host = pinned(nbytes)
    try:
        s = df.WeightStreamer(2, nbytes)
        s.load(host_ptr, nbytes)
        s.load(host_ptr, nbytes)
        with pytest.raises(df.DFError) as ei:
            s.load(host_ptr, nbytes)  # slot 0 was never released
        assert ei.value.status == -1
        with pytest.raises(df.DFError):
            s.load(host_ptr, nbytes * 2)  # larger than a slot
        with pytest.raises(df.DFError):
            s.release(5)
        s.release(0)
        slot, _ = s.load(host_ptr, nbytes)
        assert slot == 0
        s.close()
        torch.cuda.synchronize()
    finally:
        df.call("df_host_free", host_ptr)


# ---------------------------------------------------------------------------
# Config 5 as the bench runs it: the 48-layer GPT-2 XL Linear stack
# (deepfuse_amd.stack.StreamedStack, four Linears per layer), 8192 tokens,
# forward then backward with the W^T codes streamed in reverse, 6 slots and
# loads issued slots - 2 entries ahead -- the README's layer-serialized
# execution (README.md:212-226) with the NVMe loader's pinned buffers and
# async copies (apps/host-multi/NVMeLoader_Linux.hpp:22,69,124).
from deepfuse_amd.stack import StreamedStack  # noqa: E402
from oracle import pyoracle as orc  # noqa: E402

C5_LAYERS, C5_TOKENS, C5_SLOTS = 48, 8192, 6


@pytest.fixture(scope="module")
def config5(dev):
    """One streamed step and one resident step of the config-5 stack, every
    layer's Y, dX (bf16, as the bench) and dW (fp32) kept from each.  Each
    layer has its own activations and gradients."""
    stack = StreamedStack(torch, dev, layers=C5_LAYERS, tokens=C5_TOKENS, keep_outputs=True)
    try:
        streamer = df.WeightStreamer(C5_SLOTS, stack.blob)
        stack.streamed_step(streamer)
        torch.cuda.synchronize()
        streamer.close()
        streamed = stack.new_outputs()
        dev_w = stack.resident_weights()
        stack.resident_step(dev_w)
        torch.cuda.synchronize()
        yield stack, streamed, dev_w
    finally:
        stack.close()


def test_config5_streamed_equals_resident(config5):
    """Every Y, dX and dW of all 48 layers is bit-identical between the
    streamed step and the step reading resident weights."""
    stack, (Ys, dXs, dWs), _ = config5
    for l in range(C5_LAYERS):
        for i, (name, K, N) in enumerate(stack.linears):
            assert torch.equal(Ys[l][i], stack.Y[l][i]), f"Y layer {l} {name}"
            assert torch.equal(dXs[l][i], stack.dX[l][i]), f"dX layer {l} {name}"
            assert torch.equal(dWs[l][i], stack.dW[l][i]), f"dW layer {l} {name}"
    # the layers' inputs differ, so their dW do (dW = dY^T . X does not
    # involve W; equal dW would mean the layers read the same inputs)
    for i, (name, K, N) in enumerate(stack.linears):
        assert not torch.equal(dWs[1][i], dWs[0][i]), f"dW of layers 0 and 1 equal ({name})"


def test_config5_micro_batches_stream_across_passes(config5):
    """Two passes with the same weights and the loads running ahead across
    the pass boundary (stack.streamed_step(streamer, 2)), with copy timing
    on: the outputs of the second pass are bit-identical to the resident
    step's, and every one of the 2 x 96 copies is logged in load order."""
    stack, _, _ = config5
    ref = stack.new_outputs()  # the resident step's outputs
    streamer = df.WeightStreamer(C5_SLOTS, stack.blob)
    try:
        streamer.set_timing(True)
        stack.streamed_step(streamer, micro_batches=2)
        torch.cuda.synchronize()
        log = streamer.copy_log()
        assert len(log) == 2 * len(stack.seq)
        assert all(b >= a for a, b in log)
        assert streamer.copy_log() == []  # the first read cleared it
    finally:
        streamer.close()
    Ys, dXs, dWs = ref
    for l in range(C5_LAYERS):
        for i, (name, K, N) in enumerate(stack.linears):
            assert torch.equal(Ys[l][i], stack.Y[l][i]), f"Y layer {l} {name}"
            assert torch.equal(dXs[l][i], stack.dX[l][i]), f"dX layer {l} {name}"
            assert torch.equal(dWs[l][i], stack.dW[l][i]), f"dW layer {l} {name}"


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _band_rows(M, seed, band=256):
    rng = np.random.default_rng(seed)
    rows = set()
    for b0 in range(0, M, band):
        b1 = min(b0 + band, M) - 1
        rows.update((b0, b1))
        rows.update(int(r) for r in rng.integers(b0, b1 + 1, size=2))
    return np.array(sorted(rows))


@pytest.mark.parametrize("layer", [C5_LAYERS - 1, 0])
def test_config5_layer_matches_oracle(config5, layer):
    """The streamed Y, dX and dW of one layer's four Linears against the
    oracle (dnn/layers/fully_connected_layer.cu:29-35,54-59,78-83 on the
    dequantized codes): codes bit-exact; fp32 dW and the fp32 Y / dX of the
    same GEMMs (same codes, fp32 output) within 1e-4 on every 256-row band;
    the streamed bf16 Y and dX are the RNE image of those fp32 outputs."""
    stack, (Ys, dXs, dWs), dev_w = config5
    dev = stack.dev
    M = stack.M
    st = torch.cuda.current_stream().cuda_stream
    sc = stack.sc.cpu().numpy()
    sw = stack.sw.cpu().numpy()
    for i, (name, K, N) in enumerate(stack.linears):
        seed = stack.input_seed(i)
        # this layer's own inputs (seeded on the device; the bf16 bits are
        # the values every check below starts from)
        xb = _bits(stack.acts[layer][i])
        gb = _bits(stack.grads[layer][i])
        bb = synth.f32_to_bf16_bits(synth.normal((N,), 0.02, seed=seed + 2))
        wb = _bits(stack.weight_bf16(layer, i))
        s_x, s_dy, s_w = (orc.scale(orc.absmax(xb), orc.E4M3), orc.scale(orc.absmax(gb), orc.E5M2),
                          orc.scale(orc.absmax(wb), orc.E4M3))
        assert (sc[layer, i, 1], sc[layer, i, 3], sw[layer, i]) == \
            (np.float32(s_x), np.float32(s_dy), np.float32(s_w)), name
        cx, cdy, cw = orc.quantize(xb, s_x, orc.E4M3), orc.quantize(gb, s_dy, orc.E5M2), orc.quantize(wb, s_w, orc.E4M3)
        r16 = df.round16
        xq = stack.xq[layer][i]
        assert np.array_equal(xq.cpu().numpy()[:, :K], cx), f"X codes {name}"
        assert np.array_equal(stack.xt[layer][i].cpu().numpy()[:, :M], np.ascontiguousarray(cx.T)), f"X^T {name}"
        dyq = stack.dyq[layer][i]
        assert np.array_equal(dyq.cpu().numpy()[:, :N], cdy), f"dY codes {name}"
        assert np.array_equal(stack.dyt[layer][i].cpu().numpy()[:, :M], np.ascontiguousarray(cdy.T)), f"dY^T {name}"
        host = stack.host.numpy()
        fo = stack.host_offset(layer, 0) + stack.fwd_off[i]
        bo = stack.host_offset(layer, 1) + stack.bwd_off[i]
        assert np.array_equal(host[fo:fo + N * r16(K)].reshape(N, r16(K))[:, :K], cw), f"W codes {name}"
        assert np.array_equal(host[bo:bo + K * r16(N)].reshape(K, r16(N))[:, :N], np.ascontiguousarray(cw.T)), \
            f"W^T codes {name}"
        Xd = orc.dequantize(cx, s_x, orc.E4M3, "f32")
        dYd = orc.dequantize(cdy, s_dy, orc.E5M2, "f32")
        Wd = orc.dequantize(cw, s_w, orc.E4M3, "f32")
        idx = _band_rows(M, seed)
        # Y: fp32 output of the same forward GEMM on the same codes
        Y32 = torch.empty((M, N), dtype=torch.float32, device=dev)
        df.call("df_fp8_gemm_fwd", xq.data_ptr(), xq.stride(0),
                dev_w.data_ptr() + fo, r16(K), M, N, K, stack.sc_ptr(layer, i) + 4, stack.sw_ptr(layer, i),
                int(df.DType.BFLOAT16), stack.bias[i].data_ptr(), int(df.DType.FLOAT32), Y32.data_ptr(), N,
                stack.gws.data_ptr(), stack.gws.numel(), st)
        assert np.array_equal(_bits(Ys[layer][i]), synth.f32_to_bf16_bits(Y32.cpu().numpy())), f"Y bf16 {name}"
        ref = orc.fc_forward(Xd[idx], Wd, orc.bf16_to_f32(bb))
        err = orc.rel_err(Y32.cpu().numpy()[idx], ref)
        assert err <= 1e-4, f"layer {layer} {name} Y: {err:.3e}"
        # dX: fp32 output of the dX GEMM (the grouped launch's dX is the
        # separate call's, bit for bit)
        dX32 = torch.empty((M, K), dtype=torch.float32, device=dev)
        df.call("df_fp8_gemm_bwd_dx", dyq.data_ptr(), dyq.stride(0), dev_w.data_ptr() + bo,
                r16(N), M, N, K, stack.sc_ptr(layer, i) + 12, stack.sw_ptr(layer, i), int(df.DType.FLOAT32),
                dX32.data_ptr(), K, stack.gws.data_ptr(), stack.gws.numel(), st)
        assert np.array_equal(_bits(dXs[layer][i]), synth.f32_to_bf16_bits(dX32.cpu().numpy())), f"dX bf16 {name}"
        ref = orc.fc_backward_input(dYd[idx], Wd)
        err = orc.rel_err(dX32.cpu().numpy()[idx], ref)
        assert err <= 1e-4, f"layer {layer} {name} dX: {err:.3e}"
        # dW: rows and columns hitting every 256 x 256 tile
        o_idx, i_idx = _band_rows(N, seed + 9), _band_rows(K, seed + 8)
        refw = orc.fc_backward_weights(np.ascontiguousarray(dYd[:, o_idx]), np.ascontiguousarray(Xd[:, i_idx]))
        err = orc.rel_err(dWs[layer][i].cpu().numpy()[np.ix_(o_idx, i_idx)], refw)
        assert err <= 1e-4, f"layer {layer} {name} dW: {err:.3e}"
        # db from the same pass as the dY codes (fc_backward_bias, :91-106)
        assert orc.rel_err(stack.db[layer][i].cpu().numpy(), orc.fc_backward_bias(orc.bf16_to_f32(gb))) <= 1e-4
