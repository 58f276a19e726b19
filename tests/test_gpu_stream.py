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
