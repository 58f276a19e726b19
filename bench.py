#!/usr/bin/env python3
"""bench.py -- fp8 Linear path on one MI355X: fp8 Linear TFLOP/s and quantize GB/s
at GPT-2 XL shapes, as fractions of the fp8 MFMA and HBM rooflines.

Workload ("config 4"): the four GPT-2 XL Linears
(d = 1600: qkv 1600->4800, attn proj 1600->1600, fc 1600->6400, proj
6400->1600) at M = 16384 tokens, forward and backward, on seeded synthetic
bf16 tensors already resident in HBM.  One step: absmax + quantize of the
four weights W -> e4m3 (both copies) in one df_quantize_2d_batch call
(--per-linear-weights: per Linear, in its forward), then per Linear:
  forward : absmax + quantize X -> e4m3 (row copy and transposed copy),
            Y = Xq . Wq^T * sx * sw + b            (bf16 out, fused bias)
  backward: absmax + quantize dY -> e5m2 (both copies) with db = column
            sums fused into the same pass,
            dX = dYq . W * sdy * sw                  (bf16 out)
            dW = dYq^T . X * sdy * sx                (fp32 out, overwrite)
            in one grouped launch (--separate-backward: two launches)
value = GEMM flops of the step (2*M*N*K per GEMM, 12 GEMMs) / step time.

Also reported on the same JSON line:
  roofline     -- the dominant kernel (largest summed time) against fp8 MFMA
                  peak; its average duration comes from a second pass of the
                  same steps with HIP events around every C-ABI call, on the
                  stream the kernels run on.
The timed region (value, ms_per_step) is K steps replayed from a HIP graph
captured once from the same launches (--no-graph: eager launches), with one
HIP-event pair around the K steps.
  quantize     -- the step's absmax/quantize/colsum kernels against HBM peak.
  conversion   -- config 2 standalone kernels (n = 2^28, fp32 and bf16 in,
                  e4m3 and e5m2) against HBM peak.
  streaming    -- config 5: the 48-layer GPT-2 XL Linear stack, fwd+bwd at
                  8192 tokens, e4m3 weights streamed from pinned host memory
                  per layer (see streaming_bench).
  cpu_baseline -- the oracle's restatement of the reference's FC loops
                  (dnn/layers/fully_connected_layer.cu:29-35,54-59,78-83) on a
                  token slice of the same workload, timed on this host.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
M_TOKENS = 16384
SINGLE_KERNEL_FAMILIES = ("gemm_fwd", "gemm_bwd", "gemm_dx")
XL_LINEARS = [("qkv", 1600, 4800), ("attn_proj", 1600, 1600), ("fc", 1600, 6400), ("proj", 6400, 1600)]
SMALL_LINEARS = [("qkv", 768, 2304), ("attn_proj", 768, 768), ("fc", 768, 3072), ("proj", 3072, 768)]


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-conversion", action="store_true")
    p.add_argument("--no-streaming", action="store_true", help="skip the config 5 layer-streaming leg")
    p.add_argument("--no-optimizer", action="store_true", help="skip the clip + Adam leg")
    p.add_argument("--no-delayed", action="store_true", help="skip the delayed-scaling step leg")
    p.add_argument("--no-producer", action="store_true", help="skip the LayerNorm + quantize leg")
    p.add_argument("--no-config3", action="store_true", help="skip the GPT-2 small forward leg (config 3)")
    p.add_argument("--per-linear-weights", action="store_true",
                   help="quantize each weight in its own calls instead of one df_quantize_2d_batch per step")
    p.add_argument("--separate-absmax", action="store_true",
                   help="absmax pass and 2-D quantize as two calls (df_absmax_scale_bf16, df_quantize_2d*) "
                        "instead of df_quantize_2d_jit")
    p.add_argument("--separate-backward", action="store_true",
                   help="time the backward as separate dX and dW launches instead of df_fp8_gemm_bwd")
    p.add_argument("--vendor-compare", action="store_true",
                   help="also time the 12 GEMM shapes on torch._scaled_mm (hipBLASLt) for comparison")
    p.add_argument("--history", type=int, default=16, help="amax history length of the delayed-scaling leg")
    p.add_argument("--stream-layers", type=int, default=48)
    p.add_argument("--stream-slots", type=int, default=6,
                   help="device weight slots of the streaming leg (>= 3: loads run slots-2 layers ahead)")
    p.add_argument("--cpu-tokens", type=int, default=512,
                   help="token slice of configs 3 and 4 for the CPU baseline (all cores; one core: a 1/8 slice)")
    p.add_argument("--no-graph", action="store_true", help="time eager launches instead of a HIP graph")
    p.add_argument("--copy-calibration", action="store_true",
                   help="first run one plain 1 GiB device copy (HBM counter calibration under rocprofv3 --pmc)")
    p.add_argument("--conversion-only", action="store_true",
                   help="run only the config-2 conversion leg and print its JSON (profiling runs)")
    p.add_argument("--config3-only", action="store_true",
                   help="run only the config-3 leg and print its JSON (profiling runs)")
    p.add_argument("--config5-compute-only", action="store_true",
                   help="run only config 5's step once with every layer's weights resident (the streamed step's "
                        "kernels, no copies) and print its JSON; for the config-5 MFMA counter run")
    p.add_argument("--tile-timeline", action="store_true",
                   help="run only the per-tile timeline of the four config-4 forward GEMMs and print its JSON")
    p.add_argument("--summarize-profiles", action="store_true",
                   help="no GPU work: turn the rocprofv3 output of PROFILE_COMMANDS into the summaries under "
                        "profiles/")
    return p.parse_args()


class Timer:
    """HIP events around launches on the current stream, grouped by name."""

    def __init__(self, torch, enabled=True):
        self.torch = torch
        self.enabled = enabled
        self.pending = []

    def run(self, name, fn, *a, **k):
        t = self.torch
        if not self.enabled:
            return fn(*a, **k)
        e0 = t.cuda.Event(enable_timing=True)
        e1 = t.cuda.Event(enable_timing=True)
        e0.record()
        r = fn(*a, **k)
        e1.record()
        self.pending.append((name, e0, e1))
        return r

    def collect(self):
        self.torch.cuda.synchronize()
        out = {}
        for name, e0, e1 in self.pending:
            ms = e0.elapsed_time(e1)
            tot, cnt = out.get(name, (0.0, 0))
            out[name] = (tot + ms, cnt + 1)
        self.pending = []
        return out


def main():
    args = parse()
    if args.summarize_profiles:
        summarize_profiles()
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding of this path is designed, not built)", file=sys.stderr)
        sys.exit(2)
    if args.stream_slots < 3:
        print("bench.py: --stream-slots must be at least 3", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import deepfuse_amd as df
    from deepfuse_amd import DType, Fmt, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = df.lib()
    if L.df_device_arch_ok() != 1:
        raise RuntimeError("device is not gfx950")
    M = M_TOKENS
    if args.copy_calibration:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # reads and writes 1 GiB
        torch.cuda.synchronize()
        del src, dst

    def cur():  # the stream kernels go to (the capture stream while capturing)
        return torch.cuda.current_stream().cuda_stream

    if args.conversion_only:
        print(json.dumps({"conversion": conversion_bench(torch, df, synth, dev, cur())}))
        return
    if args.config3_only:
        print(json.dumps({"config3": config3_bench(torch, df, synth, dev, cur(), vendor=args.vendor_compare)}))
        return
    if args.tile_timeline:
        print(json.dumps({"tile_timeline": tile_timeline_bench(torch, df, dev, cur())}))
        return
    if args.config5_compute_only:
        print(json.dumps({"config5_compute": config5_compute_bench(torch, dev, layers=args.stream_layers)}))
        return

    def to_bf16(a):
        return torch.from_numpy(synth.f32_to_bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)

    ws = torch.empty(L.df_absmax_workspace_bytes(), dtype=torch.uint8, device=dev)
    gws_bytes = max(L.df_fp8_gemm_workspace_bytes(M, n, k) for _, k, n in XL_LINEARS)
    gws_bytes = max(gws_bytes, max(L.df_fp8_gemm_workspace_bytes(n, k, M) for _, k, n in XL_LINEARS))
    gws_bytes = max(gws_bytes, max(L.df_fp8_gemm_bwd_workspace_bytes(M, n, k) for _, k, n in XL_LINEARS))
    gws = torch.empty(gws_bytes, dtype=torch.uint8, device=dev)
    cws = torch.empty(max(L.df_quantize_2d_workspace_bytes(M, n) for _, _, n in XL_LINEARS), dtype=torch.uint8,
                      device=dev)
    layers = []
    for i, (name, K, N) in enumerate(XL_LINEARS):
        seed = synth.SEED_BASE + 4 + 10 * i
        Kp, Mp, Np = df.round16(K), df.round16(M), df.round16(N)
        lay = dict(name=name, K=K, N=N,
                   X=to_bf16(synth.normal((M, K), 1.0, seed=seed)),
                   W=to_bf16(synth.normal((N, K), 0.02, seed=seed + 1)),
                   b=to_bf16(synth.normal((N,), 0.02, seed=seed + 2)),
                   dY=to_bf16(synth.normal((M, N), 1e-3, seed=seed + 3)),
                   Xq=torch.empty((M, Kp), dtype=torch.uint8, device=dev),
                   Xt=torch.empty((K, Mp), dtype=torch.uint8, device=dev),
                   Wq=torch.empty((N, Kp), dtype=torch.uint8, device=dev),
                   Wt=torch.empty((K, Np), dtype=torch.uint8, device=dev),
                   dYq=torch.empty((M, Np), dtype=torch.uint8, device=dev),
                   dYt=torch.empty((N, Mp), dtype=torch.uint8, device=dev),
                   Y=torch.empty((M, N), dtype=torch.bfloat16, device=dev),
                   dX=torch.empty((M, K), dtype=torch.bfloat16, device=dev),
                   dW=torch.empty((N, K), dtype=torch.float32, device=dev),
                   db=torch.empty((N,), dtype=torch.float32, device=dev),
                   sc=torch.empty(6, dtype=torch.float32, device=dev))
        layers.append(lay)
    torch.cuda.synchronize()

    BF, F32 = int(DType.BFLOAT16), int(DType.FLOAT32)
    E4, E5 = int(Fmt.E4M3), int(Fmt.E5M2)

    jws_bytes = max(L.df_quantize_2d_jit_workspace_bytes(M, n, 1) for _, _, n in XL_LINEARS)
    jws = torch.empty(jws_bytes, dtype=torch.uint8, device=dev)

    def quant(tm, x, rows, cols, fmt, am, sc, q, qt, tag, db=None):
        if not args.separate_absmax:  # absmax and codes in one call (df_quantize_2d_jit)
            tm.run("quantize2d_" + tag, df.call, "df_quantize_2d_jit", BF, x.data_ptr(), rows, cols, fmt, am, sc,
                   q.data_ptr(), q.stride(0), qt.data_ptr(), qt.stride(0), None if db is None else db.data_ptr(),
                   jws.data_ptr(), jws_bytes, cur())
            return
        tm.run("absmax_" + tag, df.call, "df_absmax_scale_bf16", x.data_ptr(), x.numel(), fmt, am, sc,
               ws.data_ptr(), ws.numel(), cur())
        if db is None:
            tm.run("quantize2d_" + tag, df.call, "df_quantize_2d", BF, x.data_ptr(), rows, cols, cols, fmt, sc,
                   q.data_ptr(), q.stride(0), qt.data_ptr(), qt.stride(0), cur())
        else:
            tm.run("quantize2d_" + tag, df.call, "df_quantize_2d_colsum", BF, x.data_ptr(), rows, cols, cols, fmt,
                   sc, q.data_ptr(), q.stride(0), qt.data_ptr(), qt.stride(0), db.data_ptr(), cws.data_ptr(),
                   cws.numel(), cur())

    # all four weights in one df_quantize_2d_batch call (three launches)
    nl = len(layers)
    w_am = torch.empty(nl, dtype=torch.float32, device=dev)
    w_sc = torch.empty(nl, dtype=torch.float32, device=dev)
    qb_ws = torch.empty(L.df_quantize_2d_batch_workspace_bytes(), dtype=torch.uint8, device=dev)
    iarr = lambda vals: (ctypes.c_int * nl)(*vals)
    parr = lambda ts: (ctypes.c_void_p * nl)(*[t.data_ptr() for t in ts])
    qb_args = (parr([l["W"] for l in layers]), iarr([l["N"] for l in layers]), iarr([l["K"] for l in layers]),
               E4, w_am.data_ptr(), w_sc.data_ptr(), parr([l["Wq"] for l in layers]),
               iarr([l["Wq"].stride(0) for l in layers]), parr([l["Wt"] for l in layers]),
               iarr([l["Wt"].stride(0) for l in layers]), qb_ws.data_ptr(), qb_ws.numel())

    # The grouped backward of a Linear is one kernel launch when its plan
    # keeps dW unsplit (family gemm_bwd) and two when dW runs in K slices
    # (the persistent kernel + the ordered slice reduce: gemm_bwd_split).
    bwd_family = []
    for l in layers:
        g_, s_ = ctypes.c_int(), ctypes.c_int()
        df.call("df_fp8_gemm_bwd_plan", M, l["N"], l["K"], gws_bytes, ctypes.byref(g_), ctypes.byref(s_))
        bwd_family.append("gemm_bwd" if g_.value and s_.value == 1 else
                          "gemm_bwd_split" if g_.value else "gemm_bwd_separate")

    def step(tm, grouped=not args.separate_backward):
        if not args.per_linear_weights:
            tm.run("weights_batch", df.call, "df_quantize_2d_batch", BF, nl, *qb_args, cur())
        for i, l in enumerate(layers):
            K, N = l["K"], l["N"]
            s = l["sc"].data_ptr()
            sx_am, sx, sw_am, sw, sdy_am, sdy = (s + 4 * j for j in range(6))
            quant(tm, l["X"], M, K, E4, sx_am, sx, l["Xq"], l["Xt"], "act")
            if args.per_linear_weights:
                quant(tm, l["W"], N, K, E4, sw_am, sw, l["Wq"], l["Wt"], "weight")
            else:
                sw = w_sc.data_ptr() + 4 * i
            tm.run("gemm_fwd", df.call, "df_fp8_gemm_fwd", l["Xq"].data_ptr(), l["Xq"].stride(0),
                   l["Wq"].data_ptr(), l["Wq"].stride(0), M, N, K, sx, sw, BF, l["b"].data_ptr(), BF,
                   l["Y"].data_ptr(), N, gws.data_ptr(), gws_bytes, cur())
            quant(tm, l["dY"], M, N, E5, sdy_am, sdy, l["dYq"], l["dYt"], "grad", db=l["db"])
            if grouped:
                # dX and dW in one launch (df_fp8_gemm_bwd)
                tm.run(bwd_family[i], df.call, "df_fp8_gemm_bwd", l["dYq"].data_ptr(), l["dYq"].stride(0),
                       l["Wt"].data_ptr(), l["Wt"].stride(0), l["dYt"].data_ptr(), l["dYt"].stride(0),
                       l["Xt"].data_ptr(), l["Xt"].stride(0), M, N, K, sdy, sw, sx, BF, l["dX"].data_ptr(), K,
                       F32, l["dW"].data_ptr(), K, gws.data_ptr(), gws_bytes, cur())
                continue
            tm.run("gemm_dx", df.call, "df_fp8_gemm_bwd_dx", l["dYq"].data_ptr(), l["dYq"].stride(0),
                   l["Wt"].data_ptr(), l["Wt"].stride(0), M, N, K, sdy, sw, BF, l["dX"].data_ptr(), K,
                   gws.data_ptr(), gws_bytes, cur())
            tm.run("gemm_dw", df.call, "df_fp8_gemm_bwd_dw", l["dYt"].data_ptr(), l["dYt"].stride(0),
                   l["Xt"].data_ptr(), l["Xt"].stride(0), M, N, K, sdy, sx, F32, l["dW"].data_ptr(), K,
                   gws.data_ptr(), gws_bytes, cur())

    # algorithmic work per step: 2*M*N*K per GEMM on unpadded shapes
    gemm_flops = {}
    qbytes = {}
    for i, (_, K, N) in enumerate(XL_LINEARS):
        f = 2 * M * N * K
        fams = ("gemm_fwd", "gemm_dx", "gemm_dw") if args.separate_backward else ("gemm_fwd", bwd_family[i])
        for k in fams:
            gemm_flops[k] = gemm_flops.get(k, 0) + (f if k in ("gemm_fwd", "gemm_dx", "gemm_dw") else 2 * f)
        for tag, r, c in (("act", M, K), ("weight", N, K), ("grad", M, N)):
            if tag == "weight" and not args.per_linear_weights:
                # absmax read + quantize read + both code layouts written
                qbytes["weights_batch"] = qbytes.get("weights_batch", 0) + 2 * r * c + 2 * r * c + 2 * r * c
                continue
            # absmax read (2 bytes per value) + quantize read + both code layouts written
            absmax_fam = "absmax_" + tag if args.separate_absmax else "quantize2d_" + tag
            qbytes[absmax_fam] = qbytes.get(absmax_fam, 0) + 2 * r * c
            qbytes["quantize2d_" + tag] = qbytes.get("quantize2d_" + tag, 0) + 2 * r * c + 2 * r * c

    step_flops = sum(gemm_flops.values())

    null = Timer(torch, enabled=False)
    for _ in range(args.warmup):
        step(null)
    torch.cuda.synchronize()

    # Timed region: K steps, one HIP-event pair around all of them.  By
    # default the step is captured once as a HIP graph (the same kernel
    # launches, replayed without host launch gaps).
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(null)
        # the warm-up steps again, replayed like the timed ones (the first
        # replays after capture run a few percent slower)
        for _ in range(max(1, args.warmup)):
            graph.replay()
        torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step(null)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    elapsed = max(e0.elapsed_time(e1) / 1e3, 1e-9)
    ms_per_step = 1e3 * elapsed / args.steps
    value = step_flops / (elapsed / args.steps) / 1e12

    # Outside the timed region: the same step with the backward as the two
    # separate dX and dW launches, for comparison.
    separate = None
    if not args.separate_backward:
        g2 = None
        if not args.no_graph:
            g2 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g2):
                step(null, grouped=False)
        run_sep = g2.replay if g2 is not None else (lambda: step(null, grouped=False))
        run_grp = graph.replay if graph is not None else (lambda: step(null))
        run_sep()
        torch.cuda.synchronize()

        def avg_ms(fn):
            s0 = torch.cuda.Event(enable_timing=True)
            s1 = torch.cuda.Event(enable_timing=True)
            s0.record()
            for _ in range(args.steps):
                fn()
            s1.record()
            torch.cuda.synchronize()
            return s0.elapsed_time(s1) / args.steps

        # alternate the two, three times each; best of each
        sep_t, grp_t = [], []
        for _ in range(3):
            sep_t.append(avg_ms(run_sep))
            grp_t.append(avg_ms(run_grp))
        sep_ms, grp_ms = min(sep_t), min(grp_t)
        separate = {"ms_per_step": round(sep_ms, 4), "tflops": round(step_flops / (sep_ms * 1e-3) / 1e12, 2),
                    "grouped_ms_per_step": round(grp_ms, 4), "grouped_speedup": round(sep_ms / grp_ms, 4),
                    "note": "best of 3 alternating runs of the two step variants, after the timed region"}
        del g2

    # Per-kernel durations: the same step launched eagerly with a HIP-event
    # pair around every C-ABI call, over as many steps as the timed region.
    tm = Timer(torch)
    for _ in range(args.steps):
        step(tm)
    per = tm.collect()

    # dominant kernel = the largest summed time among the families whose
    # C-ABI call is exactly one kernel launch: gemm_fwd (the persistent
    # kernel, e4m3 x e4m3 -> bf16 + bias), gemm_bwd (the grouped dX + dW
    # persistent launch of the Linears whose dW stays unsplit) and, under
    # --separate-backward, gemm_dx.  gemm_bwd_split and gemm_dw are several
    # kernels (K-slice partial tiles + their ordered reduction) and each
    # quantize family two or three (absmax passes, 2-D quantize, column-sum
    # fold); they are reported in `kernels` but a per-launch roofline needs
    # one kernel.
    dom = max((k for k in SINGLE_KERNEL_FAMILIES if k in per), key=lambda k: per[k][0])
    tot_ms, cnt = per[dom]
    avg_ms = tot_ms / cnt
    if dom in gemm_flops:
        work_per_launch = gemm_flops[dom] * args.steps / cnt
        achieved = work_per_launch / (avg_ms * 1e-3) / 1e12
        roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": FP8_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / FP8_PEAK_TFLOPS, 4), "traffic": None,
                "avg_launch_ms": round(avg_ms, 4), "work_per_launch": work_per_launch}
    else:
        work_per_launch = qbytes[dom] * args.steps / cnt
        achieved = work_per_launch / (avg_ms * 1e-3) / 1e9
        roof = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "avg_launch_ms": round(avg_ms, 4), "work_per_launch": work_per_launch}
    roof["traffic"], roof["traffic_source"] = measured_traffic(roof["kernel"])
    kernels = {}
    for k, (t, c) in sorted(per.items()):
        d = {"ms_per_step": round(t / args.steps, 4), "launches_per_step": c // args.steps}
        if k in gemm_flops:
            d["tflops"] = round(gemm_flops[k] / (t / args.steps * 1e-3) / 1e12, 1)
        else:
            d["gbs"] = round(qbytes[k] / (t / args.steps * 1e-3) / 1e9, 1)
        kernels[k] = d
    weights_batch = None if args.per_linear_weights else (
        lambda: df.call("df_quantize_2d_batch", BF, nl, *qb_args, cur()))
    delayed = None if args.no_delayed else delayed_scaling_leg(torch, df, layers, M, args, cur, ws, gws, gws_bytes,
                                                                    ms_per_step, step_flops, weights_batch, w_sc)
    qt_ms = sum(per[k][0] for k in qbytes) / args.steps
    q_gbs = sum(qbytes.values()) / (qt_ms * 1e-3) / 1e9
    gemm_ms = sum(per[k][0] for k in gemm_flops) / args.steps
    gemm_tflops = step_flops / (gemm_ms * 1e-3) / 1e12

    out = {
        "metric": "fp8 Linear TFLOP/s + quantize GB/s at GPT-2 XL shapes, % of roofline",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8 e4m3/e5m2 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, N(0,1e-3) grads; bf16)",
        "timing": {"region": "hip_graph" if graph is not None else "eager", "wall_s": round(wall, 4)},
        "config": {"workload": "config 4: GPT-2 XL Linears (d=1600) fwd+bwd, M=16384 tokens",
                   "linears": [f"{n} {k}->{o}" for n, k, o in XL_LINEARS], "tokens": M,
                   "step_gemm_flops": step_flops},
        "frac_of_fp8_peak": round(value / FP8_PEAK_TFLOPS, 4),
        "gemm_only": {"tflops": round(gemm_tflops, 1), "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
                      "ms_per_step": round(gemm_ms, 4)},
        "quantize": {"gbs": round(q_gbs, 1), "frac": round(q_gbs / HBM_PEAK_GBS, 4),
                     "ms_per_step": round(qt_ms, 4)},
        "roofline": roof,
        "kernels": kernels,
    }
    if separate is not None:
        out["backward_separate_launches"] = separate
    if delayed is not None:
        out["delayed_scaling"] = delayed
    if not args.no_conversion:
        out["conversion"] = conversion_bench(torch, df, synth, dev, cur())
    if args.vendor_compare:
        out["vendor_compare"] = vendor_bench(torch, df, dev, cur())
    if not args.no_config3:
        out["config3"] = config3_bench(torch, df, synth, dev, cur(), vendor=args.vendor_compare)
    if not args.no_producer:
        out["producer"] = producer_bench(torch, df, synth, dev, cur())
    if not args.no_optimizer:
        out["optimizer"] = optimizer_bench(torch, df, dev, cur(), layers=args.stream_layers)
    if not args.no_streaming:
        out["streaming"] = streaming_bench(torch, df, synth, dev, layers=args.stream_layers,
                                           slots=args.stream_slots)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_tokens)
    print(json.dumps(out))


def measured_traffic(kernel_family):
    """HBM bytes per launch of a kernel family from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (profiles/hbm_traffic.json, written from
    those runs with the copy-kernel scale factor applied), and where that
    figure comes from (the file, the tree the runs measured, their
    commands); (None, None) without it.  rocprofv3 cannot count inside the
    process it measures, so the figure is as fresh as the last profile
    run."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as fh:
            data = json.load(fh)
        fam = data["families"][kernel_family]
        src = {"file": "profiles/hbm_traffic.json", "tree": data.get("tree"), "kernel": fam["kernel"],
               "commands": [data["command_fetch"], data["command_write"]]}
        return fam["bytes_per_launch"], src
    except (OSError, KeyError, ValueError):
        return None, None


# The profiling runs behind profiles/ (from the repository root on one
# MI355X, with TMPDIR=/tmp), and the directories they write.
PROFILE_COMMANDS = {
    "stats": ("rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_bench -o bench -- "
              "python3 bench.py --steps 20 --warmup 3 --no-cpu-baseline --no-conversion --no-streaming "
              "--no-optimizer --no-producer --no-delayed --no-config3 > gpurun_out/prof_bench_line.json"),
    "fetch": ("timeout -s KILL 180 rocprofv3 --pmc FETCH_SIZE --kernel-trace --output-format csv "
              "-d gpurun_out/pmc_fetch -o bench -- python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline "
              "--no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph "
              "--copy-calibration"),
    "write": ("timeout -s KILL 180 rocprofv3 --pmc WRITE_SIZE --kernel-trace --output-format csv "
              "-d gpurun_out/pmc_write -o bench -- python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline "
              "--no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph "
              "--copy-calibration"),
    "stats_conversion": ("rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_conversion -o bench "
                         "-- python3 bench.py --conversion-only"),
    "fetch_conversion": ("timeout -s KILL 180 rocprofv3 --pmc FETCH_SIZE --kernel-trace --output-format csv "
                         "-d gpurun_out/pmc_fetch_conv -o bench -- python3 bench.py --conversion-only --copy-calibration"),
    "write_conversion": ("timeout -s KILL 180 rocprofv3 --pmc WRITE_SIZE --kernel-trace --output-format csv "
                         "-d gpurun_out/pmc_write_conv -o bench -- python3 bench.py --conversion-only --copy-calibration"),
    "mfma": ("timeout -s KILL 180 rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_BUSY_CYCLES "
             "SQ_INSTS_VALU_MFMA_MOPS_F8 --kernel-trace --output-format csv -d gpurun_out/pmc_mfma -o bench -- "
             "python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming --no-optimizer "
             "--no-producer --no-delayed --no-config3 --no-graph"),
    "mfma_config3": ("timeout -s KILL 180 rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_BUSY_CYCLES "
                     "SQ_INSTS_VALU_MFMA_MOPS_F8 --kernel-trace --output-format csv -d gpurun_out/pmc_mfma_config3 "
                     "-o bench -- python3 bench.py --config3-only"),
    "mfma_config5": ("timeout -s KILL 300 rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_BUSY_CYCLES "
                     "SQ_INSTS_VALU_MFMA_MOPS_F8 --kernel-trace --output-format csv -d gpurun_out/pmc_mfma_config5 "
                     "-o bench -- python3 bench.py --config5-compute-only"),
    "stats_consumer": ("rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_consumer -o bench "
                       "-- python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming "
                       "--no-producer --no-delayed --no-config3"),
    "streaming": ("python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-conversion --no-optimizer "
                  "--no-producer --no-delayed --no-config3"),
    "timeline": "python3 bench.py --tile-timeline",
    "pmc_sq1": ("timeout -s KILL 180 rocprofv3 --pmc SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS SQ_VALU_MFMA_BUSY_CYCLES --kernel-trace --output-format csv "
                "-d gpurun_out/pmc_sq1 -o bench -- python3 bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph"),
    "pmc_sq2": ("timeout -s KILL 180 rocprofv3 --pmc SQ_VMEM_TA_ADDR_FIFO_FULL SQ_VMEM_TA_CMD_FIFO_FULL SQ_LDS_BANK_CONFLICT SQ_LDS_DATA_FIFO_FULL SQ_INSTS_LDS SQ_WAIT_INST_LDS SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR --kernel-trace --output-format csv "
                "-d gpurun_out/pmc_sq2 -o bench -- python3 bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph"),
    "pmc_tatd": ("timeout -s KILL 180 rocprofv3 --pmc TA_TA_BUSY_sum TA_ADDR_STALLED_BY_TC_CYCLES_sum TD_TD_BUSY_sum TD_TC_STALL_sum GRBM_GUI_ACTIVE GRBM_COUNT --kernel-trace --output-format csv "
                "-d gpurun_out/pmc_tatd -o bench -- python3 bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph"),
    "pmc_tcp": ("timeout -s KILL 180 rocprofv3 --pmc TCP_PENDING_STALL_CYCLES_sum TCP_TCC_READ_REQ_LATENCY_sum TCP_TCC_READ_REQ_sum TCP_UTCL1_TRANSLATION_MISS_sum TCC_HIT_sum TCC_MISS_sum --kernel-trace --output-format csv "
                "-d gpurun_out/pmc_tcp -o bench -- python3 bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph"),
    "pmc_ea": ("timeout -s KILL 180 rocprofv3 --pmc TCC_EA0_WRREQ_sum TCC_EA0_RDREQ_sum TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum --kernel-trace --output-format csv "
                "-d gpurun_out/pmc_ea -o bench -- python3 bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming --no-optimizer --no-producer --no-delayed --no-config3 --no-graph"),
    "stats_producer": ("rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_producer -o bench "
                       "-- python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-conversion --no-streaming "
                       "--no-optimizer --no-delayed --no-config3"),
    "stats_config3": ("rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_config3 -o bench "
                      "-- python3 bench.py --config3-only"),
}
# extra kernel-stat summaries: (command key, csv directory, output file, title,
# substrings that select the leg's own kernels)
EXTRA_STATS = (
    ("stats_consumer", "prof_consumer", "consumer_clip_adam_kernel_stats.md",
     "clip + Adam over GPT-2 XL's 48 x 4 Linears (1.475 G fp32 parameters)",
     ("adam_kernel", "sumsq_kernel", "clip_kernel", "norm_finalize_kernel")),
    ("stats_producer", "prof_producer", "layernorm_quantize_kernel_stats.md",
     "LayerNorm + e4m3 codes, 16384 x 1600 bf16 (unfused chain, fused, fused delayed)",
     ("ln_stats_kernel", "true>(unsigned short const*", "amax_history_kernel")),
    ("stats_producer", "prof_producer", "gemm_producer_kernel_stats.md",
     "GEMMs that also fold their output's absmax: fc1's forward and fc2's grouped backward at the config-4 fc "
     "shapes (the producer leg's gemm_producer variants)",
     ("persistent_amax_kernel", "grouped_amax_kernel")),
)
# GEMM families whose C-ABI call is exactly one kernel, by the persistent
# kernel's template arguments: <A format, B format, output, bias type, bias,
# K-split>.
TRAFFIC_FAMILIES = {
    "gemm_fwd": ("gemm_nt_persistent_kernel<0, 0, unsigned short, unsigned short, true, false, void>",),
    "gemm_bwd": ("gemm_nt_persistent_kernel<1, 0, float, float, false, false, unsigned short>",),
    "gemm_dx": ("gemm_nt_persistent_kernel<1, 0, unsigned short, float, false, false, void>",),
}


def _tree_id():
    """The git commit of this tree, with -dirty when files outside profiles/
    (the summaries being written) differ from it; recorded beside profile
    summaries.  None outside a git checkout."""
    import subprocess

    root = os.path.dirname(os.path.abspath(__file__))
    try:
        head = subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], capture_output=True, text=True, cwd=root,
                              timeout=20).stdout.strip()
        if not head:
            return None
        st = subprocess.run(["git", "status", "--porcelain", "--untracked-files=no", "--", ".", ":(exclude)profiles"],
                            capture_output=True, text=True, cwd=root, timeout=20).stdout.strip()
        return head + ("-dirty" if st else "")
    except (OSError, subprocess.SubprocessError):
        return None


def _short_kernel(name):
    """Kernel name without its parameter list."""
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def line_kernel_check(out_dir):
    """Lines comparing, within the stats run, the bench line's per-launch
    time of its dominant kernel (HIP events in the eager per-kernel pass)
    with rocprof's durations of the same dispatches: that pass is the last
    use of the kernel in the run, so they are the kernel's last
    steps x launches_per_step dispatches in the trace.  [] when the run's
    line or trace is missing."""
    import csv

    line_path = os.path.join(out_dir, "prof_bench_line.json")
    trace = os.path.join(out_dir, "prof_bench", "bench_kernel_trace.csv")
    if not (os.path.exists(line_path) and os.path.exists(trace)):
        return []
    with open(line_path) as fh:
        lines = [ln for ln in fh.read().splitlines() if ln.strip().startswith("{")]
    if not lines:
        return []
    d = json.loads(lines[-1])
    roof = d["roofline"]
    dom = roof["kernel"]
    pats = TRAFFIC_FAMILIES.get(dom)
    if not pats:
        return []
    n = d["steps"] * d["kernels"][dom]["launches_per_step"]
    with open(trace) as fh:
        disp = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in csv.DictReader(fh)
                if any(_short_kernel(r["Kernel_Name"]).endswith(p) for p in pats)]
    disp.sort()
    last = disp[-n:]
    if len(last) < n or n == 0:
        return []
    prof_ms = sum(e - b for b, e in last) / n / 1e6
    ev_ms = roof["avg_launch_ms"]
    work = roof["work_per_launch"]
    peak = roof["peak"]
    f_ev, f_pr = work / (ev_ms * 1e-3) / 1e12 / peak, work / (prof_ms * 1e-3) / 1e12 / peak
    return ["", "## The bench line's dominant kernel, within this run", "",
            f"The run's own JSON line (stdout, kept as `gpurun_out/prof_bench_line.json`) names `{dom}` "
            f"(`{pats[0]}`) with `roofline.avg_launch_ms` = {ev_ms:.4f}: HIP events around each of its {n} "
            "launches in the eager per-kernel pass.  Those launches are the kernel's last "
            f"{n} dispatches in this run's kernel trace.", "",
            "| source | ms per launch | TFLOP/s | fraction of 5.0 PF |", "|---|---|---|---|",
            f"| HIP events (the line) | {ev_ms:.4f} | {work / (ev_ms * 1e-3) / 1e12:.1f} | {f_ev:.4f} |",
            f"| rocprof, same {n} dispatches | {prof_ms:.4f} | {work / (prof_ms * 1e-3) / 1e12:.1f} | "
            f"{f_pr:.4f} |", "",
            f"They differ by {abs(prof_ms / ev_ms - 1) * 100:.1f}%.  The table above averages every dispatch of the "
            "run (graph replays, the separate-launch comparison and the per-kernel pass); between boxes the "
            "same kernels vary by about 4%, with the shader clock they hold."]


def config4_stats_summary(out_dir, prof):
    """profiles/bench_config4_kernel_stats.md from the stats run (and the
    bench line it printed)."""
    import csv

    stats_csv = os.path.join(out_dir, "prof_bench", "bench_kernel_stats.csv")
    with open(stats_csv) as fh:
        rows = list(csv.DictReader(fh))
    lines = ["# rocprofv3 kernel statistics -- bench.py, config 4 (GPT-2 XL Linears fwd+bwd, M=16384)", "",
             "Command (from the repository root, on one MI355X):", "", "    " + PROFILE_COMMANDS["stats"], "",
             "Steps, in order: 3 eager warm-up steps, the HIP-graph capture, 3 warm-up replays, 20 timed "
             "replays (the timed region); then, for comparison, three alternations of 20 replays of the step with "
             "separate dX and dW launches and 20 of the grouped step; then 20 eager steps with HIP events (the "
             "per-kernel pass).  The grouped dX + dW launch is the persistent kernel whose last template argument "
             "is the dX output type (`unsigned short`); `void` marks single-GEMM launches.  Durations in "
             "microseconds.", "",
             "| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in rows:
        lines.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    lines += line_kernel_check(out_dir)
    with open(os.path.join(prof, "bench_config4_kernel_stats.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return rows


def config4_traffic_summary(out_dir, prof):
    """profiles/hbm_traffic_config4.md and hbm_traffic.json from the fetch
    and write runs."""
    import csv

    def counters(which, counter):
        path = os.path.join(out_dir, "pmc_" + which, "bench_counter_collection.csv")
        vals = {}
        with open(path) as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] == counter:
                    vals.setdefault(_short_kernel(r["Kernel_Name"]), []).append(float(r["Counter_Value"]))
        return vals

    fetch_all = counters("fetch", "FETCH_SIZE")
    write_all = counters("write", "WRITE_SIZE")
    copy = "__amd_rocclr_copyBuffer"
    # calibration: the largest copy dispatch is the 1 GiB device-to-device
    # copy (--copy-calibration); it reads and writes exactly 2^30 bytes
    copy_f, copy_w = max(fetch_all.pop(copy)), max(write_all.pop(copy))
    fscale = (1 << 30) / (copy_f * 1024)
    wscale = (1 << 30) / (copy_w * 1024)
    fetch = {k: (sum(v) / len(v), len(v)) for k, v in fetch_all.items()}
    write = {k: (sum(v) / len(v), len(v)) for k, v in write_all.items()}
    fams = {}
    for fam, pats in TRAFFIC_FAMILIES.items():
        names = [k for k in fetch if k.startswith("void dfk::") and any(k.endswith(p) for p in pats)]
        if len(names) != 1 or names[0] not in write:
            continue
        k = names[0]
        fams[fam] = {"kernel": k, "bytes_per_launch": int(round(fetch[k][0] * 1024 * fscale + write[k][0] * 1024 * wscale)),
                     "fetch_KiB": fetch[k][0], "write_KiB": write[k][0]}
    data = {"tree": _tree_id(), "command_fetch": PROFILE_COMMANDS["fetch"], "command_write": PROFILE_COMMANDS["write"],
            "calibration": {"kernel": copy, "bytes": 1 << 30, "fetch_KiB": copy_f, "write_KiB": copy_w,
                            "fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4)},
            "families": fams}
    # the tree id names the code the counters were read on: summarizing the
    # same counter output again later keeps the id it was first written with
    try:
        with open(os.path.join(prof, "hbm_traffic.json")) as fh:
            old = json.load(fh)
        if old.get("families") == fams and old.get("calibration") == data["calibration"]:
            data["tree"] = old.get("tree")
    except (OSError, ValueError):
        pass
    with open(os.path.join(prof, "hbm_traffic.json"), "w") as fh:
        json.dump(data, fh, indent=1)
        fh.write("\n")
    lines = ["# HBM-side traffic per launch -- rocprofv3 FETCH_SIZE / WRITE_SIZE, config 4", "",
             "Commands (two separate counter runs, eager launches, from the repository root):", "",
             "    " + PROFILE_COMMANDS["fetch"], "    " + PROFILE_COMMANDS["write"], "",
             f"Calibration: the 1 GiB device-to-device copy (`{copy}`, one dispatch) reads FETCH_SIZE = "
             f"{copy_f:.1f} KiB and WRITE_SIZE = {copy_w:.1f} KiB, so bytes = FETCH_SIZE x 1024 x {fscale:.4f} "
             f"and WRITE_SIZE x 1024 x {wscale:.4f}.  FETCH_SIZE counts L2 misses served by the fabric "
             "(Infinity Cache or HBM).", "",
             "| kernel | launches | FETCH KiB | WRITE KiB | calibrated MB/launch |", "|---|---|---|---|---|"]
    for k in sorted(set(fetch) & set(write)):
        mb = (fetch[k][0] * 1024 * fscale + write[k][0] * 1024 * wscale) / 1e6
        lines.append(f"| `{k}` | {fetch[k][1]} | {fetch[k][0]:.1f} | {write[k][0]:.1f} | {mb:.1f} |")
    with open(os.path.join(prof, "hbm_traffic_config4.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return fams


def summarize_profiles():
    """Write profiles/bench_config4_kernel_stats.md, hbm_traffic_config4.md
    and hbm_traffic.json from the output of PROFILE_COMMANDS."""
    import csv

    root = os.path.dirname(os.path.abspath(__file__))
    prof = os.path.join(root, "profiles")
    out_dir = os.path.join(root, "gpurun_out")
    os.makedirs(prof, exist_ok=True)

    rows, fams = [], {}
    if os.path.exists(os.path.join(out_dir, "prof_bench", "bench_kernel_stats.csv")):
        rows = config4_stats_summary(out_dir, prof)
    if os.path.exists(os.path.join(out_dir, "pmc_fetch", "bench_counter_collection.csv")) and \
            os.path.exists(os.path.join(out_dir, "pmc_write", "bench_counter_collection.csv")):
        fams = config4_traffic_summary(out_dir, prof)
    extra = []
    if conversion_summary(out_dir, prof):
        extra.append("conversion_config2_kernels.md")
    if mfma_summary(out_dir, prof):
        extra.append("gemm_mfma_busy_config4.md")
    if mfma_summary(out_dir, prof, key="mfma_config3", out_name="gemm_mfma_busy_config3.md",
                    title="MFMA busy and shader clock of the config-3 GEMMs (GPT-2 small, M = 8192, forward)",
                    what="The config-3 leg: each Linear's GEMM 1 + 20 times back to back, eager, counters per "
                         "dispatch (the kernels run one at a time under counter collection)."):
        extra.append("gemm_mfma_busy_config3.md")
    if mfma_summary(out_dir, prof, key="mfma_config5", out_name="gemm_mfma_busy_config5.md",
                    title="MFMA busy and shader clock of the config-5 GEMMs (48-layer GPT-2 XL stack, 8192 tokens)",
                    what="Config 5's step twice with every layer's weights resident (the streamed step's kernels "
                         "without the copies; copies do not change which GEMMs run), eager, counters per dispatch "
                         "(the kernels run one at a time under counter collection)."):
        extra.append("gemm_mfma_busy_config5.md")
    for key, sub, fname, title, keep in EXTRA_STATS:
        path = os.path.join(out_dir, sub, "bench_kernel_stats.csv")
        if not os.path.exists(path):
            continue
        with open(path) as fh:
            rows_x = [r for r in csv.DictReader(fh) if any(k in r["Name"] for k in keep)]
        lines = [f"# rocprofv3 kernel statistics -- {title}", "",
                 "Command (from the repository root, on one MI355X):", "", "    " + PROFILE_COMMANDS[key], "",
                 "Only this leg's own kernels are listed (the config-4 step also runs in the same process).  "
                 "Durations in microseconds.", "",
                 "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
        for r in rows_x:
            lines.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} |")
        with open(os.path.join(prof, fname), "w") as fh:
            fh.write("\n".join(lines) + "\n")
        extra.append(fname)
    if streaming_summary(out_dir, prof):
        extra.append("streaming_config5.md")
    if timeline_summary(out_dir, prof):
        extra.append("gemm_tile_timeline_config4.md")
    if limiter_summary(out_dir, prof):
        extra.append("limiters_config4.md")
    if config3_summary(out_dir, prof):
        extra.append("gemm_config3_kernels.md")
    print(f"wrote profiles/ summaries ({len(rows)} kernels, traffic families {sorted(fams)}, extra {extra})")


CONVERSION_KERNELS = ("absmax_f32_stage1", "absmax_bf16_stage1", "absmax_stage2", "quantize_f32_kernel",
                      "quantize_bf16_kernel", "dequantize_f32_kernel", "dequantize_bf16_kernel", "hbm_probe_kernel")


def conversion_summary(out_dir, prof):
    """profiles/conversion_config2_kernels.md from the stats_conversion,
    fetch_conversion and write_conversion runs: per kernel instantiation of
    the config-2 leg (n = 2^28), average duration, FETCH / WRITE bytes per
    dispatch (copy-calibrated) and the resulting GB/s."""
    import csv

    stats = os.path.join(out_dir, "prof_conversion", "bench_kernel_stats.csv")
    if not os.path.exists(stats):
        return False
    with open(stats) as fh:
        rows = [r for r in csv.DictReader(fh) if any(k in r["Name"] for k in CONVERSION_KERNELS)]

    def per_dispatch(sub, counter):
        path = os.path.join(out_dir, sub, "bench_counter_collection.csv")
        vals = {}
        if not os.path.exists(path):
            return vals
        with open(path) as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] == counter:
                    vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return vals

    fetch = per_dispatch("pmc_fetch_conv", "FETCH_SIZE")
    write = per_dispatch("pmc_write_conv", "WRITE_SIZE")
    copy = [k for k in fetch if "copyBuffer" in k]
    fscale = wscale = None
    if copy and any("copyBuffer" in k for k in write):
        cf = max(max(fetch[k]) for k in copy)
        cw = max(max(v) for k, v in write.items() if "copyBuffer" in k)
        fscale, wscale = (1 << 30) / (cf * 1024), (1 << 30) / (cw * 1024)
    lines = ["# rocprofv3: config-2 conversion kernels (n = 268,435,456; fp32 and bf16 in, e4m3 and e5m2)", "",
             "Commands (from the repository root, on one MI355X; three separate runs):", "",
             "    " + PROFILE_COMMANDS["stats_conversion"], "    " + PROFILE_COMMANDS["fetch_conversion"],
             "    " + PROFILE_COMMANDS["write_conversion"], "",
             "Each conversion runs 1 + 10 times (warm-up, timed).  `hbm_probe_kernel<R, W, U>` is the bandwidth "
             "calibration with the same access pattern (R bytes read, W written per 16-byte vector slot).  "
             "Traffic: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by the 1 GiB device copy of the same "
             f"runs (fetch x {fscale:.4f}, write x {wscale:.4f}); GB/s = (calibrated fetch + write) / average "
             "duration." if fscale else "Traffic runs missing.", "",
             "| kernel | calls | avg us | fetch MB | write MB | GB/s |", "|---|---|---|---|---|---|"]
    for r in rows:
        name = r["Name"]
        avg_us = float(r["AverageNs"]) / 1e3
        f = fetch.get(name)
        w = write.get(name)
        if f and w and fscale:
            fmb = sum(f) / len(f) * 1024 * fscale / 1e6
            wmb = sum(w) / len(w) * 1024 * wscale / 1e6
            gbs = (fmb + wmb) * 1e6 / (avg_us * 1e-6) / 1e9
            lines.append(f"| `{_short_kernel(name)}` | {r['Calls']} | {avg_us:.1f} | {fmb:.1f} | {wmb:.1f} | "
                         f"{gbs:.0f} |")
        else:
            lines.append(f"| `{_short_kernel(name)}` | {r['Calls']} | {avg_us:.1f} | - | - | - |")
    with open(os.path.join(prof, "conversion_config2_kernels.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return True


def config3_summary(out_dir, prof):
    """profiles/gemm_config3_kernels.md from the config-3 run: config3_bench
    launches each Linear's GEMM 1 + reps times back to back (qkv, attn_proj,
    fc, proj), so the GEMM dispatches in start order split into those runs;
    per Linear the median duration of its timed launches (a split-K GEMM adds
    its reduce kernel) against the bench's attainable bound."""
    import csv

    path = os.path.join(out_dir, "prof_config3", "bench_kernel_trace.csv")
    if not os.path.exists(path):
        return False
    with open(path) as fh:
        tr = sorted(csv.DictReader(fh), key=lambda r: int(r["Start_Timestamp"]))
    reps = 20
    gem = [r for r in tr if "gemm_nt_persistent" in r["Kernel_Name"] or "gemm_nt_dma128" in r["Kernel_Name"]
           or "gemm_nt_kernel" in r["Kernel_Name"]]
    if len(gem) < 4 * (reps + 1):
        return False
    red = [r for r in tr if "splitk_reduce_kernel" in r["Kernel_Name"]]
    med = lambda v: sorted(v)[len(v) // 2]
    M = 8192
    lines = ["# rocprofv3: config-3 GEMMs (GPT-2 small Linears, M = 8192, forward, bf16 out + bf16 bias)", "",
             "Command (from the repository root, on one MI355X):", "", "    " + PROFILE_COMMANDS["stats_config3"], "",
             f"Each Linear's GEMM runs 1 + {reps} times back to back; the table takes the median of its {reps} timed "
             "dispatches (kernel start to end; a split-K launch adds its reduce kernel).  Attainable bound: "
             "min(5.0 PFLOP/s, AI x 8 TB/s), AI = 2MNK / (MK + NK + 2MN) (fp8 operands read once, bf16 output "
             "written once).", "",
             "| Linear | M x N x K | kernel | grid | us | TFLOP/s | attainable TFLOP/s | fraction |",
             "|---|---|---|---|---|---|---|---|"]
    for i, (name, K, N) in enumerate(SMALL_LINEARS):
        run = gem[i * (reps + 1) + 1:(i + 1) * (reps + 1)]
        t0, t1 = int(run[0]["Start_Timestamp"]), int(run[-1]["End_Timestamp"])
        rd = [r for r in red if t0 <= int(r["Start_Timestamp"]) <= t1]
        dur = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in run]
        t = med(dur) + (med([int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rd]) if rd else 0)
        flops = 2.0 * M * N * K
        bound = min(5.0e15, flops / (M * K + N * K + 2 * M * N) * 8.0e12)
        grid = int(run[0].get("Grid_Size", run[0].get("Grid_Size_X", 0))) // max(
            1, int(run[0].get("Workgroup_Size", run[0].get("Workgroup_Size_X", 1))))
        lines.append(f"| {name} | {M} x {N} x {K} | `{_short_kernel(run[0]['Kernel_Name'])}`"
                     f"{' + reduce' if rd else ''} | {grid} | {t / 1e3:.1f} | {flops / (t * 1e-9) / 1e12:.0f} | "
                     f"{bound / 1e12:.0f} | {flops / (t * 1e-9) / bound:.3f} |")
    with open(os.path.join(prof, "gemm_config3_kernels.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return True


def mfma_summary(out_dir, prof, key="mfma", out_name="gemm_mfma_busy_config4.md",
                 title="MFMA busy and shader clock of the config-4 GEMMs",
                 what="Two eager config-4 steps after one warm-up."):
    """profiles/gemm_mfma_busy_config4.md (or, key="mfma_config3", the
    config-3 file) from an mfma counter run: per GEMM dispatch, MFMA-busy
    cycles over the SIMDs' available cycles, and the shader clock the run
    held.  GRBM_GUI_ACTIVE as collected is the sum over the 8 XCDs (each
    counts GPU-busy cycles at the shader clock), so busy cycles per XCD =
    GRBM_GUI_ACTIVE / 8; the 1024 SIMDs (256 CUs x 4) each have that many
    cycles available."""
    import csv

    path = os.path.join(out_dir, "pmc_" + key, "bench_counter_collection.csv")
    kt_path = os.path.join(out_dir, "pmc_" + key, "bench_kernel_trace.csv")
    if not os.path.exists(path):
        return False
    per = {}
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if "gemm_nt_persistent" not in r["Kernel_Name"]:
                continue
            e = per.setdefault(r["Dispatch_Id"], {"name": _short_kernel(r["Kernel_Name"]),
                                                  "full": r["Kernel_Name"], "grid": int(r["Grid_Size"])})
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            e["t"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    if os.path.exists(kt_path):
        with open(kt_path) as fh:
            for r in csv.DictReader(fh):
                if r["Dispatch_Id"] in per:
                    per[r["Dispatch_Id"]]["t"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    lines = ["# rocprofv3: " + title, "",
             "Command (from the repository root, on one MI355X):", "", "    " + PROFILE_COMMANDS[key], "",
             what + "  Per dispatch: MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / "
             "(GRBM_GUI_ACTIVE / 8 x 1024 SIMDs); clock = GRBM_GUI_ACTIVE / 8 / duration; fp8 flop = "
             "SQ_INSTS_VALU_MFMA_MOPS_F8 x 512 (the MFMA work issued, padding of partial tiles included).  "
             "`<A fmt, B fmt, out, bias type, bias, split, dX out>`: `<0, 0, ...>` forward, `<1, 0, ..., void>` "
             "dX alone, the last argument non-void the grouped dX + dW launch.", "",
             "| kernel | grid | us | clock GHz | MFMA busy | issued fp8 TFLOP | TFLOP/s issued | issued / 5.0 PF |",
             "|---|---|---|---|---|---|---|---|"]
    # one row per distinct GEMM (kernel and issued work), medians over its dispatches
    groups = {}
    for did in sorted(per, key=int):
        e = per[did]
        gui = e.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
        if not gui or not e.get("t"):
            continue
        tmpl = e["full"][e["full"].find("<"):e["full"].find(">(") + 1] if "<" in e["full"] else ""
        tfl = e.get("SQ_INSTS_VALU_MFMA_MOPS_F8", 0.0) * 512 / 1e12
        g = groups.setdefault((tmpl, round(tfl, 4), e["grid"]), {"grid": e["grid"] // 512, "t": [], "clk": [], "busy": [],
                                                      "cyc": [], "bcyc": [],
                                                      "kname": "gemm_nt_persistent_narrow_kernel"
                                                      if "narrow" in e["name"] else "gemm_nt_persistent_kernel"})
        g["t"].append(e["t"])
        g["clk"].append(gui / e["t"])
        g["busy"].append(e.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (gui * 1024))
        g["cyc"].append(gui * 1024)
        g["bcyc"].append(e.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0))
    med = lambda v: sorted(v)[len(v) // 2]
    tot_b = tot_c = 0.0
    fast_clock = False
    for (tmpl, tfl, _), g in groups.items():
        t = med(g["t"])
        tot_b += sum(g["bcyc"])
        tot_c += sum(g["cyc"])
        fast_clock |= med(g["clk"]) > 2.45
        lines.append(f"| `{g['kname']}{tmpl}` (x{len(g['t'])}) | {g['grid']} | {t / 1e3:.1f} | "
                     f"{med(g['clk']):.2f} | {med(g['busy']):.3f} | {tfl:.3f} | {tfl / (t * 1e-9):.0f} | "
                     f"{tfl / (t * 1e-9) / FP8_PEAK_TFLOPS:.3f} |")
    if tot_c:
        lines += ["", f"All GEMM dispatches together: MFMA busy {tot_b / tot_c:.3f} of the SIMD cycles they held."]
    if fast_clock:
        lines += ["", "Some dispatches read a clock above the part's 2.4 GHz maximum: for dispatches this short the "
                      "busy window GRBM_GUI_ACTIVE counts under counter collection is longer than the kernel's own "
                      "duration, so their clock and MFMA-busy columns are not reliable; the issued rate (fp8 work "
                      "issued over the kernel's duration) against the 5.0 PF peak is."]
    with open(os.path.join(prof, out_name), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return True


def streaming_summary(out_dir, prof):
    """profiles/streaming_config5.md from the streaming run's bench line
    (gpurun_out/prof_streaming.log, the stdout of PROFILE_COMMANDS
    ["streaming"]): the step, compute and copy times of config 5, every
    copy timed by HIP events on its copy stream (rocprofv3's memory-copy
    trace dropped completion callbacks on this leg, so it is not used)."""
    log = os.path.join(out_dir, "prof_streaming.log")
    if not os.path.exists(log):
        return False
    line = [l for l in open(log) if l.startswith('{"metric"')]
    if not line:
        return False
    st = json.loads(line[-1])["streaming"]
    if "copies_alone" not in st:
        return False
    ca, cs, ss = st["copies_alone"], st["copies_streamed"], st["steady_state"]
    lines = ["# Config 5 weight streaming: step, compute and copy times (HIP events)", "",
             "Command (from the repository root, on one MI355X; stdout to gpurun_out/prof_streaming.log):", "",
             "    " + PROFILE_COMMANDS["streaming"], "",
             st["workload"] + ".  Every copy is one layer's e4m3 weight codes "
             f"({st['copy_bytes'] / 1e6:.2f} MB; W for the forward sweep, W^T for the backward), "
             f"{st['copies_per_step']} per step, timed by HIP events recorded on its copy stream right before and "
             "after it (df_streamer_set_timing).  A copy's own duration runs from its stream reaching it to its "
             "end; with the streamer's two copy streams two copies share the link for most of that time, so the "
             "link's rate is the bytes over the time any copy was in flight (busy).", "",
             "| quantity | value |", "|---|---|",
             f"| streamed step | {st['ms_per_step']} ms ({st['value']} TFLOP/s) |",
             f"| compute alone (weights resident) / the same under concurrent copies | {st['compute_alone_ms']} / "
             f"{st.get('compute_under_copies_ms')} ms |",
             f"| compute alone: forward sweep / backward sweep | {st['compute_fwd_sweep_ms']} / "
             f"{st['compute_bwd_sweep_ms']} ms |",
             f"| copies alone | {st['h2d_alone_ms']} ms ({st['h2d_gbs']} GB/s) |",
             f"| overlap = max(compute, copies) / streamed | {st['overlap']} |",
             f"| flow-shop bound of the entry order (per-entry copy and compute times) | {st['flowshop_bound_ms']} ms "
             f"(streamed step at {st['overlap_vs_flowshop_bound']} of it) |",
             f"| steady state: {ss['micro_batches']} passes, same weights, {ss['slots']} slots | {ss['ms_per_pass']} ms "
             f"per pass (overlap {ss['overlap']}) |", "",
             "| copies | count | median copy | its rate | sum of durations | busy | link rate | copies in flight |",
             "|---|---|---|---|---|---|---|---|"]
    for name, c in (("alone", ca), ("in the streamed step", cs)):
        lines.append(f"| {name} | {c['copies']} | {c['median_copy_ms']} ms | {c['median_copy_gbs']} GB/s | "
                     f"{c['sum_copy_ms']} ms | {c['busy_ms']} ms | {c['busy_gbs']} GB/s | {c['copies_in_flight_avg']} |")
    with open(os.path.join(prof, "streaming_config5.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return True


def timeline_summary(out_dir, prof):
    """profiles/gemm_tile_timeline_config4.md from the timeline run's JSON
    (gpurun_out/prof_timeline.log, the stdout of PROFILE_COMMANDS["timeline"])."""
    log = os.path.join(out_dir, "prof_timeline.log")
    if not os.path.exists(log):
        return False
    line = [l for l in open(log) if l.startswith('{"tile_timeline"')]
    if not line:
        return False
    tl = json.loads(line[-1])["tile_timeline"]
    lines = ["# Per-tile timeline of the persistent GEMM -- config-4 forward GEMMs (M = 16384, bf16 bias and output)",
             "", "Command (from the repository root, on one MI355X; stdout to gpurun_out/prof_timeline.log):", "",
             "    " + PROFILE_COMMANDS["timeline"], "",
             "df_fp8_gemm_fwd_timeline runs the forward's persistent kernel with wave 0 of every block stamping the "
             "GPU's 100 MHz real-time counter at the block's start and at each of its tiles' start, epilogue start "
             "and epilogue end (the shortest of three runs per shape).  Main loop = a tile's DMA steps and MFMAs "
             "(the next tile's first two DMA steps are issued inside it); epilogue = scale, bias, bf16 conversion, "
             "LDS slab passes and stores; gap = epilogue end to the next tile's start; prologue = block start to "
             "its first tile.  Medians over tiles or blocks, microseconds.", "",
             "| GEMM | N | K | K steps | tiles / blocks | main loop | per K step | epilogue | gap | epilogue share "
             "| block prologue | first / last block end | kernel span |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for name, d in tl["shapes"].items():
        lines.append(f"| {name} | {d['N']} | {d['K']} | {d['k_steps']} | {d['tiles']} / {d['blocks']} | "
                     f"{d['tile_main_loop_us']} | {d['main_loop_per_k_step_us']} | {d['tile_epilogue_us']} | "
                     f"{d['gap_to_next_tile_us']} | {d['epilogue_share_of_tile']} | {d['block_prologue_us']} | "
                     f"{d['block_end_first_us']} / {d['block_end_last_us']} | {d['kernel_span_us']} |")
    tails = [(n, d) for n, d in tl["shapes"].items() if d.get("tail_column_main_loop_us")]
    if tails:
        lines += ["", "Tiles of the last tile column, whose columns past N are outside the operand buffer (their DMA "
                  "lanes return zeros without a memory request), against all tiles of the same launch (medians):", "",
                  "| GEMM | columns in range of the last tile column | its tiles' main loop | all tiles' main loop |",
                  "|---|---|---|---|"]
        for n, d in tails:
            lines.append(f"| {n} | {d['tail_column_valid_cols']} of 256 | {d['tail_column_main_loop_us']} | "
                         f"{d['tile_main_loop_us']} |")
    with open(os.path.join(prof, "gemm_tile_timeline_config4.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return True


# kernel families of the limiter summary: (label, kernel name prefix)
LIMITER_KERNELS = (
    ("gemm_fwd", "void dfk::gemm_nt_persistent_kernel<0, 0, unsigned short, unsigned short, true, false, void>"),
    ("gemm_bwd (dW unsplit)", "void dfk::gemm_nt_persistent_kernel<1, 0, float, float, false, false, unsigned short>"),
    ("quantize X", "void dfk::quantize_2d_jit_w5_kernel<unsigned short, 0, false>"),
    ("quantize dY + db", "void dfk::quantize_2d_jit_w5_kernel<unsigned short, 1, true>"),
)


def limiter_summary(out_dir, prof):
    """profiles/limiters_config4.md from the pmc_* runs: per kernel family,
    counter averages per dispatch and the fractions that name what bounds
    it.  Normalisation: cycles per dispatch = GRBM_GUI_ACTIVE / 8 (one count
    per XCD); per-CU blocks (TA, TD, TCP) over 256 CUs, L2 channels (TCC)
    over 8 x 16; SQ wave counters as fractions of SQ_WAVE_CYCLES."""
    import csv

    vals = {}
    for key in ("sq1", "sq2", "tatd", "tcp", "ea"):
        path = os.path.join(out_dir, "pmc_" + key, "bench_counter_collection.csv")
        if not os.path.exists(path):
            return False
        with open(path) as fh:
            for r in csv.DictReader(fh):
                for label, pre in LIMITER_KERNELS:
                    if r["Kernel_Name"].startswith(pre):
                        vals.setdefault(label, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    avg = {lab: {c: sum(v) / len(v) for c, v in d.items()} for lab, d in vals.items()}
    labs = [lab for lab, _ in LIMITER_KERNELS if lab in avg]
    lines = ["# What bounds the config-4 GEMM main loop and 2-D quantize -- rocprofv3 counters", "",
             "Commands (five counter runs of the same eager config-4 steps, from the repository root):", ""]
    lines += ["    " + PROFILE_COMMANDS["pmc_" + k] for k in ("sq1", "sq2", "tatd", "tcp", "ea")]
    lines += ["", "Kernels: " + "; ".join(f"{lab} = `{pre[len('void dfk::'):]}`" for lab, pre in LIMITER_KERNELS
                                          if lab in avg) + ".",
              "", "Per kernel family, averages per dispatch.  cycles = GRBM_GUI_ACTIVE / 8; per-CU fractions divide "
              "the counter's sum over the 256 CUs by 256 x cycles; L2 fractions divide by 128 channels x cycles; "
              "wave fractions divide by SQ_WAVE_CYCLES.", "",
              "| quantity | " + " | ".join(labs) + " |", "|---|" + "---|" * len(labs)]

    def row(name, fn, fmt="{:.3f}"):
        cells = []
        for lab in labs:
            try:
                cells.append(fmt.format(fn(avg[lab])))
            except (KeyError, ZeroDivisionError, TypeError):
                cells.append("-")
        lines.append(f"| {name} | " + " | ".join(cells) + " |")

    cyc = lambda a: a["GRBM_GUI_ACTIVE"] / 8
    row("cycles per dispatch", cyc, "{:.0f}")
    row("MFMA busy (of 1024 SIMDs)", lambda a: a["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc(a) * 1024))
    row("waves waiting on a dependency (s_waitcnt, barrier)", lambda a: a["SQ_WAIT_ANY"] / a["SQ_WAVE_CYCLES"])
    row("waves with an instruction ready but not issued", lambda a: a["SQ_WAIT_INST_ANY"] / a["SQ_WAVE_CYCLES"])
    row("VMEM issue blocked: TA command FIFO full (per CU)", lambda a: a["SQ_VMEM_TA_CMD_FIFO_FULL"] / (256 * cyc(a)))
    row("VMEM issue blocked: TA address FIFO full (per CU)", lambda a: a["SQ_VMEM_TA_ADDR_FIFO_FULL"] / (256 * cyc(a)))
    row("TA busy", lambda a: a["TA_TA_BUSY_sum"] / (256 * cyc(a)))
    row("TD busy", lambda a: a["TD_TD_BUSY_sum"] / (256 * cyc(a)))
    row("TD stalled on the L1 (TC)", lambda a: a["TD_TC_STALL_sum"] / (256 * cyc(a)))
    row("L1 (TCP) stalled on data pending from L2", lambda a: a["TCP_PENDING_STALL_CYCLES_sum"] / (256 * cyc(a)))
    row("L2 read latency seen by L1 (cycles)",
        lambda a: a["TCP_TCC_READ_REQ_LATENCY_sum"] / a["TCP_TCC_READ_REQ_sum"], "{:.0f}")
    row("L2 hit rate", lambda a: a["TCC_HIT_sum"] / (a["TCC_HIT_sum"] + a["TCC_MISS_sum"]))
    row("TLB (UTCL1) misses per dispatch", lambda a: a["TCP_UTCL1_TRANSLATION_MISS_sum"], "{:.0f}")
    row("LDS bank-conflict cycles per LDS instruction", lambda a: a["SQ_LDS_BANK_CONFLICT"] / a["SQ_INSTS_LDS"])
    row("DRAM read credit stall (per L2 channel)", lambda a: a["TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum"] / (128 * cyc(a)))
    row("DRAM write credit stall (per L2 channel)",
        lambda a: a["TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum"] / (128 * cyc(a)))
    row("fabric read requests per dispatch", lambda a: a["TCC_EA0_RDREQ_sum"], "{:.0f}")
    row("fabric write requests per dispatch", lambda a: a["TCC_EA0_WRREQ_sum"], "{:.0f}")
    with open(os.path.join(prof, "limiters_config4.md"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    return True


def conversion_bench(torch, df, synth, dev, stream, reps=10):
    """Config 2: n = 268,435,456 standalone absmax / quantize / dequantize."""
    import numpy as np
    n = 268_435_456
    x32 = torch.from_numpy(synth.conversion_input(n)).to(dev)
    x16 = x32.to(torch.bfloat16)
    q = torch.empty(n, dtype=torch.uint8, device=dev)
    o32 = torch.empty(n, dtype=torch.float32, device=dev)
    o16 = torch.empty(n, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(df.lib().df_absmax_workspace_bytes(), dtype=torch.uint8, device=dev)
    sc = torch.empty(2, dtype=torch.float32, device=dev)
    res = {"n": n}
    for src, x, o, esz in (("f32", x32, o32, 4), ("bf16", x16, o16, 2)):
        for fmt, fname in ((0, "e4m3"), (1, "e5m2")):
            absfn = "df_absmax_scale_f32" if src == "f32" else "df_absmax_scale_bf16"
            qfn = f"df_quantize_{src}_{fname}"
            dfn = f"df_dequantize_{fname}_{src}"
            calls = {
                "absmax": (lambda: df.call(absfn, x.data_ptr(), n, fmt, sc.data_ptr(), sc.data_ptr() + 4,
                                           ws.data_ptr(), ws.numel(), stream), n * esz),
                "quantize": (lambda: df.call(qfn, x.data_ptr(), n, sc.data_ptr() + 4, q.data_ptr(), stream),
                             n * esz + n),
                "dequantize": (lambda: df.call(dfn, q.data_ptr(), n, sc.data_ptr() + 4, o.data_ptr(), stream),
                               n + n * esz),
            }
            for kname, (fn, nbytes) in calls.items():
                fn()
                torch.cuda.synchronize()
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / reps
                gbs = nbytes / (ms * 1e-3) / 1e9
                res[f"{kname}_{src}_{fname}"] = {"ms": round(ms, 4), "gbs": round(gbs, 1),
                                                 "frac": round(gbs / HBM_PEAK_GBS, 4)}
    # The ceiling of each access pattern on this part: the same loads and
    # stores as the kernels above (df_hbm_probe: non-temporal loads and
    # stores, as many per thread as the kernel with that pattern issues,
    # one chunk per block), no arithmetic.
    probe_dst = torch.empty(max(int(df.lib().df_hbm_probe_dst_bytes(16, 16, n * 4)), 16), dtype=torch.uint8,
                            device=dev)
    ceil = {}
    for key, rb, wb, src_t in (("read_f32", 16, 0, x32), ("read_bf16", 16, 0, x16),
                               ("f32_to_fp8", 16, 4, x32), ("bf16_to_fp8", 16, 8, x16),
                               ("fp8_to_f32", 4, 16, q), ("fp8_to_bf16", 8, 16, q),
                               ("copy_f32", 16, 16, x32)):
        sbytes = src_t.numel() * src_t.element_size()
        nbytes = sbytes + (sbytes // rb) * wb

        def fn(rb=rb, wb=wb, src_t=src_t, sbytes=sbytes):
            df.call("df_hbm_probe", rb, wb, src_t.data_ptr(), sbytes, probe_dst.data_ptr(), stream)

        fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        ceil[key] = {"pattern": f"{rb}:{wb}", "bytes": nbytes, "ms": round(ms, 4), "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)}
    res["pattern_ceilings"] = ceil
    pattern_of = {"absmax_f32": "read_f32", "absmax_bf16": "read_bf16", "quantize_f32": "f32_to_fp8",
                  "quantize_bf16": "bf16_to_fp8", "dequantize_f32": "fp8_to_f32", "dequantize_bf16": "fp8_to_bf16"}
    for key, v in res.items():
        if isinstance(v, dict) and "gbs" in v and key != "pattern_ceilings":
            kind, src = key.split("_")[0], key.split("_")[1]
            c = ceil[pattern_of[f"{kind}_{src}"]]["gbs"]
            v["frac_of_pattern_ceiling"] = round(v["gbs"] / c, 4)
    del x32, x16, q, o32, o16, probe_dst
    torch.cuda.empty_cache()
    return res


def delayed_scaling_leg(torch, df, layers, M, args, cur, ws, gws, gws_bytes, jit_ms, step_flops,
                        weights_batch=None, w_sc=None):
    """The config-4 step with delayed scaling: every activation and gradient
    (X, dY of each Linear) is quantized at the scale of its amax history and
    measures its own absmax in the same pass (df_quantize_2d_delayed), so
    their separate absmax passes disappear.  The weights are quantized as in
    the just-in-time step: in one df_quantize_2d_batch call (weights_batch,
    scales in w_sc), or with --per-linear-weights delayed like the others.
    Histories are seeded from the operands' own absmax first.  Two steps are
    captured per graph (the two scale slots of each operand alternate),
    replayed args.steps // 2 + 1 times."""
    from deepfuse_amd import DType, Fmt
    BF, F32 = int(DType.BFLOAT16), int(DType.FLOAT32)
    E4, E5 = int(Fmt.E4M3), int(Fmt.E5M2)
    H = args.history
    dws_bytes = 0
    roles = []
    for l in layers:
        K, N = l["K"], l["N"]
        r = {}
        for name, x, rows, cols, fmt, q, qt, cs in (("x", l["X"], M, K, E4, l["Xq"], l["Xt"], None),
                                                    ("w", l["W"], N, K, E4, l["Wq"], l["Wt"], None),
                                                    ("dy", l["dY"], M, N, E5, l["dYq"], l["dYt"], l["db"])):
            st = {"x": x, "rows": rows, "cols": cols, "fmt": fmt, "q": q, "qt": qt, "cs": cs,
                  "hist": torch.empty(H, dtype=torch.float32, device=x.device),
                  "sc": torch.empty(3, dtype=torch.float32, device=x.device)}
            dws_bytes = max(dws_bytes, df.lib().df_quantize_2d_delayed_workspace_bytes(
                rows, cols, q.stride(0), qt.stride(0), int(cs is not None)))
            df.call("df_absmax_bf16", x.data_ptr(), x.numel(), st["sc"].data_ptr() + 8, ws.data_ptr(), ws.numel(),
                    cur())
            df.call("df_amax_history_init", st["sc"].data_ptr() + 8, fmt, st["hist"].data_ptr(), H,
                    st["sc"].data_ptr(), cur())
            r[name] = st
        roles.append(r)
    dws = torch.empty(dws_bytes, dtype=torch.uint8, device=layers[0]["X"].device)

    def quant(st, parity):
        used = st["sc"].data_ptr() + 4 * parity
        nxt = st["sc"].data_ptr() + 4 * (parity ^ 1)
        cs = st["cs"]
        df.call("df_quantize_2d_delayed", BF, st["x"].data_ptr(), st["rows"], st["cols"], st["cols"], st["fmt"],
                used, nxt, st["hist"].data_ptr(), H, st["q"].data_ptr(), st["q"].stride(0), st["qt"].data_ptr(),
                st["qt"].stride(0), None if cs is None else cs.data_ptr(), dws.data_ptr(), dws_bytes, cur())
        return used

    def step(parity):
        if weights_batch is not None:
            weights_batch()
        for i, (l, r) in enumerate(zip(layers, roles)):
            K, N = l["K"], l["N"]
            sx = quant(r["x"], parity)
            sw = quant(r["w"], parity) if weights_batch is None else w_sc.data_ptr() + 4 * i
            df.call("df_fp8_gemm_fwd", l["Xq"].data_ptr(), l["Xq"].stride(0), l["Wq"].data_ptr(),
                    l["Wq"].stride(0), M, N, K, sx, sw, BF, l["b"].data_ptr(), BF, l["Y"].data_ptr(), N,
                    gws.data_ptr(), gws_bytes, cur())
            sdy = quant(r["dy"], parity)
            if args.separate_backward:
                df.call("df_fp8_gemm_bwd_dx", l["dYq"].data_ptr(), l["dYq"].stride(0), l["Wt"].data_ptr(),
                        l["Wt"].stride(0), M, N, K, sdy, sw, BF, l["dX"].data_ptr(), K, gws.data_ptr(),
                        gws_bytes, cur())
                df.call("df_fp8_gemm_bwd_dw", l["dYt"].data_ptr(), l["dYt"].stride(0), l["Xt"].data_ptr(),
                        l["Xt"].stride(0), M, N, K, sdy, sx, F32, l["dW"].data_ptr(), K, gws.data_ptr(),
                        gws_bytes, cur())
            else:
                df.call("df_fp8_gemm_bwd", l["dYq"].data_ptr(), l["dYq"].stride(0), l["Wt"].data_ptr(),
                        l["Wt"].stride(0), l["dYt"].data_ptr(), l["dYt"].stride(0), l["Xt"].data_ptr(),
                        l["Xt"].stride(0), M, N, K, sdy, sw, sx, BF, l["dX"].data_ptr(), K, F32,
                        l["dW"].data_ptr(), K, gws.data_ptr(), gws_bytes, cur())

    for _ in range(max(1, args.warmup)):
        step(0)
        step(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(0)
        step(1)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, args.steps // 2)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (2 * reps)
    del graph
    return {"history": H, "weights": "per Linear, delayed" if weights_batch is None else "batched, just-in-time",
            "steps": 2 * reps, "ms_per_step": round(ms, 4),
            "tflops": round(step_flops / (ms * 1e-3) / 1e12, 2),
            "speedup_vs_just_in_time": round(jit_ms / ms, 4)}


def vendor_bench(torch, df, dev, stream, M=16384, reps=10):
    """The 12 config-4 GEMM shapes on the vendor fp8 GEMM (hipBLASLt through
    torch._scaled_mm, OCP fp8, bf16 output) next to this library's GEMM on
    the same operands: a comparison, not part of the product path.  Each
    shape is C[m,n] = sum_k A[m,k] B[n,k] with A in e4m3 (forward) or e5m2
    (backward) and B in e4m3."""
    from deepfuse_amd import DType, Fmt
    shapes = []
    for _, K, N in XL_LINEARS:
        shapes += [("fwd", M, N, K, Fmt.E4M3), ("dx", M, K, N, Fmt.E5M2), ("dw", N, K, M, Fmt.E5M2)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    one = torch.ones(1, dtype=torch.float32, device=dev)
    tdt = {Fmt.E4M3: torch.float8_e4m3fn, Fmt.E5M2: torch.float8_e5m2}
    res = {"shapes": len(shapes)}
    tot_flop = tot_ours = tot_vendor = 0.0
    errors = []

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    for fam, m, n, k, fa in shapes:
        a = (torch.randn(m, k, device=dev, generator=gen) * 4).to(tdt[fa])
        b = (torch.randn(n, k, device=dev, generator=gen) * 4).to(torch.float8_e4m3fn)
        c = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        wsb = df.lib().df_fp8_gemm_workspace_bytes(m, n, k)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
        ours = lambda: df.call("df_fp8_gemm_nt", int(fa), a.data_ptr(), k, int(Fmt.E4M3), b.data_ptr(), k, m, n, k,
                               one.data_ptr(), one.data_ptr(), int(DType.BFLOAT16), None, int(DType.BFLOAT16),
                               c.data_ptr(), n, ws.data_ptr(), wsb, stream)
        vendor = lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
        flop = 2.0 * m * n * k
        t_ours = timed(ours)
        try:
            t_vendor = timed(vendor)
        except Exception as exc:  # the vendor path may refuse a format pair
            errors.append(f"{fam} {m}x{n}x{k}: {type(exc).__name__}")
            t_vendor = None
        tot_flop += flop
        tot_ours += t_ours
        if t_vendor is not None:
            tot_vendor += t_vendor
        del a, b, c, ws
    res["ours_tflops"] = round(tot_flop / (tot_ours * 1e-3) / 1e12, 1)
    if not errors:
        res["vendor_tflops"] = round(tot_flop / (tot_vendor * 1e-3) / 1e12, 1)
        res["ratio"] = round(tot_vendor / tot_ours, 3)
    res["vendor"] = "torch._scaled_mm (hipBLASLt), bf16 output, unit scales"
    if errors:
        res["vendor_errors"] = errors
    torch.cuda.empty_cache()
    return res


def config3_bench(torch, df, synth, dev, stream, M=8192, reps=20, vendor=False):
    """Config 3: the four GPT-2 small Linears at 8192 tokens, forward only.
    Per Linear: absmax + e4m3 codes of X [M, K] and W [N, K] (bf16), then
    the fp8 GEMM with the fused scale, bf16 bias and bf16 output.  Reported:
    each GEMM alone (average launch), the four GEMMs, and the whole forward
    with its quantization (weights per Linear, and all four in one
    df_quantize_2d_batch call), against the per-shape attainable bound
    min(5.0 PF, AI x 8 TB/s) (AI: fp8 A and B read once, bf16 C written
    once).  With vendor, each GEMM is also timed on torch._scaled_mm
    (hipBLASLt) over the same codes, bias and output type, unit scales: a
    comparison, not part of the product path."""
    import numpy as np
    from deepfuse_amd import DType, Fmt
    BF, E4 = int(DType.BFLOAT16), int(Fmt.E4M3)
    bf = lambda a: torch.from_numpy(synth.f32_to_bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)
    aws = torch.empty(df.lib().df_absmax_workspace_bytes(), dtype=torch.uint8, device=dev)
    gws_b = max(df.lib().df_fp8_gemm_workspace_bytes(M, n, k) for _, k, n in SMALL_LINEARS)
    gws = torch.empty(max(gws_b, 16), dtype=torch.uint8, device=dev)
    lin = []
    for i, (name, K, N) in enumerate(SMALL_LINEARS):
        seed = synth.SEED_BASE + 3 + 10 * i
        lin.append(dict(name=name, K=K, N=N, X=bf(synth.normal((M, K), 1.0, seed=seed)),
                        W=bf(synth.normal((N, K), 0.02, seed=seed + 1)), b=bf(synth.normal((N,), 0.02, seed=seed + 2)),
                        Xq=torch.empty((M, K), dtype=torch.uint8, device=dev),
                        Wq=torch.empty((N, K), dtype=torch.uint8, device=dev),
                        Y=torch.empty((M, N), dtype=torch.bfloat16, device=dev),
                        sc=torch.empty(4, dtype=torch.float32, device=dev)))

    def quant(l):
        s = l["sc"].data_ptr()
        for t, q, am, sp in ((l["X"], l["Xq"], s, s + 4), (l["W"], l["Wq"], s + 8, s + 12)):
            df.call("df_absmax_scale_bf16", t.data_ptr(), t.numel(), E4, am, sp, aws.data_ptr(), aws.numel(), stream)
            df.call("df_quantize_bf16_e4m3", t.data_ptr(), t.numel(), sp, q.data_ptr(), stream)

    def gemm(l):
        s = l["sc"].data_ptr()
        df.call("df_fp8_gemm_fwd", l["Xq"].data_ptr(), l["K"], l["Wq"].data_ptr(), l["K"], M, l["N"], l["K"], s + 4,
                s + 12, BF, l["b"].data_ptr(), BF, l["Y"].data_ptr(), l["N"], gws.data_ptr(), gws.numel(), stream)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    res = {"workload": f"config 3: GPT-2 small Linears, M={M} tokens, forward, bf16 out + fused bias", "linears": {}}
    tot_flops, tot_ms = 0, 0.0
    for l in lin:
        quant(l)
        K, N = l["K"], l["N"]
        flops = 2 * M * N * K
        ms = timed(lambda: gemm(l))
        ai = flops / (M * K + N * K + 2 * M * N)
        bound = min(5.0e15, ai * 8.0e12)
        res["linears"][l["name"]] = {"shape": [M, N, K], "ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                                     "attainable_tflops": round(bound / 1e12, 1),
                                     "frac_of_attainable": round(flops / (ms * 1e-3) / bound, 4)}
        if vendor:
            one = torch.ones(1, dtype=torch.float32, device=dev)
            a8, b8 = l["Xq"].view(torch.float8_e4m3fn), l["Wq"].view(torch.float8_e4m3fn)
            try:
                vms = timed(lambda: torch._scaled_mm(a8, b8.t(), scale_a=one, scale_b=one, bias=l["b"],
                                                     out_dtype=torch.bfloat16))
                res["linears"][l["name"]]["vendor"] = {"ms": round(vms, 4),
                                                       "tflops": round(flops / (vms * 1e-3) / 1e12, 1),
                                                       "frac_of_attainable": round(flops / (vms * 1e-3) / bound, 4)}
            except Exception as exc:  # the vendor path may refuse the bias or the format
                res["linears"][l["name"]]["vendor"] = {"error": type(exc).__name__}
        tot_flops += flops
        tot_ms += ms
    res["gemm_only"] = {"ms": round(tot_ms, 4), "tflops": round(tot_flops / (tot_ms * 1e-3) / 1e12, 1),
                        "frac_of_fp8_peak": round(tot_flops / (tot_ms * 1e-3) / 5.0e15, 4)}
    if vendor:
        res["vendor"] = "torch._scaled_mm (hipBLASLt), bf16 output + bf16 bias, unit scales"

    def forward():
        for l in lin:
            quant(l)
            gemm(l)

    ms = timed(forward)
    res["forward_with_quantize"] = {"ms": round(ms, 4), "tflops": round(tot_flops / (ms * 1e-3) / 1e12, 1)}

    # the same forward with the four weights' codes from one df_quantize_2d_batch call
    import ctypes
    nl = len(lin)
    wsc = torch.empty(nl, dtype=torch.float32, device=dev)
    qws = torch.empty(df.lib().df_quantize_2d_batch_workspace_bytes(), dtype=torch.uint8, device=dev)
    iarr = lambda vals: (ctypes.c_int * nl)(*vals)
    parr = lambda ts: (ctypes.c_void_p * nl)(*[t.data_ptr() for t in ts])
    wargs = (parr([l["W"] for l in lin]), iarr([l["N"] for l in lin]), iarr([l["K"] for l in lin]), E4, None,
             wsc.data_ptr(), parr([l["Wq"] for l in lin]), iarr([l["K"] for l in lin]), None, None,
             qws.data_ptr(), qws.numel())

    def forward_batched():
        df.call("df_quantize_2d_batch", BF, nl, *wargs, stream)
        for i, l in enumerate(lin):
            s = l["sc"].data_ptr()
            df.call("df_absmax_scale_bf16", l["X"].data_ptr(), l["X"].numel(), E4, s, s + 4, aws.data_ptr(),
                    aws.numel(), stream)
            df.call("df_quantize_bf16_e4m3", l["X"].data_ptr(), l["X"].numel(), s + 4, l["Xq"].data_ptr(), stream)
            df.call("df_fp8_gemm_fwd", l["Xq"].data_ptr(), l["K"], l["Wq"].data_ptr(), l["K"], M, l["N"], l["K"],
                    s + 4, wsc.data_ptr() + 4 * i, BF, l["b"].data_ptr(), BF, l["Y"].data_ptr(), l["N"],
                    gws.data_ptr(), gws.numel(), stream)

    ms = timed(forward_batched)
    res["forward_with_quantize_weights_batched"] = {"ms": round(ms, 4),
                                                    "tflops": round(tot_flops / (ms * 1e-3) / 1e12, 1)}

    # the same forward with X at delayed scaling (df_quantize_2d_delayed: the
    # scale from a 16-entry amax history, the absmax measured in the same
    # pass; two scale slots alternate), the weights batched just-in-time
    H = 16
    dws_b = max(df.lib().df_quantize_2d_delayed_workspace_bytes(M, l["K"], l["K"], 0, 0) for l in lin)
    dws = torch.empty(max(dws_b, 16), dtype=torch.uint8, device=dev)
    for l in lin:
        l["hist"] = torch.empty(H, dtype=torch.float32, device=dev)
        l["dsc"] = torch.empty(3, dtype=torch.float32, device=dev)
        d = l["dsc"].data_ptr()
        df.call("df_absmax_bf16", l["X"].data_ptr(), l["X"].numel(), d + 8, aws.data_ptr(), aws.numel(), stream)
        df.call("df_amax_history_init", d + 8, E4, l["hist"].data_ptr(), H, d, stream)

    def forward_delayed(parity):
        df.call("df_quantize_2d_batch", BF, nl, *wargs, stream)
        for i, l in enumerate(lin):
            d = l["dsc"].data_ptr()
            used, nxt = d + 4 * parity, d + 4 * (parity ^ 1)
            df.call("df_quantize_2d_delayed", BF, l["X"].data_ptr(), M, l["K"], l["K"], E4, used, nxt,
                    l["hist"].data_ptr(), H, l["Xq"].data_ptr(), l["K"], None, 0, None, dws.data_ptr(), dws.numel(),
                    stream)
            df.call("df_fp8_gemm_fwd", l["Xq"].data_ptr(), l["K"], l["Wq"].data_ptr(), l["K"], M, l["N"], l["K"],
                    used, wsc.data_ptr() + 4 * i, BF, l["b"].data_ptr(), BF, l["Y"].data_ptr(), l["N"],
                    gws.data_ptr(), gws.numel(), stream)

    ms = timed(lambda: (forward_delayed(0), forward_delayed(1))) / 2
    res["forward_with_quantize_delayed"] = {"ms": round(ms, 4), "tflops": round(tot_flops / (ms * 1e-3) / 1e12, 1),
                                            "history": H, "weights": "batched, just-in-time"}
    return res


def producer_bench(torch, df, synth, dev, stream, M=16384, C=1600, reps=10):
    """Row f3 at the GPT-2 XL LayerNorm shape (M tokens x d = 1600, bf16, with
    gamma/beta): the unfused chain the reference's layers imply (LayerNorm
    writes y; the Linear reads it for the absmax, then again to quantize it
    into row and transposed e4m3 codes) against the fused producer (row
    statistics + absmax in one pass, codes in a second; y never written),
    just-in-time and delayed.  Bytes per element: unfused 2+2 | 2 | 2+2
    (LN | absmax | quantize), fused 2 | 2+2, minimum 2+2 (read x once,
    write both code layouts)."""
    import numpy as np
    from deepfuse_amd import DType, Fmt
    BF, E4 = int(DType.BFLOAT16), int(Fmt.E4M3)
    bf = lambda a: torch.from_numpy(synth.f32_to_bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)
    x = bf(synth.normal((M, C), 2.0, seed=1700, mean=0.5))
    g = bf(synth.normal((C,), 0.2, seed=1701, mean=1.0))
    b = bf(synth.normal((C,), 0.5, seed=1702))
    y = torch.empty_like(x)
    Cp, Mp = df.round16(C), df.round16(M)
    q = torch.empty((M, Cp), dtype=torch.uint8, device=dev)
    qt = torch.empty((C, Mp), dtype=torch.uint8, device=dev)
    sc = torch.empty(4, dtype=torch.float32, device=dev)
    hist = torch.zeros(16, dtype=torch.float32, device=dev)
    lws_b = df.lib().df_layernorm_workspace_bytes(M, C, Cp, Mp)
    lws = torch.empty(lws_b, dtype=torch.uint8, device=dev)
    aws = torch.empty(df.lib().df_absmax_workspace_bytes(), dtype=torch.uint8, device=dev)
    p = sc.data_ptr()

    def unfused():
        df.call("df_layernorm", BF, x.data_ptr(), M, C, C, g.data_ptr(), b.data_ptr(), 1e-5, y.data_ptr(), C,
                lws.data_ptr(), lws_b, stream)
        df.call("df_absmax_scale_bf16", y.data_ptr(), y.numel(), E4, None, p, aws.data_ptr(), aws.numel(), stream)
        df.call("df_quantize_2d", BF, y.data_ptr(), M, C, C, E4, p, q.data_ptr(), Cp, qt.data_ptr(), Mp, stream)

    def fused():
        df.call("df_layernorm_quantize", BF, x.data_ptr(), M, C, C, g.data_ptr(), b.data_ptr(), 1e-5, None, 0,
                E4, p + 4, None, q.data_ptr(), Cp, qt.data_ptr(), Mp, lws.data_ptr(), lws_b, stream)

    def fused_delayed():
        df.call("df_layernorm_quantize_delayed", BF, x.data_ptr(), M, C, C, g.data_ptr(), b.data_ptr(), 1e-5, None,
                0, E4, p + 8, p + 8, hist.data_ptr(), 16, q.data_ptr(), Cp, qt.data_ptr(), Mp, lws.data_ptr(),
                lws_b, stream)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    n = M * C
    res = {"shape": [M, C], "dtype": "bf16", "min_bytes_per_elem": 4}
    for name, fn, bpe in (("unfused", unfused, 10), ("fused", fused, 6), ("fused_delayed", fused_delayed, 6)):
        ms = timed(fn)
        res[name] = {"ms": round(ms, 4), "bytes_per_elem": bpe, "gbs": round(n * bpe / (ms * 1e-3) / 1e9, 1),
                     "min_bytes_gbs": round(n * 4 / (ms * 1e-3) / 1e9, 1)}
    res["fused_speedup"] = round(res["unfused"]["ms"] / res["fused"]["ms"], 3)
    res["gemm_producer"] = gemm_producer_bench(torch, df, synth, dev, stream, M=M, C=C, reps=reps)
    return res


def gemm_producer_bench(torch, df, synth, dev, stream, M=16384, C=1600, reps=10, rounds=7):
    """The GEMM producer at the config-4 fc shapes, both directions, up to the
    next Linear's codes.  The reference block passes fc1's bf16 Y to fc2 and,
    in the backward, fc2's dX to fc1 as its output gradient
    (transformer_block.cu:79-81, :127-134), so each next scale is an absmax
    of a GEMM output.
    - forward (M x 1600 -> M x 6400): fc1 GEMM, absmax pass over Y, quantize
      Y (two calls; or the one-call quantize, "unfused_jit") against the GEMM
      that folds |Y| in its epilogue, then the quantize at its scale;
    - backward (fc2: dY M x 1600, W 1600 x 6400): the grouped dX + dW GEMM,
      then fc1's dY quantize with the bias gradient's column sums (absmax
      pass + quantize, or the one-call quantize) against the grouped GEMM
      that folds |dX|, then the quantize at its scale.
    The absmax pass the fusions remove reads 2 bytes per output element.
    Every variant is timed in rounds that rotate their order; medians."""
    from deepfuse_amd import DType, Fmt
    BF, F32, E4, E5 = int(DType.BFLOAT16), int(DType.FLOAT32), int(Fmt.E4M3), int(Fmt.E5M2)
    N = 4 * C
    L = df.lib()

    def operand(shape, std, seed, fmt, want_q, want_qt):
        x = torch.from_numpy(synth.normal(shape, std, seed=seed)).to(dev).to(torch.bfloat16)
        _, s = df.absmax_scale(x, fmt)
        q_, qt_ = df.quantize_2d(x, s, fmt, want_q=want_q, want_qt=want_qt)
        return q_, qt_, s

    def timed(fn):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def rotated(variants):
        # back-to-back blocks of one variant drift with the clock
        for _, fn in variants:
            fn()
        times = {name: [] for name, _ in variants}
        for r in range(rounds):
            for j in range(len(variants)):
                name, fn = variants[(j + r) % len(variants)]
                times[name].append(timed(fn))
        return {name + "_ms": round(sorted(t)[rounds // 2], 4) for name, t in times.items()}

    Kp, Np, Mp = df.round16(C), df.round16(N), df.round16(M)
    sc = torch.empty(8, dtype=torch.float32, device=dev)
    p = sc.data_ptr()
    # ---- forward: fc1
    xq, _, sx = operand((M, C), 1.0, 1710, Fmt.E4M3, True, False)
    wq, _, sw = operand((N, C), 0.02, 1711, Fmt.E4M3, True, False)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    q = torch.empty((M, Np), dtype=torch.uint8, device=dev)
    qt = torch.empty((N, Mp), dtype=torch.uint8, device=dev)
    gws_b = max(int(L.df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, C)), int(L.df_fp8_gemm_workspace_bytes(M, N, C)),
                int(L.df_absmax_workspace_bytes()), int(L.df_quantize_2d_jit_workspace_bytes(M, N, 1)),
                int(L.df_fp8_gemm_bwd_absmax_workspace_bytes(M, C, N)))
    gws = torch.empty(gws_b, dtype=torch.uint8, device=dev)

    def gemm():
        df.call("df_fp8_gemm_fwd", xq.data_ptr(), Kp, wq.data_ptr(), Kp, M, N, C, sx.data_ptr(), sw.data_ptr(),
                F32, None, BF, y.data_ptr(), N, gws.data_ptr(), gws_b, stream)

    def absmax():
        df.call("df_absmax_scale_bf16", y.data_ptr(), y.numel(), E4, None, p, gws.data_ptr(), gws_b, stream)

    def fused_gemm():
        df.call("df_fp8_gemm_fwd_absmax", xq.data_ptr(), Kp, wq.data_ptr(), Kp, M, N, C, sx.data_ptr(),
                sw.data_ptr(), F32, None, BF, y.data_ptr(), N, E4, None, p, gws.data_ptr(), gws_b, stream)

    def quant():
        df.call("df_quantize_2d", BF, y.data_ptr(), M, N, N, E4, p, q.data_ptr(), Np, qt.data_ptr(), Mp, stream)

    def quant_jit():
        df.call("df_quantize_2d_jit", BF, y.data_ptr(), M, N, E4, None, p, q.data_ptr(), Np, qt.data_ptr(), Mp,
                None, gws.data_ptr(), gws_b, stream)

    fwd = {"shape": [M, C, N], "y_dtype": "bf16"}
    fwd.update(rotated((("gemm", gemm), ("absmax_pass", absmax), ("gemm_absmax", fused_gemm), ("quantize", quant),
                        ("unfused", lambda: (gemm(), absmax(), quant())),
                        ("unfused_jit", lambda: (gemm(), quant_jit())),
                        ("fused", lambda: (fused_gemm(), quant())))))
    fwd["epilogue_fold_ms"] = round(fwd["gemm_absmax_ms"] - fwd["gemm_ms"], 4)  # with the partials' fold
    fwd["absmax_pass_gbs"] = round(M * N * 2 / (fwd["absmax_pass_ms"] * 1e-3) / 1e9, 1)
    fwd["saved_ms"] = round(fwd["unfused_ms"] - fwd["fused_ms"], 4)
    fwd["saved_vs_jit_ms"] = round(fwd["unfused_jit_ms"] - fwd["fused_ms"], 4)
    del xq, wq
    # ---- backward: fc2 (dY [M, C] e5m2, W [C, N] e4m3, X = fc1's Y [M, N]); dX [M, N] is fc1's dY
    dyq, dyt, sdy = operand((M, C), 1e-3, 1712, Fmt.E5M2, True, True)
    _, wt, sw2 = operand((C, N), 0.02, 1713, Fmt.E4M3, False, True)
    _, xt, sx2 = operand((M, N), 1.0, 1714, Fmt.E4M3, False, True)
    dX = y  # [M, N] bf16
    dW = torch.empty((C, N), dtype=torch.float32, device=dev)
    db = torch.empty(N, dtype=torch.float32, device=dev)
    bws_b = int(L.df_fp8_gemm_bwd_workspace_bytes(M, C, N))
    cws = torch.empty(int(L.df_quantize_2d_workspace_bytes(M, N)), dtype=torch.uint8, device=dev)

    def bwd():
        df.call("df_fp8_gemm_bwd", dyq.data_ptr(), dyq.stride(0), wt.data_ptr(), wt.stride(0), dyt.data_ptr(),
                dyt.stride(0), xt.data_ptr(), xt.stride(0), M, C, N, sdy.data_ptr(), sw2.data_ptr(), sx2.data_ptr(),
                BF, dX.data_ptr(), N, F32, dW.data_ptr(), N, gws.data_ptr(), bws_b, stream)

    def absmax_dx():
        df.call("df_absmax_scale_bf16", dX.data_ptr(), dX.numel(), E5, None, p + 4, gws.data_ptr(), gws_b, stream)

    def fused_bwd():
        df.call("df_fp8_gemm_bwd_absmax", dyq.data_ptr(), dyq.stride(0), wt.data_ptr(), wt.stride(0),
                dyt.data_ptr(), dyt.stride(0), xt.data_ptr(), xt.stride(0), M, C, N, sdy.data_ptr(), sw2.data_ptr(),
                sx2.data_ptr(), BF, dX.data_ptr(), N, F32, dW.data_ptr(), N, E5, None, p + 4, gws.data_ptr(), gws_b,
                stream)

    def quant_dy():
        df.call("df_quantize_2d_colsum", BF, dX.data_ptr(), M, N, N, E5, p + 4, q.data_ptr(), Np, qt.data_ptr(), Mp,
                db.data_ptr(), cws.data_ptr(), cws.numel(), stream)

    def quant_dy_jit():
        df.call("df_quantize_2d_jit", BF, dX.data_ptr(), M, N, E5, None, p + 4, q.data_ptr(), Np, qt.data_ptr(), Mp,
                db.data_ptr(), gws.data_ptr(), gws_b, stream)

    bw = {"shape": [M, C, N], "dx_dtype": "bf16", "dw_dtype": "fp32",
          "grouped_plan": list(df.gemm_bwd_plan(M, C, N))}
    bw.update(rotated((("gemm_bwd", bwd), ("absmax_pass", absmax_dx), ("gemm_bwd_absmax", fused_bwd),
                       ("quantize_colsum", quant_dy),
                       ("unfused", lambda: (bwd(), absmax_dx(), quant_dy())),
                       ("unfused_jit", lambda: (bwd(), quant_dy_jit())),
                       ("fused", lambda: (fused_bwd(), quant_dy())))))
    bw["epilogue_fold_ms"] = round(bw["gemm_bwd_absmax_ms"] - bw["gemm_bwd_ms"], 4)
    bw["saved_ms"] = round(bw["unfused_ms"] - bw["fused_ms"], 4)
    bw["saved_vs_jit_ms"] = round(bw["unfused_jit_ms"] - bw["fused_ms"], 4)
    return {"note": f"median of {rounds} rotated rounds of {reps} calls", "forward": fwd, "backward": bw}


def optimizer_bench(torch, df, dev, stream, layers=48, reps=5):
    """Consumer side of dW over the GPT-2 XL stack's Linear parameters
    (48 x {qkv, proj, fc1, fc2} weights and biases, fp32): the global norm,
    clip in place, the Adam update, and the two orders of a clipped step --
    the reference's (clip_grad_norm then Adam::step) and the fused one (norm,
    then Adam applying the clip factor).  HBM bytes per element: norm 4,
    clip 4 + 8, Adam 16 read + 12 written; the clipped orders clip on every
    call."""
    import ctypes
    shapes = []
    for _ in range(layers):
        for _, k, o in XL_LINEARS:
            shapes += [(o, k), (o,)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    P = [torch.randn(s, device=dev, generator=gen) * 0.02 for s in shapes]
    G = [torch.randn(s, device=dev, generator=gen) * 1e-3 for s in shapes]
    M = [torch.zeros(s, device=dev) for s in shapes]
    V = [torch.zeros(s, device=dev) for s in shapes]
    n = sum(t.numel() for t in P)
    cnt = len(P)
    arr = lambda ts: (ctypes.c_void_p * cnt)(*[t.data_ptr() for t in ts])
    pp, gp, mp, vp = arr(P), arr(G), arr(M), arr(V)
    sizes = (ctypes.c_int64 * cnt)(*[t.numel() for t in P])
    wsb = df.lib().df_grad_norm_workspace_bytes(cnt, sizes)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    norm = torch.empty(1, dtype=torch.float32, device=dev)
    step = [0]

    def gnorm():
        df.call("df_grad_norm_f32", gp, sizes, cnt, norm.data_ptr(), ws.data_ptr(), wsb, stream)

    gnorm()
    torch.cuda.synchronize()
    n0 = norm.item()
    calls = [0]

    def clip():
        # every call clips: max_norm is half the norm the previous call left
        # (the k-th call sees norm ~ n0 / 2^k), so each pass rewrites the
        # gradients, as a clipping step of the reference does
        k = calls[0]
        calls[0] += 1
        df.call("df_clip_grad_norm_f32", gp, sizes, cnt, n0 * 0.5 ** (k + 1), norm.data_ptr(), ws.data_ptr(),
                wsb, stream)

    def adam(clip_norm=None):
        step[0] += 1
        df.call("df_adam_update_f32", pp, gp, mp, vp, sizes, cnt, 1e-4, 0.9, 0.999, 1e-8, 0.0, step[0],
                clip_norm, 1.0, stream)

    def fused():
        gnorm()
        adam(norm.data_ptr())

    def reference_order():
        clip()
        adam()

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    res = {"params": n, "tensors": cnt, "layers": layers}
    # context: a plain device-to-device copy of 4 GiB (read + write)
    a = torch.empty(1 << 30, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    ms = timed(lambda: b.copy_(a))
    res["copy_4GiB"] = {"ms": round(ms, 3), "gbs": round(2 * a.numel() * 4 / (ms * 1e-3) / 1e9, 1)}
    del a, b
    for name, fn, bpe in (("grad_norm", gnorm, 4), ("adam", adam, 28), ("clip_then_adam", reference_order, 40),
                          ("fused_clip_adam", fused, 32)):
        ms = timed(fn)
        gbs = n * bpe / (ms * 1e-3) / 1e9
        res[name] = {"ms": round(ms, 3), "bytes_per_param": bpe, "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)}
    res["fused_saving"] = round(1 - res["fused_clip_adam"]["ms"] / res["clip_then_adam"]["ms"], 3)

    # The optimizer step followed by the e4m3 codes of every weight (row and
    # transposed, for the next step's GEMMs): Adam, then the batched
    # quantize with its own absmax pass, against Adam measuring the weights'
    # absmax as it writes them and the batched quantize taking it.  The list
    # puts the weights first so their absmax values are contiguous.
    W = P[0::2]
    order = lambda ts: ts[0::2] + ts[1::2]
    pp2, gp2, mp2, vp2 = arr(order(P)), arr(order(G)), arr(order(M)), arr(order(V))
    sizes2 = (ctypes.c_int64 * cnt)(*[t.numel() for t in order(P)])
    nw = len(W)
    qw = [torch.empty((t.shape[0], df.round16(t.shape[1])), dtype=torch.uint8, device=dev) for t in W]
    qtw = [torch.empty((t.shape[1], df.round16(t.shape[0])), dtype=torch.uint8, device=dev) for t in W]
    am = torch.empty(cnt, dtype=torch.float32, device=dev)
    wsc = torch.empty(nw, dtype=torch.float32, device=dev)
    qws = torch.empty(df.lib().df_quantize_2d_batch_workspace_bytes(), dtype=torch.uint8, device=dev)
    iarr = lambda vals: (ctypes.c_int * nw)(*vals)
    warr = lambda ts: (ctypes.c_void_p * nw)(*[t.data_ptr() for t in ts])
    wargs = (warr(W), iarr([t.shape[0] for t in W]), iarr([t.shape[1] for t in W]), 0)
    codes = (warr(qw), iarr([q.stride(0) for q in qw]), warr(qtw), iarr([q.stride(0) for q in qtw]))

    def adam2(absmax=None):
        step[0] += 1
        a = (pp2, gp2, mp2, vp2, sizes2, cnt, 1e-4, 0.9, 0.999, 1e-8, 0.0, step[0], None, 1.0)
        if absmax is None:
            df.call("df_adam_update_f32", *a, stream)
        else:
            df.call("df_adam_update_absmax_f32", *a, absmax, stream)

    def requant_unfused():
        adam2()
        df.call("df_quantize_2d_batch", int(df.DType.FLOAT32), nw, *wargs, None, wsc.data_ptr(), *codes,
                qws.data_ptr(), qws.numel(), stream)

    def requant_fused():
        adam2(am.data_ptr())
        df.call("df_quantize_2d_batch_absmax", int(df.DType.FLOAT32), nw, *wargs, am.data_ptr(), wsc.data_ptr(),
                *codes, stream)

    nwp = sum(t.numel() for t in W)
    for name, fn, wbytes in (("adam_then_weight_codes", requant_unfused, 4 + 4 + 2),
                             ("adam_absmax_then_weight_codes", requant_fused, 4 + 2)):
        ms = timed(fn)
        byts = n * 28 + nwp * wbytes
        res[name] = {"ms": round(ms, 3), "bytes": byts, "gbs": round(byts / (ms * 1e-3) / 1e9, 1)}
    res["weight_codes_saving"] = round(1 - res["adam_absmax_then_weight_codes"]["ms"]
                                       / res["adam_then_weight_codes"]["ms"], 3)
    del P, G, M, V, W, qw, qtw
    torch.cuda.empty_cache()
    return res


def _tile_column(block, t, grid, tiles_m, tiles_n, group_m=8):
    """Tile column of block `block`'s t-th tile in the unsplit persistent
    kernel: the XCD-aware block remap and the grouped tile order of
    persistent_body (csrc/gemm_fp8.hip), restated on the host."""
    q, rr = grid >> 3, grid & 7
    xcd, idx = block & 7, block >> 3
    bl = xcd * (q + 1) + idx if xcd < rr else rr * (q + 1) + (xcd - rr) * q + idx
    lt = bl + t * grid
    per_group = group_m * tiles_n
    group = lt // per_group
    gsize = min(tiles_m - group * group_m, group_m)
    return (lt - group * per_group) // gsize


def tile_timeline_bench(torch, df, dev, stream, M=M_TOKENS, reps=3):
    """Where a persistent-kernel tile's time goes: the four config-4 forward
    GEMMs (bf16 bias and output) through df_fp8_gemm_fwd_timeline, the same
    kernel body with wave 0 of every block stamping the 100 MHz real-time
    counter at the block's start and at each tile's start, epilogue start
    and epilogue end.  Operands: device-seeded X ~ N(0, 1), W ~ N(0, 0.02)
    codes.  Per shape (the run with the shortest kernel span of `reps`):
    per tile, the main loop (its DMA steps and MFMAs), the epilogue and the
    gap to the block's next tile; per block, the prologue (start to first
    tile) and the end; the main loop per 128-byte K step."""
    import ctypes

    gen = torch.Generator(device=dev)
    out = {"clock": "s_memrealtime, 100 MHz", "M": M, "shapes": {}}
    for i, (name, K, N) in enumerate(XL_LINEARS):
        gen.manual_seed(8100 + i)
        X = (torch.randn((M, K), generator=gen, device=dev)).to(torch.bfloat16)
        W = (torch.randn((N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        b = (torch.randn((N,), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        _, sx = df.absmax_scale(X, df.Fmt.E4M3)
        _, sw = df.absmax_scale(W, df.Fmt.E4M3)
        xq, _ = df.quantize_2d(X, sx, df.Fmt.E4M3, want_qt=False)
        wq, _ = df.quantize_2d(W, sw, df.Fmt.E4M3, want_qt=False)
        del X, W
        Y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        tiles = ((M + 255) // 256) * ((N + 255) // 256)
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        spb = 1 + 3 * -(-tiles // cus)  # the kernel's grid is min(tiles, CUs)
        stamps = torch.zeros(cus * spb, dtype=torch.int64, device=dev)
        grid = ctypes.c_int()
        best = None
        for _ in range(reps + 1):
            stamps.zero_()
            df.call("df_fp8_gemm_fwd_timeline", xq.data_ptr(), xq.stride(0), wq.data_ptr(), wq.stride(0), M, N, K,
                    sx.data_ptr(), sw.data_ptr(), b.data_ptr(), Y.data_ptr(), N, stamps.data_ptr(), spb,
                    ctypes.byref(grid), stream)
            torch.cuda.synchronize()
            st = stamps[:grid.value * spb].view(grid.value, spb).cpu().numpy().astype("int64")
            span = int(st[st > 0].max() - st[:, 0].min())
            if best is None or span < best[0]:
                best = (span, st)
        span, st = best
        us = 0.01  # one tick = 10 ns
        nk = -(-K // 128)
        main, epi, gap, pro, ends, tail = [], [], [], [], [], []
        tiles_m, tiles_n = (M + 255) // 256, (N + 255) // 256
        t0 = st[:, 0].min()
        for b_id, blk in enumerate(st):
            ntl = 0
            while 3 + 3 * ntl < spb and blk[1 + 3 * ntl] > 0:
                ntl += 1
            if ntl == 0:
                continue
            pro.append((blk[1] - blk[0]) * us)
            for t in range(ntl):
                s0, e0, e1 = blk[1 + 3 * t], blk[2 + 3 * t], blk[3 + 3 * t]
                main.append((e0 - s0) * us)
                if N % 256 and _tile_column(b_id, t, grid.value, tiles_m, tiles_n) == tiles_n - 1:
                    tail.append((e0 - s0) * us)
                epi.append((e1 - e0) * us)
                if t + 1 < ntl:
                    gap.append((blk[4 + 3 * t] - e1) * us)
            ends.append((blk[3 * ntl] - t0) * us)

        def med(v):
            v = sorted(v)
            return round(v[len(v) // 2], 3) if v else None

        out["shapes"][name] = {
            "N": N, "K": K, "k_steps": nk, "tiles": tiles, "blocks": grid.value,
            "kernel_span_us": round(span * us, 2),
            "tile_main_loop_us": med(main), "tile_epilogue_us": med(epi), "gap_to_next_tile_us": med(gap),
            "main_loop_per_k_step_us": round(med(main) / nk, 3) if main else None,
            "block_prologue_us": med(pro), "block_end_first_us": round(min(ends), 2),
            "block_end_last_us": round(max(ends), 2),
            "epilogue_share_of_tile": round(med(epi) / (med(main) + med(epi) + (med(gap) or 0.0)), 4),
            # tiles of the last tile column, which is only N % 256 columns wide (None when N % 256 == 0)
            "tail_column_main_loop_us": med(tail), "tail_column_valid_cols": N % 256 or None,
        }
        del xq, wq, Y, stamps
    return out


def _copy_stats(log, nbytes):
    """Summary of a streamer copy log [(start, end) ms]: per-copy duration
    (its copy stream reaching it to its end), time the link was busy (union
    of the copies' intervals) and the rates that follow."""
    if not log:
        return None
    dur = sorted(b - a for a, b in log)
    ivs = sorted(log)
    busy, cur_a, cur_b = 0.0, ivs[0][0], ivs[0][1]
    for a, b in ivs[1:]:
        if a > cur_b:
            busy += cur_b - cur_a
            cur_a, cur_b = a, b
        else:
            cur_b = max(cur_b, b)
    busy += cur_b - cur_a
    span = max(b for _, b in log) - min(a for a, _ in log)
    n = len(log)
    med = dur[n // 2]
    return {"copies": n, "bytes_each": nbytes, "median_copy_ms": round(med, 4),
            "median_copy_gbs": round(nbytes / (med * 1e-3) / 1e9, 2),
            "sum_copy_ms": round(sum(dur), 3), "busy_ms": round(busy, 3), "span_ms": round(span, 3),
            "busy_gbs": round(n * nbytes / (busy * 1e-3) / 1e9, 2),
            "copies_in_flight_avg": round(sum(dur) / busy, 3) if busy > 0 else None}


def flowshop_bound(copy_ms, compute_ms):
    """Shortest time a fixed sequence of entries can take when entry j's
    copy (copy_ms[j], on one link, in order) must end before its compute
    (compute_ms[j], on the GPU, in order) starts, with unlimited buffering:
    max over k of (copies 0..k) + (computes k..end) -- the two-machine flow
    shop's makespan for that order."""
    best, pre = 0.0, 0.0
    suf = [0.0] * (len(compute_ms) + 1)
    for j in range(len(compute_ms) - 1, -1, -1):
        suf[j] = suf[j + 1] + compute_ms[j]
    for k in range(len(copy_ms)):
        pre += copy_ms[k]
        best = max(best, pre + suf[k])
    return best


def config5_compute_bench(torch, dev, layers=48, tokens=8192):
    """Config 5's step once (after one warm-up step) with every layer's
    weights resident in HBM: the kernels of the streamed step, in its order,
    without the copies.  The config-5 MFMA counter run
    (PROFILE_COMMANDS["mfma_config5"]) profiles these dispatches."""
    from deepfuse_amd.stack import StreamedStack

    stack = StreamedStack(torch, dev, layers=layers, tokens=tokens)
    try:
        dev_w = stack.resident_weights()
        stack.resident_step(dev_w)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        stack.resident_step(dev_w)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        del dev_w
        return {"workload": f"config 5 step, {layers} layers, {tokens} tokens, weights resident",
                "ms": round(ms, 3), "tflops": round(stack.step_flops / ms / 1e9, 1)}
    finally:
        stack.close()


def streaming_bench(torch, df, synth, dev, layers=48, tokens=8192, slots=6, steps=2, micro_batches=3,
                    steady_slots=12):
    """Config 5: a 48-layer GPT-2 XL Linear stack (4 Linears per layer) at
    `tokens` tokens, forward then backward, with every layer's e4m3 weight
    codes in pinned host memory: the forward sweep streams W [N, K] per layer,
    the backward sweep (layers in reverse) streams W^T [K, N] for dX, through
    a ring of `slots` device slots filled on the streamer's copy streams while
    earlier layers compute (deepfuse_amd.stack.StreamedStack, the same code
    tests/test_gpu_stream.py checks).  Per layer and Linear the step
    quantizes the layer's own activation (e4m3, row copy + the transposed copy
    cached for dW) and upstream gradient (e5m2, both copies, db fused), and
    runs the forward, dX and dW GEMMs; dW is kept per layer (fp32).

    Also timed: the same step with all weights resident in HBM (compute
    alone, with a HIP event per layer entry) and the 2*layers weight copies
    alone on the copy streams (PCIe alone), every copy timed by HIP events on
    its copy stream (df_streamer_set_timing).  overlap = max(compute,
    copies) / streamed; bound = the flow-shop makespan of the entry order from
    the measured per-entry copy and compute times (the forward sweep is
    PCIe-bound and the backward compute-bound, so one step cannot reach
    max(compute, copies)); steady state = micro_batches passes back to back
    with the same weights, loads running ahead across passes through
    steady_slots slots; compute under copies = the resident step while the
    2*layers copies run on the copy streams beside it."""
    from deepfuse_amd.stack import StreamedStack

    stack = StreamedStack(torch, dev, layers=layers, tokens=tokens)
    try:
        def timed(fn, reps):
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / reps, (time.perf_counter() - t0) * 1e3 / reps

        streamer = df.WeightStreamer(slots, stack.blob)
        stack.streamed_step(streamer)  # warm-up
        stream_ms, stream_wall = timed(lambda: stack.streamed_step(streamer), steps)
        # one more streamed step with every copy timed on its copy stream
        streamer.set_timing(True)
        stack.streamed_step(streamer)
        torch.cuda.synchronize()
        stream_copies = _copy_stats(streamer.copy_log(), stack.blob)
        streamer.set_timing(False)
        # steady state: micro_batches passes with the same weights
        steady = df.WeightStreamer(steady_slots, stack.blob)
        stack.streamed_step(steady)
        mb_ms, _ = timed(lambda: stack.streamed_step(steady, micro_batches), 1)
        steady.close()

        # PCIe alone: the same 2*layers loads with no kernels; the idle
        # compute stream waits for each slot's copy and releases it (the
        # streamer's copies alternate between its two copy streams)
        cur = torch.cuda.current_stream().cuda_stream

        def copies_only():
            for d, l in stack.seq:
                slot, _ = streamer.load(stack.host_ptr + stack.host_offset(l, d), stack.blob)
                streamer.wait(slot, cur)
                streamer.release(slot, cur)

        torch.cuda.synchronize()
        streamer.set_timing(True)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        copies_only()
        e1.record()
        torch.cuda.synchronize()
        h2d_ms = e0.elapsed_time(e1)
        alone_log = streamer.copy_log()
        alone_copies = _copy_stats(alone_log, stack.blob)
        streamer.close()
        # per-entry copy time for the bound: one copy's bytes at the better
        # of the two link rates measured (busy time of the copies alone and
        # of the streamed step's copies; the link ran at different rates in
        # the two on some boxes)
        link_gbs = max(alone_copies["busy_gbs"], stream_copies["busy_gbs"])
        copy_each = [stack.blob / (link_gbs * 1e9) * 1e3] * len(stack.seq)

        # compute alone: weights resident in HBM (one device copy of the
        # blobs), a HIP event before every entry
        dev_w = stack.resident_weights()
        stack.resident_step(dev_w)
        compute_ms, compute_wall = timed(lambda: stack.resident_step(dev_w), steps)
        torch.cuda.synchronize()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(len(stack.seq) + 1)]
        for j, (d, l) in enumerate(stack.seq):
            evs[j].record()
            stack.resident_entry(dev_w, d, l)
        evs[-1].record()
        torch.cuda.synchronize()
        compute_each = [evs[j].elapsed_time(evs[j + 1]) for j in range(len(stack.seq))]
        # the resident step with the 2*layers copies running beside it (the
        # copies wait on and release their slots on a side stream, so the
        # compute stream never waits for them): what concurrent copies cost
        # the kernels themselves
        side = torch.cuda.Stream()
        beside = df.WeightStreamer(slots, stack.blob)
        torch.cuda.synchronize()
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        c0.record()
        stack.resident_step(dev_w)
        c1.record()
        for d, l in stack.seq:
            slot, _ = beside.load(stack.host_ptr + stack.host_offset(l, d), stack.blob)
            beside.wait(slot, side.cuda_stream)
            beside.release(slot, side.cuda_stream)
        torch.cuda.synchronize()
        beside.close()
        under_copies_ms = c0.elapsed_time(c1)
        # the same resident step replayed from a HIP graph: no host launch gaps
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            stack.resident_step(dev_w)
        graph.replay()
        compute_graph_ms, _ = timed(graph.replay, steps)
        del graph, dev_w
        bound_ms = flowshop_bound(copy_each, compute_each)
        h2d_bytes = 2 * layers * stack.blob
        step_flops = stack.step_flops
        half = len(stack.seq) // 2
        return {
            "workload": f"config 5: {layers}-layer GPT-2 XL Linear stack, {tokens} tokens, fwd+bwd, e4m3 weights "
                        f"streamed from pinned host memory through {slots} device slots; every layer has its own "
                        f"activations and gradients",
            "value": round(step_flops / (stream_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
            "ms_per_step": round(stream_ms, 3), "host_ms_per_step": round(stream_wall, 3),
            "step_gemm_flops": step_flops,
            "compute_alone_ms": round(compute_ms, 3), "compute_alone_host_ms": round(compute_wall, 3),
            "compute_alone_tflops": round(step_flops / (compute_ms * 1e-3) / 1e12, 2),
            "compute_alone_graph_ms": round(compute_graph_ms, 3),
            "compute_under_copies_ms": round(under_copies_ms, 3),
            "compute_fwd_sweep_ms": round(sum(compute_each[:half]), 3),
            "compute_bwd_sweep_ms": round(sum(compute_each[half:]), 3),
            "h2d_alone_ms": round(h2d_ms, 3), "h2d_gbs": round(h2d_bytes / (h2d_ms * 1e-3) / 1e9, 2),
            "h2d_bytes_per_step": h2d_bytes, "copy_bytes": stack.blob, "copies_per_step": 2 * layers,
            "copies_alone": alone_copies, "copies_streamed": stream_copies,
            "bound": "pcie" if h2d_ms > compute_ms else "compute",
            "overlap": round(max(h2d_ms, compute_ms) / stream_ms, 4),
            "flowshop_bound_ms": round(bound_ms, 3), "overlap_vs_flowshop_bound": round(bound_ms / stream_ms, 4),
            "flowshop_link_gbs": link_gbs,
            "overlap_vs_compute_under_copies": round(max(h2d_ms, under_copies_ms) / stream_ms, 4),
            "steady_state": {"micro_batches": micro_batches, "slots": steady_slots,
                             "ms_per_pass": round(mb_ms / micro_batches, 3),
                             "overlap_vs_compute_under_copies": round(max(h2d_ms, under_copies_ms) /
                                                                      (mb_ms / micro_batches), 4),
                             "tflops": round(step_flops / (mb_ms / micro_batches * 1e-3) / 1e12, 2),
                             "overlap": round(max(h2d_ms, compute_ms) / (mb_ms / micro_batches), 4),
                             "note": "passes with the same weights (gradient accumulation), loads running ahead "
                                     "across pass boundaries; each pass overwrites dW as the reference's backward "
                                     "does"},
            "steps": steps,
        }
    finally:
        stack.close()


def cpu_baseline(tokens):
    """The reference's host path timed on this host, as the CPU baseline:
    plain C restatements of the reference's FC loops -- (i) the GTest helper's
    bias-first forward (tests/layers/fully_connected_layer_test.cu:29-46;
    its backward helpers are the kernel's loop order for dX and a one-sample
    outer product for dW), (ii) the kernel-order forward, dX and dW
    (dnn/layers/fully_connected_layer.cu:29-35,54-59,78-83) -- and the
    conversion contract (absmax, e4m3 quantize, dequantize), built with
    -O3 -march=native for this host's CPU (make -C oracle native; falls back
    to the -O2 oracle build if the compiler is unavailable).  Each runs on
    one thread and on every core this process may use; `tokens` is the token
    slice of configs 3 and 4 on all cores (single-thread config 4 uses an
    eighth of it).  Config 1 and config 2 run in full."""
    import subprocess
    import tempfile

    import numpy as np

    from deepfuse_amd import synth
    from oracle import pyoracle as orc

    root = os.path.dirname(os.path.abspath(__file__))
    build = "-O3 -march=native (make -C oracle native)"
    tmp = tempfile.mkdtemp(prefix="df_cpu_baseline_")
    out = os.path.join(tmp, "libdf_oracle_native.so")
    try:
        subprocess.run(["make", "-s", "-C", os.path.join(root, "oracle"), "native", f"NATIVE_OUT={out}"],
                       check=True, timeout=120, capture_output=True)
        L = orc.load(out)
    except (OSError, subprocess.SubprocessError):
        build = "-O2 -ffp-contract=off (the oracle build; the native build failed)"
        L = orc.lib()
    hw = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = hw
    omp = os.environ.get("OMP_NUM_THREADS")
    all_threads = max(1, min(avail, int(omp))) if omp and omp.isdigit() else avail
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    P = lambda a: a.ctypes.data

    def best(fn, reps):
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return min(t)

    def fc_case(N, K, O, seed, threads, reps, backward):
        X = synth.normal((N, K), 1.0, seed=seed)
        W = synth.normal((O, K), 0.02, seed=seed + 1)
        b = synth.normal((O,), 0.02, seed=seed + 2)
        Y = np.empty((N, O), np.float32)
        r = {}
        fl = 2.0 * N * K * O
        t = best(lambda: L.dfo_fc_forward(P(X), P(W), P(b), P(Y), N, K, O, threads), reps)
        r["fwd_kernel_order"] = fl / t / 1e9
        t = best(lambda: L.dfo_fc_forward_bias_first(P(X), P(W), P(b), P(Y), N, K, O, threads), reps)
        r["fwd_gtest_bias_first"] = fl / t / 1e9
        if backward:
            dY = synth.normal((N, O), 1e-3, seed=seed + 3)
            dX = np.empty((N, K), np.float32)
            dW = np.empty((O, K), np.float32)
            t = best(lambda: (L.dfo_fc_backward_input(P(dY), P(W), P(dX), N, K, O, threads),
                              L.dfo_fc_backward_weights(P(dY), P(X), P(dW), N, K, O, threads)), reps)
            r["bwd_dx_dw_kernel_order"] = 2 * fl / t / 1e9
        return r, fl

    res = {"build": build, "hardware_concurrency": hw, "cores_available": avail, "threads_all": all_threads,
           "cpu": model, "unit": "GFLOP/s (FC) or GB/s (conversion), best of the repetitions"}
    # config 1: 64 x 768 -> 3072, in full
    for th in (1, all_threads):
        r, _ = fc_case(64, 768, 3072, synth.SEED_BASE + 1, th, 5, False)
        res[f"config1_{th}t"] = {k: round(v, 2) for k, v in r.items()}
    # config 3: the four GPT-2 small Linears, forward, on a token slice
    for th, n_tok, reps in ((1, tokens, 1), (all_threads, tokens, 3)):
        agg = {}
        for i, (_, K, N) in enumerate(SMALL_LINEARS):
            r, fl = fc_case(n_tok, K, N, synth.SEED_BASE + 3 + 10 * i, th, reps, False)
            for k, v in r.items():
                agg.setdefault(k, [0.0, 0.0])
                agg[k][0] += fl
                agg[k][1] += fl / (v * 1e9)
        res[f"config3_{th}t"] = {"tokens": n_tok, **{k: round(a / b / 1e9, 2) for k, (a, b) in agg.items()}}
    # config 4: the four GPT-2 XL Linears, forward and backward
    c4_flops = c4_time = 0.0
    for th, n_tok, reps in ((1, max(tokens // 8, 16), 1), (all_threads, tokens, 2)):
        agg = {}
        for i, (_, K, N) in enumerate(XL_LINEARS):
            r, fl = fc_case(n_tok, K, N, synth.SEED_BASE + 4 + 10 * i, th, reps, True)
            for k, v in r.items():
                w = 2 * fl if k.startswith("bwd") else fl
                agg.setdefault(k, [0.0, 0.0])
                agg[k][0] += w
                agg[k][1] += w / (v * 1e9)
        res[f"config4_{th}t"] = {"tokens": n_tok, **{k: round(a / b / 1e9, 2) for k, (a, b) in agg.items()}}
        if th == all_threads:
            c4_flops = agg["fwd_kernel_order"][0] + agg["bwd_dx_dw_kernel_order"][0]
            c4_time = agg["fwd_kernel_order"][1] + agg["bwd_dx_dw_kernel_order"][1]
    # config 2: the conversion contract on the full 2^28-element fp32 tensor, e4m3
    n = 1 << 28
    x = synth.conversion_input(n)
    q = np.empty(n, np.uint8)
    d = np.empty(n, np.float32)
    conv = {"n": n, "input": "config-2 fp32 tensor (outliers, +-inf, NaN, subnormals)", "fmt": "e4m3"}
    t = best(lambda: L.dfo_absmax_f32(P(x), n), 1)
    am = L.dfo_absmax_f32(P(x), n)
    conv["absmax_1t"] = round(4 * n / t / 1e9, 3)
    sc = L.dfo_scale(am, orc.E4M3)
    t = best(lambda: L.dfo_quantize_f32(P(x), n, sc, orc.E4M3, P(q)), 1)
    conv["quantize_1t"] = round(5 * n / t / 1e9, 3)
    chunk = (n + all_threads - 1) // all_threads

    def quant_all():
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(all_threads) as ex:
            list(ex.map(lambda j: L.dfo_quantize_f32(P(x) + 4 * j * chunk, min(chunk, n - j * chunk), sc,
                                                     orc.E4M3, P(q) + j * chunk), range(all_threads)))

    t = best(quant_all, 2)
    conv[f"quantize_{all_threads}t"] = round(5 * n / t / 1e9, 3)
    t = best(lambda: L.dfo_dequantize_f32(P(q), n, sc, orc.E4M3, P(d)), 1)
    conv["dequantize_1t"] = round(5 * n / t / 1e9, 3)
    res["config2"] = conv
    del x, q, d
    value = c4_flops / c4_time / 1e12
    return {"value": round(value, 5), "unit": "TFLOP/s", "cores": all_threads, "kind": "port",
            "cpu": model, "hardware_concurrency": hw, "build": build,
            "sample": f"kernel-order FC loops (the reference's fully_connected_layer.cu:29-35,54-59,78-83, "
                      f"restated in C), fwd + dX + dW of the 4 GPT-2 XL Linears on a {tokens}-token slice of "
                      f"config 4, {all_threads} threads ({hw} hardware threads on this host); per-config and "
                      f"single-thread figures in `detail`",
            "detail": res}

if __name__ == "__main__":
    main()
