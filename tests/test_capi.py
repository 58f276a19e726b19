"""The C-ABI library loads, exports every symbol include/df_capi.h declares,
and rejects bad arguments with status codes before touching a GPU
(CPU only: none of these calls launches a kernel)."""
import ctypes

import pytest

import deepfuse_amd as df
from deepfuse_amd import DType, Fmt


def test_exports_every_header_symbol():
    L = df.lib()
    names = df.header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(df._SIGS), "ctypes signature table and header disagree"


def test_version_and_sizes():
    L = df.lib()
    assert L.df_version() == 100
    assert L.df_absmax_workspace_bytes() >= 1024
    assert L.df_quantize_2d_workspace_bytes(16384, 6400) == 128 * 6400 * 4
    assert L.df_quantize_2d_workspace_bytes(0, 10) == 0
    # split-K workspace only for outputs too small to fill the GPU
    assert L.df_fp8_gemm_workspace_bytes(16384, 4800, 1600) == 0
    assert L.df_fp8_gemm_workspace_bytes(1600, 1600, 16384) > 0


def status(fn, *args):
    return getattr(df.lib(), fn)(*args)


def err():
    return df.lib().df_last_error_string().decode()


FAKE = 0x1000  # never dereferenced: each call fails its checks first


def test_argument_errors():
    ws_ok = df.lib().df_absmax_workspace_bytes()
    assert status("df_quantize_f32_e4m3", None, -1, None, None, None) == -1
    assert "n < 0" in err()
    assert status("df_quantize_f32_e4m3", None, 5, None, None, None) == -1
    assert status("df_quantize_f32_e4m3", FAKE + 4, 5, FAKE, FAKE, None) == -4  # misaligned x
    assert status("df_quantize_f32_e4m3", None, 0, None, None, None) == 0  # empty is fine
    assert status("df_dequantize_e4m3_f32", FAKE, 8, FAKE, FAKE + 8, None) == -4
    assert status("df_absmax_f32", FAKE, 8, FAKE, None, ws_ok, None) == -5  # no workspace
    assert status("df_absmax_f32", FAKE, 8, FAKE, FAKE, 16, None) == -5      # too small
    assert status("df_absmax_scale_f32", FAKE, 8, 7, FAKE, FAKE, FAKE, ws_ok, None) == -2  # bad format
    assert status("df_compute_scale", FAKE, 3, FAKE, None) == -2
    # 2-D quantize: ld rules
    assert status("df_quantize_2d", int(DType.FLOAT32), FAKE, 4, 20, 20, 0, FAKE, FAKE, 20, None, 0, None) == -4
    assert status("df_quantize_2d", int(DType.INT8), FAKE, 4, 4, 4, 0, FAKE, FAKE, 16, None, 0, None) == -2
    assert status("df_quantize_2d", int(DType.FLOAT32), FAKE, 4, 4, 3, 0, FAKE, FAKE, 16, None, 0, None) == -1
    assert status("df_quantize_2d_colsum", int(DType.FLOAT32), FAKE, 4, 4, 4, 0, FAKE, None, 0, None, 0,
                  FAKE, None, 0, None) == -5
    # GEMM
    g = df.lib().df_fp8_gemm_nt
    assert g(0, FAKE, 16, 0, FAKE, 16, 4, 4, 32, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == -4  # ld < K
    assert g(0, FAKE, 24, 0, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == -4  # ld % 16
    assert g(0, FAKE + 8, 16, 0, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == -4
    assert g(0, FAKE, 16, 3, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == -2
    assert g(0, FAKE, 16, 0, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, int(DType.INT8), FAKE, 4, None, 0, None) == -2
    # an f16 bias goes with an f16 output only; a bf16 bias not with an f16 output
    assert g(0, FAKE, 16, 0, FAKE, 16, 4, 4, 16, FAKE, FAKE, int(DType.HALF), FAKE, 0, FAKE, 4, None, 0, None) == -2
    assert g(0, FAKE, 16, 0, FAKE, 16, 4, 4, 16, FAKE, FAKE, int(DType.BFLOAT16), FAKE, int(DType.HALF), FAKE, 4,
             None, 0, None) == -2
    assert g(0, FAKE, 16, 0, FAKE, 16, 4, 5, 16, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == -1  # ldc < N
    assert g(0, FAKE, 16, 0, FAKE, 16, -1, 4, 16, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == -1
    assert g(0, FAKE, 16, 0, FAKE, 16, 0, 4, 16, FAKE, FAKE, 0, None, 0, FAKE, 4, None, 0, None) == 0  # M = 0
    # forward GEMM with Y's absmax: bf16 / f16 / fp32 Y only, a known format, an output, contiguous Y
    fa = df.lib().df_fp8_gemm_fwd_absmax
    bf, f32 = int(DType.BFLOAT16), int(DType.FLOAT32)
    assert fa(FAKE, 16, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, int(DType.INT8), FAKE, 4, 0, FAKE, FAKE, FAKE,
              4096, None) == -2
    assert fa(FAKE, 16, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, bf, FAKE, 4, 7, FAKE, FAKE, FAKE, 4096, None) == -2
    assert fa(FAKE, 16, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, bf, FAKE, 4, 0, None, None, FAKE, 4096, None) == -1
    assert fa(FAKE, 16, FAKE, 16, 4, 4, 16, FAKE, FAKE, 0, None, f32, FAKE, 8, 0, FAKE, None, FAKE, 4096, None) == -1
    assert "contiguous" in err()
    assert df.lib().df_fp8_gemm_fwd_absmax_workspace_bytes(16384, 6400, 1600) >= 64 * 25 * 8 * 4
    # backward with dX's absmax: bf16 / f16 / fp32 dX, a known format, an output, contiguous dX, room for the
    # partials
    ba = lambda dxt, lddx, fmt, am, sc, wsb: status(
        "df_fp8_gemm_bwd_absmax", FAKE, 16, FAKE, 16, FAKE, 16, FAKE, 16, 16, 16, 16, FAKE, FAKE, FAKE, dxt, FAKE, lddx,
        f32, FAKE, 16, fmt, am, sc, FAKE, wsb, None)
    assert ba(int(DType.INT8), 16, 1, FAKE, FAKE, 1 << 20) == -2
    assert ba(bf, 16, 9, FAKE, FAKE, 1 << 20) == -2
    assert ba(bf, 16, 1, None, None, 1 << 20) == -1
    assert ba(f32, 32, 1, FAKE, None, 1 << 20) == -1
    assert "contiguous" in err()
    assert ba(bf, 16, 1, None, FAKE, 1024) == -5
    # tensor utilities
    assert status("df_fill", FAKE, 4, 3, ctypes.byref(ctypes.c_int(0)), None) == -2
    assert status("df_add", 99, FAKE, FAKE, FAKE, 4, None) == -2
    assert status("df_approx_equal_mask", int(DType.FP8E4M3), FAKE, FAKE, FAKE, 4, 0.1, None) == -2
    # clip / Adam lists
    P = ctypes.c_void_p
    sizes = (ctypes.c_int64 * 3)(32768, 32769, 0)  # 32768-element partial blocks
    assert df.lib().df_grad_norm_workspace_bytes(3, sizes) == 3 * 8
    assert df.lib().df_grad_norm_workspace_bytes(0, None) == 8
    ptrs = (P * 3)(FAKE, FAKE + 16, None)  # the empty entry may be NULL
    assert status("df_grad_norm_f32", ptrs, sizes, 3, FAKE, FAKE, 16, None) == -5
    assert status("df_grad_norm_f32", ptrs, sizes, 3, FAKE, FAKE + 4, 64, None) == -4  # ws alignment
    bad = (P * 3)(FAKE, FAKE + 4, None)
    assert status("df_clip_grad_norm_f32", bad, sizes, 3, 1.0, FAKE, FAKE, 64, None) == -4
    neg = (ctypes.c_int64 * 1)(-1)
    assert status("df_grad_norm_f32", ptrs, neg, 1, FAKE, FAKE, 64, None) == -1
    nul = (P * 1)(None)
    one = (ctypes.c_int64 * 1)(4)
    assert status("df_adam_update_f32", nul, nul, nul, nul, one, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1,
                  None, 0.0, None) == -1
    ok = (P * 1)(FAKE)
    assert status("df_adam_update_f32", ok, ok, ok, ok, one, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0,
                  None, 0.0, None) == -1
    assert "timestep" in err()
    assert status("df_adam_update_f32", ok, ok, (P * 1)(FAKE + 8), ok, one, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1,
                  None, 0.0, None) == -4
    # just-in-time quantize: scale output required, x aligned, codes asked for, workspace size
    BF = int(DType.BFLOAT16)
    wb = df.lib().df_quantize_2d_jit_workspace_bytes(64, 64, 0)
    assert wb >= 2048 * 4 and df.lib().df_quantize_2d_jit_workspace_bytes(256, 64, 1) >= wb + 2 * 64 * 4
    jit = lambda *a: status("df_quantize_2d_jit", BF, *a)
    assert jit(FAKE, 64, 64, 0, FAKE, None, FAKE, 64, None, 0, None, FAKE, wb, None) == -1  # no scale output
    assert jit(FAKE + 2, 64, 64, 0, None, FAKE, FAKE, 64, None, 0, None, FAKE, wb, None) == -4
    assert jit(FAKE, 64, 64, 0, None, FAKE, None, 0, None, 0, FAKE, FAKE, wb, None) == -1  # column sums only
    assert jit(FAKE, 64, 64, 3, None, FAKE, FAKE, 64, None, 0, None, FAKE, wb, None) == -2
    assert jit(FAKE, 64, 64, 0, None, FAKE, FAKE, 64, None, 0, None, FAKE, wb - 4, None) == -5
    assert jit(FAKE, 64, 64, 0, None, FAKE, FAKE, 64, None, 0, FAKE, FAKE, wb, None) == -5  # + column sums


def test_error_raises_in_python_binding():
    with pytest.raises(df.DFError) as ei:
        df.call("df_quantize_bf16_e5m2", None, -3, None, None, None)
    assert ei.value.status == -1
    assert "n < 0" in str(ei.value)


def test_enums_mirror_reference():
    """OnnxLoader::DType (dnn/utils/onnx_loader.cuh:16-22) values 0-4 kept."""
    assert [DType.FLOAT32, DType.HALF, DType.INT8, DType.UINT8, DType.BFLOAT16] == [0, 1, 2, 3, 4]
    assert (DType.FP8E4M3, DType.FP8E5M2) == (5, 6)
    assert (Fmt.E4M3, Fmt.E5M2) == (0, 1)


def test_grouped_backward_and_batch_argument_errors():
    F32, BF16 = int(DType.FLOAT32), int(DType.BFLOAT16)
    # df_fp8_gemm_bwd checks both problems before planning: misaligned dY codes, bad ld, bad dtype
    args = [FAKE, 32, FAKE, 32, FAKE, 64, FAKE, 64, 64, 32, 32, FAKE, FAKE, FAKE, F32, FAKE, 32, F32, FAKE, 32,
            None, 0, None]
    bad = list(args)
    bad[0] = FAKE + 4
    assert status("df_fp8_gemm_bwd", *bad) == -4 and "(dX)" in err()
    bad = list(args)
    bad[5] = 24  # ldyt not a multiple of 16
    assert status("df_fp8_gemm_bwd", *bad) == -4 and "(dW)" in err()
    bad = list(args)
    bad[17] = int(DType.INT8)  # dW dtype
    assert status("df_fp8_gemm_bwd", *bad) == -2
    g, sl = ctypes.c_int(7), ctypes.c_int(7)
    assert status("df_fp8_gemm_bwd_plan", 0, 10, 10, 0, ctypes.byref(g), ctypes.byref(sl)) == 0
    assert (g.value, sl.value) == (0, 0)
    assert status("df_fp8_gemm_bwd_plan", 1, 1, 1, 0, None, None) == -1
    # df_quantize_2d_batch
    one_p = (ctypes.c_void_p * 1)(FAKE)
    one_i = (ctypes.c_int * 1)(16)
    ws_b = df.lib().df_quantize_2d_batch_workspace_bytes()
    assert status("df_quantize_2d_batch", BF16, 0, None, None, None, 0, None, None, None, None, None, None, None, 0,
                  None) == 0  # nothing to do
    assert status("df_quantize_2d_batch", BF16, -1, None, None, None, 0, None, None, None, None, None, None, None,
                  0, None) == -1
    assert status("df_quantize_2d_batch", BF16, 1, one_p, one_i, one_i, 0, None, None, one_p, one_i, None, None,
                  FAKE, ws_b, None) == -1  # no scale output
    assert status("df_quantize_2d_batch", BF16, 1, one_p, one_i, one_i, 0, None, FAKE, one_p, one_i, None, None,
                  None, 0, None) == -5  # no workspace
    assert status("df_quantize_2d_batch", int(DType.HALF), 1, one_p, one_i, one_i, 0, None, FAKE, one_p, one_i,
                  None, None, FAKE, ws_b, None) == -2
    mis = (ctypes.c_void_p * 1)(FAKE + 2)
    assert status("df_quantize_2d_batch", BF16, 1, mis, one_i, one_i, 0, None, FAKE, one_p, one_i, None, None,
                  FAKE, ws_b, None) == -4 and "tensor 0" in err()
    assert status("df_quantize_2d_batch_absmax", BF16, 1, one_p, one_i, one_i, 0, None, FAKE, one_p, one_i, None,
                  None, None) == -1  # absmax input missing
    # Adam with absmax: the absmax array is required
    one_f = (ctypes.c_void_p * 1)(FAKE)
    one_n = (ctypes.c_int64 * 1)(64)
    assert status("df_adam_update_absmax_f32", one_f, one_f, one_f, one_f, one_n, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0,
                  1, None, 0.0, None, None) == -1


def test_flat_wrappers_refuse_binary16():
    """The flat quantize/dequantize kernels take fp32 and bf16 only; a float16
    tensor is refused on the host rather than sent to the bf16 kernel."""
    import torch
    from deepfuse_amd import Fmt
    with pytest.raises(TypeError):
        df.quantize(torch.zeros(8, dtype=torch.float16), None, Fmt.E4M3)
    with pytest.raises(TypeError):
        df.dequantize(torch.zeros(8, dtype=torch.uint8), None, Fmt.E4M3, torch.float16)


def test_error_message_is_per_thread():
    """df_last_error_string is thread-local: two threads that fail different
    checks at the same time each read their own message (no GPU work: each
    call fails its argument checks first)."""
    import threading
    L = df.lib()
    go = threading.Barrier(2)
    seen = {}

    def worker(tag, fn):
        go.wait()
        rc = fn()
        go.wait()  # both calls have returned before either reads its message
        seen[tag] = (rc, L.df_last_error_string().decode())

    t1 = threading.Thread(target=worker, args=("fmt", lambda: L.df_quantize_2d(
        int(DType.BFLOAT16), FAKE, 4, 4, 4, 9, FAKE, FAKE, 16, None, 0, None)))
    t2 = threading.Thread(target=worker, args=("n", lambda: L.df_quantize_bf16_e5m2(None, -3, None, None, None)))
    t1.start(); t2.start(); t1.join(); t2.join()
    assert seen["fmt"][0] == -2 and "format" in seen["fmt"][1]
    assert seen["n"][0] == -1 and "n < 0" in seen["n"][1]
