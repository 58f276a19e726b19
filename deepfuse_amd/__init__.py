"""deepfuse_amd -- MI355X-native fp8 Linear path of DeepFuse, Python side.

The product is the C ABI in ``include/df_capi.h`` implemented by
``deepfuse_amd/libdeepfuse_amd.so`` (hand-written HIP for gfx950).  This module
binds it with ctypes and offers thin helpers over torch device tensors (torch
is only the allocator and stream provider here).  Nothing in this package has
a CPU fallback: if the HIP library is missing, :func:`lib` raises.

Reference mapping (SensorVista/DeepFuse):
  - ``DType`` mirrors ``OnnxLoader::DType`` (dnn/utils/onnx_loader.cuh:16-22),
    extended with the 1-byte fp8 formats.
  - ``fc_forward`` / ``fc_backward`` mirror ``FullyConnectedLayer<T>::forward``
    / ``backward`` (dnn/layers/fully_connected_layer.cu:164-357) in fp8 compute.
"""
from __future__ import annotations

import ctypes
import enum
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdeepfuse_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "df_capi.h")


class DType(enum.IntEnum):
    FLOAT32 = 0
    HALF = 1
    INT8 = 2
    UINT8 = 3
    BFLOAT16 = 4
    FP8E4M3 = 5
    FP8E5M2 = 6
    INT32 = 7


class Fmt(enum.IntEnum):
    E4M3 = 0
    E5M2 = 1


FMAX = {Fmt.E4M3: 448.0, Fmt.E5M2: 57344.0}


class DFError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


_c_int, _c_i64, _c_sz, _c_f = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
_vp = ctypes.c_void_p

# name -> (restype, argtypes); every function declared in df_capi.h
_SIGS = {
    "df_last_error_string": (ctypes.c_char_p, []),
    "df_version": (_c_int, []),
    "df_device_arch_ok": (_c_int, []),
    "df_absmax_workspace_bytes": (_c_sz, []),
    "df_absmax_f32": (_c_int, [_vp, _c_i64, _vp, _vp, _c_sz, _vp]),
    "df_absmax_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _c_sz, _vp]),
    "df_absmax_scale_f32": (_c_int, [_vp, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "df_absmax_scale_bf16": (_c_int, [_vp, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "df_absmax_f16": (_c_int, [_vp, _c_i64, _vp, _vp, _c_sz, _vp]),
    "df_absmax_scale_f16": (_c_int, [_vp, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "df_compute_scale": (_c_int, [_vp, _c_int, _vp, _vp]),
    "df_hbm_probe_dst_bytes": (_c_sz, [_c_int, _c_int, _c_i64]),
    "df_hbm_probe": (_c_int, [_c_int, _c_int, _vp, _c_i64, _vp, _vp]),
    "df_quantize_f32_e4m3": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_quantize_f32_e5m2": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_quantize_bf16_e4m3": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_quantize_bf16_e5m2": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_dequantize_e4m3_f32": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_dequantize_e5m2_f32": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_dequantize_e4m3_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_dequantize_e5m2_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "df_quantize_2d": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int,
                                _vp, _c_int, _vp]),
    "df_quantize_2d_workspace_bytes": (_c_sz, [_c_int, _c_int]),
    "df_quantize_2d_colsum": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int,
                                       _vp, _c_int, _vp, _vp, _c_sz, _vp]),
    "df_quantize_2d_jit_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int]),
    "df_quantize_2d_jit": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _vp,
                                    _vp, _c_sz, _vp]),
    "df_colsum": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_sz, _vp]),
    "df_quantize_2d_batch_workspace_bytes": (_c_sz, []),
    "df_quantize_2d_batch": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _c_sz, _vp]),
    "df_quantize_2d_batch_absmax": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp]),
    "df_fp8_gemm_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int]),
    "df_fp8_gemm_fwd_absmax_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int]),
    "df_fp8_gemm_fwd_absmax": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp,
                                        _c_int, _vp, _c_int, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "df_fp8_gemm_nt": (_c_int, [_c_int, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                                _vp, _vp, _c_int, _vp, _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_fp8_gemm_nt_plan": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _vp, _c_sz, _vp, _vp]),
    "df_fp8_gemm_fwd_timeline": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp,
                                          _c_int, _vp, _c_int, ctypes.POINTER(_c_int), _vp]),
    "df_fp8_gemm_fwd": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                 _c_int, _vp, _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_fp8_gemm_bwd_dx": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                    _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_fp8_gemm_bwd_dw": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                    _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_fp8_gemm_bwd_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int]),
    "df_fp8_gemm_bwd_plan": (_c_int, [_c_int, _c_int, _c_int, _c_sz, _vp, _vp]),
    "df_fp8_gemm_bwd": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                 _vp, _vp, _c_int, _vp, _c_int, _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_fp8_gemm_bwd_absmax_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int]),
    "df_fp8_gemm_bwd_absmax": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                                        _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _vp, _vp,
                                        _vp, _c_sz, _vp]),
    "df_fill": (_c_int, [_vp, _c_i64, _c_int, _vp, _vp]),
    "df_add": (_c_int, [_c_int, _vp, _vp, _vp, _c_i64, _vp]),
    "df_convert": (_c_int, [_c_int, _vp, _c_int, _vp, _c_i64, _vp]),
    "df_equal_mask": (_c_int, [_c_int, _vp, _vp, _vp, _c_i64, _vp]),
    "df_approx_equal_mask": (_c_int, [_c_int, _vp, _vp, _vp, _c_i64, _c_f, _vp]),
    "df_host_alloc": (_c_int, [_c_sz, ctypes.POINTER(_vp)]),
    "df_host_free": (_c_int, [_vp]),
    "df_streamer_create": (_c_int, [_c_int, _c_sz, ctypes.POINTER(_vp)]),
    "df_streamer_destroy": (_c_int, [_vp]),
    "df_streamer_load": (_c_int, [_vp, _vp, _c_sz, ctypes.POINTER(_c_int), ctypes.POINTER(_vp)]),
    "df_streamer_wait": (_c_int, [_vp, _c_int, _vp]),
    "df_streamer_release": (_c_int, [_vp, _c_int, _vp]),
    "df_streamer_slot": (_c_int, [_vp, _c_int, ctypes.POINTER(_vp)]),
    "df_streamer_copy_stream": (_c_int, [_vp, _c_int, ctypes.POINTER(_vp)]),
    "df_streamer_set_timing": (_c_int, [_vp, _c_int]),
    "df_streamer_copy_log": (_c_int, [_vp, _vp, _vp, _c_int, ctypes.POINTER(_c_int)]),
    "df_amax_history_init": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _vp]),
    "df_quantize_2d_delayed_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "df_quantize_2d_delayed": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp,
                                        _c_int, _vp, _c_int, _vp, _vp, _c_sz, _vp]),
    "df_quantize_2d_delayed_noalloc": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                                _c_int, _vp, _c_int, _vp, _c_int, _vp, _vp]),
    "df_layernorm_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int, _c_int]),
    "df_layernorm": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_f, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_layernorm_quantize": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_f, _vp, _c_int, _c_int,
                                       _vp, _vp, _vp, _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "df_layernorm_quantize_delayed": (_c_int, [_c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_f, _vp, _c_int,
                                               _c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _vp, _c_int, _vp, _c_sz,
                                               _vp]),
    "df_grad_norm_workspace_bytes": (_c_sz, [_c_int, _vp]),
    "df_grad_norm_f32": (_c_int, [_vp, _vp, _c_int, _vp, _vp, _c_sz, _vp]),
    "df_clip_grad_norm_f32": (_c_int, [_vp, _vp, _c_int, _c_f, _vp, _vp, _c_sz, _vp]),
    "df_adam_update_f32": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_f, _c_f, _c_f, _c_f, _c_f,
                                    _c_int, _vp, _c_f, _vp]),
    "df_adam_update_absmax_f32": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_f, _c_f, _c_f, _c_f, _c_f,
                                           _c_int, _vp, _c_f, _vp, _vp]),
}

_lib = None


def header_functions() -> list[str]:
    """Names of the functions include/df_capi.h declares."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(df_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    """Load libdeepfuse_amd.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(make -C deepfuse_amd); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, status: int) -> None:
    if status != 0:
        msg = lib().df_last_error_string()
        raise DFError(fn, status, msg.decode() if msg else "")


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))


# ----------------------------------------------------------------------------
# torch helpers (device memory + current stream); the compute is the C ABI
# ----------------------------------------------------------------------------
def _torch():
    import torch
    return torch


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    torch = _torch()
    return torch.cuda.current_stream().cuda_stream


def _in_dtype(t) -> DType:
    torch = _torch()
    if t.dtype == torch.float32:
        return DType.FLOAT32
    if t.dtype == torch.bfloat16:
        return DType.BFLOAT16
    if t.dtype == torch.float16:
        return DType.HALF
    raise TypeError(f"unsupported input dtype {t.dtype}")


_ABSMAX_SCALE = {DType.FLOAT32: "df_absmax_scale_f32", DType.BFLOAT16: "df_absmax_scale_bf16",
                 DType.HALF: "df_absmax_scale_f16"}


_WS = {}


def _ws_key(device, tag: str):
    """Cached workspaces are kept per device and per stream (the current
    torch stream, the one the calls go to).  Calls on different streams
    never share one.  A workspace replaced by a larger one was allocated
    while its stream was current, and only that stream used it, so torch's
    allocator reuses its memory in that stream's order."""
    return (str(device), tag, _stream())


def _workspace(device):
    torch = _torch()
    key = _ws_key(device, "absmax")
    if key not in _WS:
        _WS[key] = torch.empty(lib().df_absmax_workspace_bytes(), dtype=torch.uint8, device=device)
    return _WS[key]


def absmax_scale(x, fmt: Fmt):
    """(absmax, scale) as 1-element fp32 device tensors, contract D1/D2."""
    torch = _torch()
    am = torch.empty(1, dtype=torch.float32, device=x.device)
    sc = torch.empty(1, dtype=torch.float32, device=x.device)
    ws = _workspace(x.device)
    call(_ABSMAX_SCALE[_in_dtype(x)], _ptr(x), x.numel(), int(fmt), _ptr(am), _ptr(sc), _ptr(ws), ws.numel(),
         _stream())
    return am, sc


def quantize(x, scale, fmt: Fmt):
    """Flat quantize of a contiguous fp32/bf16 tensor -> uint8 codes (same shape)."""
    torch = _torch()
    src = {DType.FLOAT32: "f32", DType.BFLOAT16: "bf16"}.get(_in_dtype(x))
    if src is None:  # the flat kernels take fp32 and bf16; df_quantize_2d also binary16
        raise TypeError(f"quantize: {x.dtype} has no flat kernel (use quantize_2d)")
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    fn = f"df_quantize_{src}_{'e4m3' if fmt == Fmt.E4M3 else 'e5m2'}"
    call(fn, _ptr(x), x.numel(), _ptr(scale), _ptr(q), _stream())
    return q


def dequantize(q, scale, fmt: Fmt, out_dtype):
    torch = _torch()
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"dequantize: output {out_dtype} not supported (fp32 or bf16)")
    out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    dst = "f32" if out_dtype == torch.float32 else "bf16"
    fn = f"df_dequantize_{'e4m3' if fmt == Fmt.E4M3 else 'e5m2'}_{dst}"
    call(fn, _ptr(q), q.numel(), _ptr(scale), _ptr(out), _stream())
    return out


def round16(v: int) -> int:
    return (v + 15) // 16 * 16


def _scratch(device, nbytes: int, tag: str):
    torch = _torch()
    key = _ws_key(device, tag)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def quantize_2d(x, scale, fmt: Fmt, want_q=True, want_qt=False, colsum=False):
    """2-D quantize into GEMM operand layout: returns (q [R, ceil16(C)],
    qt [C, ceil16(R)]) with zero padding (either may be None), plus the fp32
    column sums when colsum=True."""
    torch = _torch()
    rows, cols = x.shape
    q = torch.empty((rows, round16(cols)), dtype=torch.uint8, device=x.device) if want_q else None
    qt = torch.empty((cols, round16(rows)), dtype=torch.uint8, device=x.device) if want_qt else None
    ldq = q.shape[1] if q is not None else 0
    ldqt = qt.shape[1] if qt is not None else 0
    if not colsum:
        call("df_quantize_2d", int(_in_dtype(x)), _ptr(x), rows, cols, x.stride(0), int(fmt), _ptr(scale),
             _ptr(q), ldq, _ptr(qt), ldqt, _stream())
        return q, qt
    cs = torch.empty(cols, dtype=torch.float32, device=x.device)
    ws = _scratch(x.device, int(lib().df_quantize_2d_workspace_bytes(rows, cols)), "colsum")
    call("df_quantize_2d_colsum", int(_in_dtype(x)), _ptr(x), rows, cols, x.stride(0), int(fmt),
         _ptr(scale), _ptr(q), ldq, _ptr(qt), ldqt, _ptr(cs), _ptr(ws), ws.numel(), _stream())
    return q, qt, cs


def quantize_2d_jit(x, fmt: Fmt, want_q=True, want_qt=False, colsum=False):
    """absmax, scale and the 2-D quantize at that scale in one call
    (df_quantize_2d_jit): returns (absmax, scale, q, qt), plus the fp32
    column sums when colsum=True; x is contiguous."""
    torch = _torch()
    if not x.is_contiguous():
        raise ValueError("quantize_2d_jit: x must be contiguous")
    rows, cols = x.shape
    am = torch.empty(1, dtype=torch.float32, device=x.device)
    sc = torch.empty(1, dtype=torch.float32, device=x.device)
    q = torch.empty((rows, round16(cols)), dtype=torch.uint8, device=x.device) if want_q else None
    qt = torch.empty((cols, round16(rows)), dtype=torch.uint8, device=x.device) if want_qt else None
    cs = torch.empty(cols, dtype=torch.float32, device=x.device) if colsum else None
    ws = _scratch(x.device, int(lib().df_quantize_2d_jit_workspace_bytes(rows, cols, int(colsum))), "jit")
    call("df_quantize_2d_jit", int(_in_dtype(x)), _ptr(x), rows, cols, int(fmt), _ptr(am), _ptr(sc), _ptr(q),
         q.shape[1] if q is not None else 0, _ptr(qt), qt.shape[1] if qt is not None else 0, _ptr(cs), _ptr(ws),
         ws.numel(), _stream())
    return (am, sc, q, qt, cs) if colsum else (am, sc, q, qt)


def gemm_workspace(M: int, N: int, K: int, device):
    """Device workspace sized so split-K is never limited (cached per device
    and current stream, grown as needed)."""
    torch = _torch()
    nbytes = int(lib().df_fp8_gemm_workspace_bytes(M, N, K))
    key = _ws_key(device, "gemm")
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def gemm_nt(a_q, fmt_a: Fmt, b_q, fmt_b: Fmt, K: int, sa, sb, bias=None, out_dtype=None,
            split_k=True):
    """C[M,N] = (A[M,:K] . B[N,:K]^T) * sa * sb + bias on fp8 MFMA."""
    torch = _torch()
    out_dtype = out_dtype or torch.float32
    M, N = a_q.shape[0], b_q.shape[0]
    c = torch.empty((M, N), dtype=out_dtype, device=a_q.device)
    bias_dt = int(DType.FLOAT32) if bias is None else int(_in_dtype(bias))
    c_dt = int(_in_dtype(c))
    ws = gemm_workspace(M, N, K, a_q.device) if split_k else None
    call("df_fp8_gemm_nt", int(fmt_a), _ptr(a_q), a_q.stride(0), int(fmt_b), _ptr(b_q), b_q.stride(0),
         M, N, K, _ptr(sa), _ptr(sb), bias_dt, _ptr(bias), c_dt, _ptr(c), c.stride(0), _ptr(ws),
         ws.numel() if ws is not None else 0, _stream())
    return c


def gemm_fwd_absmax(x_q, w_q, K: int, sx, sw, bias=None, out_dtype=None, next_fmt: Fmt = Fmt.E4M3):
    """Y = X . W^T * sx * sw + bias (df_fp8_gemm_fwd_absmax): returns (Y,
    absmax of Y as stored, the rule-D1/D2 scale of Y for next_fmt); Y is
    bf16 (default), float16 or fp32."""
    torch = _torch()
    out_dtype = out_dtype or torch.bfloat16
    M, N = x_q.shape[0], w_q.shape[0]
    y = torch.empty((M, N), dtype=out_dtype, device=x_q.device)
    am = torch.empty(1, dtype=torch.float32, device=x_q.device)
    sc = torch.empty(1, dtype=torch.float32, device=x_q.device)
    nbytes = int(lib().df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x_q.device)
    bias_dt = int(DType.FLOAT32) if bias is None else int(_in_dtype(bias))
    call("df_fp8_gemm_fwd_absmax", _ptr(x_q), x_q.stride(0), _ptr(w_q), w_q.stride(0), M, N, K, _ptr(sx), _ptr(sw),
         bias_dt, _ptr(bias), int(_in_dtype(y)), _ptr(y), y.stride(0), int(next_fmt), _ptr(am), _ptr(sc), _ptr(ws),
         ws.numel(), _stream())
    return y, am, sc


class GemmKernel(enum.IntEnum):
    """DF_GEMM_KERNEL_* of include/df_capi.h."""
    PERSISTENT = 0
    TILED_DMA_256 = 1
    TILED_DMA_128 = 2
    TILED_REG_256 = 3
    TILED_REG_128 = 4
    PERSISTENT_NARROW = 5


def gemm_plan(M: int, N: int, K: int, lda: int, ldb: int, bias=None, ws_bytes: int = 0):
    """(GemmKernel, K slices) that df_fp8_gemm_nt takes for these arguments;
    ``bias`` is the bias tensor the call would pass (its alignment counts)."""
    k, s = _c_int(), _c_int()
    call("df_fp8_gemm_nt_plan", M, N, K, lda, ldb, _ptr(bias), ws_bytes, ctypes.byref(k), ctypes.byref(s))
    return GemmKernel(k.value), s.value


def gemm_bwd(dy_q, wt_q, dyt_q, xt_q, M: int, N: int, K: int, sdy, sw, sx, dx_dtype=None, dw_dtype=None,
             workspace=True):
    """dX [M, K] and dW [N, K] of one Linear in one call (df_fp8_gemm_bwd):
    dy_q [M, >=N] and dyt_q [N, >=M] e5m2, wt_q [K, >=N] and xt_q [K, >=M]
    e4m3, as df_quantize_2d writes them."""
    torch = _torch()
    dx_dtype = dx_dtype or torch.float32
    dw_dtype = dw_dtype or torch.float32
    dev = dy_q.device
    dX = torch.empty((M, K), dtype=dx_dtype, device=dev)
    dW = torch.empty((N, K), dtype=dw_dtype, device=dev)
    dt = lambda t: int(_in_dtype(torch.empty(0, dtype=t)))
    ws = None
    if workspace:
        ws = _scratch(dev, max(int(lib().df_fp8_gemm_bwd_workspace_bytes(M, N, K)), 16), "gemm_bwd")
    call("df_fp8_gemm_bwd", _ptr(dy_q), dy_q.stride(0), _ptr(wt_q), wt_q.stride(0), _ptr(dyt_q), dyt_q.stride(0),
         _ptr(xt_q), xt_q.stride(0), M, N, K, _ptr(sdy), _ptr(sw), _ptr(sx), dt(dx_dtype), _ptr(dX), K,
         dt(dw_dtype), _ptr(dW), K, _ptr(ws), ws.numel() if ws is not None else 0, _stream())
    return dX, dW


def quantize_2d_batch(tensors, fmt: Fmt, want_q=True, want_qt=True, absmax=None):
    """df_quantize_2d_batch over contiguous 2-D device tensors (fp32 or
    bf16, one dtype): returns (absmax [count], scale [count], [q], [qt])
    with q [R, ceil16(C)] and qt [C, ceil16(R)] (None where not wanted).
    With ``absmax`` given (device fp32 [count]) the absmax pass is skipped
    (df_quantize_2d_batch_absmax) and that tensor is returned."""
    torch = _torch()
    count = len(tensors)
    dev = tensors[0].device
    am = torch.empty(count, dtype=torch.float32, device=dev) if absmax is None else absmax
    sc = torch.empty(count, dtype=torch.float32, device=dev)
    qs = [torch.empty((t.shape[0], round16(t.shape[1])), dtype=torch.uint8, device=dev) if want_q else None
          for t in tensors]
    qts = [torch.empty((t.shape[1], round16(t.shape[0])), dtype=torch.uint8, device=dev) if want_qt else None
           for t in tensors]
    arr = lambda vals: (_c_int * count)(*vals)
    ptrs = lambda ts: (_vp * count)(*[_ptr(t) for t in ts])
    head = (int(_in_dtype(tensors[0])), count, ptrs(tensors), arr([t.shape[0] for t in tensors]),
            arr([t.shape[1] for t in tensors]), int(fmt), _ptr(am), _ptr(sc))
    tail = (ptrs(qs) if want_q else None, arr([q.stride(0) for q in qs]) if want_q else None,
            ptrs(qts) if want_qt else None, arr([q.stride(0) for q in qts]) if want_qt else None)
    if absmax is None:
        ws = _scratch(dev, int(lib().df_quantize_2d_batch_workspace_bytes()), "qbatch")
        call("df_quantize_2d_batch", *head, *tail, _ptr(ws), ws.numel(), _stream())
    else:
        call("df_quantize_2d_batch_absmax", *head, *tail, _stream())
    return am, sc, qs, qts


def gemm_bwd_absmax(dy_q, wt_q, dyt_q, xt_q, M: int, N: int, K: int, sdy, sw, sx, dx_dtype=None, dw_dtype=None,
                    next_fmt: Fmt = Fmt.E5M2):
    """gemm_bwd whose dX also gives its absmax and the rule-D1/D2 scale for
    next_fmt (df_fp8_gemm_bwd_absmax): returns (dX, dW, absmax, scale)."""
    torch = _torch()
    dx_dtype = dx_dtype or torch.bfloat16
    dw_dtype = dw_dtype or torch.float32
    dev = dy_q.device
    dX = torch.empty((M, K), dtype=dx_dtype, device=dev)
    dW = torch.empty((N, K), dtype=dw_dtype, device=dev)
    am = torch.empty(1, dtype=torch.float32, device=dev)
    sc = torch.empty(1, dtype=torch.float32, device=dev)
    dt = lambda t: int(_in_dtype(torch.empty(0, dtype=t)))
    ws = _scratch(dev, max(int(lib().df_fp8_gemm_bwd_absmax_workspace_bytes(M, N, K)), 16), "gemm_bwd_absmax")
    call("df_fp8_gemm_bwd_absmax", _ptr(dy_q), dy_q.stride(0), _ptr(wt_q), wt_q.stride(0), _ptr(dyt_q),
         dyt_q.stride(0), _ptr(xt_q), xt_q.stride(0), M, N, K, _ptr(sdy), _ptr(sw), _ptr(sx), dt(dx_dtype), _ptr(dX),
         K, dt(dw_dtype), _ptr(dW), K, int(next_fmt), _ptr(am), _ptr(sc), _ptr(ws), ws.numel(), _stream())
    return dX, dW, am, sc


def gemm_bwd_plan(M: int, N: int, K: int, ws_bytes: int | None = None):
    """(grouped, dW slices) that df_fp8_gemm_bwd picks; ws_bytes defaults
    to df_fp8_gemm_bwd_workspace_bytes."""
    if ws_bytes is None:
        ws_bytes = int(lib().df_fp8_gemm_bwd_workspace_bytes(M, N, K))
    g, s = _c_int(), _c_int()
    call("df_fp8_gemm_bwd_plan", M, N, K, ws_bytes, ctypes.byref(g), ctypes.byref(s))
    return bool(g.value), s.value


def colsum(x):
    torch = _torch()
    rows, cols = x.shape
    out = torch.empty(cols, dtype=torch.float32, device=x.device)
    ws = _scratch(x.device, int(lib().df_quantize_2d_workspace_bytes(rows, cols)), "colsum")
    call("df_colsum", int(_in_dtype(x)), _ptr(x), rows, cols, x.stride(0), _ptr(out), _ptr(ws), ws.numel(),
         _stream())
    return out


class WeightStreamer:
    """Ring of device weight slots filled from pinned host memory on a copy
    stream (``df_streamer_*`` in include/df_capi.h).  ``load`` returns
    (slot, device pointer); ``wait`` / ``release`` order the slot against the
    current torch stream."""

    def __init__(self, slots: int, slot_bytes: int):
        h = _vp()
        call("df_streamer_create", slots, slot_bytes, ctypes.byref(h))
        self.handle = h
        self.slots = slots

    def load(self, host_ptr: int, nbytes: int):
        slot = _c_int()
        dev = _vp()
        call("df_streamer_load", self.handle, host_ptr, nbytes, ctypes.byref(slot), ctypes.byref(dev))
        return slot.value, dev.value

    def wait(self, slot: int, stream: int | None = None):
        call("df_streamer_wait", self.handle, slot, _stream() if stream is None else stream)

    def release(self, slot: int, stream: int | None = None):
        call("df_streamer_release", self.handle, slot, _stream() if stream is None else stream)

    def set_timing(self, on: bool = True):
        """Record HIP events around every later copy (see copy_log)."""
        call("df_streamer_set_timing", self.handle, 1 if on else 0)

    def copy_log(self) -> list[tuple[float, float]]:
        """(start, end) in ms of every timed copy since the last call, in load
        order (waits for them to finish); clears the log."""
        n = ctypes.c_int()
        call("df_streamer_copy_log", self.handle, None, None, 0, ctypes.byref(n))
        cap = n.value
        a, b = (ctypes.c_float * max(cap, 1))(), (ctypes.c_float * max(cap, 1))()
        call("df_streamer_copy_log", self.handle, a, b, cap, ctypes.byref(n))
        return [(a[i], b[i]) for i in range(min(cap, n.value))]

    def copy_streams(self) -> tuple[int, int]:
        """The two copy streams (load i runs on stream i % 2)."""
        out = []
        for which in (0, 1):
            st = _vp()
            call("df_streamer_copy_stream", self.handle, which, ctypes.byref(st))
            out.append(st.value or 0)
        return out[0], out[1]

    def close(self):
        if self.handle is not None:
            call("df_streamer_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------------------
# consumer side: global-norm clipping and Adam over lists of fp32 tensors
# (dnn/utils/clip_grad_norm.cu:31-67, dnn/optimizers/adam_optimizer.cu:11-109)
# ----------------------------------------------------------------------------
def _ptrs(tensors):
    return (_vp * max(len(tensors), 1))(*[t.data_ptr() for t in tensors])


def _sizes(tensors):
    return (_c_i64 * max(len(tensors), 1))(*[t.numel() for t in tensors])


def grad_norm(grads, clip: float | None = None):
    """Global L2 norm of fp32 device tensors as a 1-element device tensor;
    with ``clip`` the tensors are scaled in place by clip / norm when
    norm > clip (utils::clip_grad_norm)."""
    torch = _torch()
    dev = grads[0].device
    sizes = _sizes(grads)
    nbytes = lib().df_grad_norm_workspace_bytes(len(grads), sizes)
    ws = _scratch(dev, nbytes, "grad_norm")
    norm = torch.empty(1, dtype=torch.float32, device=dev)
    if clip is None:
        call("df_grad_norm_f32", _ptrs(grads), sizes, len(grads), _ptr(norm), _ptr(ws), ws.numel(), _stream())
    else:
        call("df_clip_grad_norm_f32", _ptrs(grads), sizes, len(grads), float(clip), _ptr(norm), _ptr(ws),
             ws.numel(), _stream())
    return norm


def adam_update(params, grads, ms, vs, timestep: int, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                weight_decay=0.0, clip_norm=None, max_norm=0.0, absmax=None):
    """One Adam step (AdamOptimizer<float>::step) over fp32 device tensors,
    in place on params, ms and vs; ``clip_norm`` (a device norm from
    :func:`grad_norm`) applies max_norm / norm to the gradients on the fly.
    ``absmax`` (an fp32 device tensor of len(params)) also receives max |p|
    of each updated tensor (df_adam_update_absmax_f32)."""
    n = len(params)
    assert len(grads) == n and len(ms) == n and len(vs) == n
    args = (_ptrs(params), _ptrs(grads), _ptrs(ms), _ptrs(vs), _sizes(params), n, float(lr), float(beta1),
            float(beta2), float(eps), float(weight_decay), int(timestep), _ptr(clip_norm), float(max_norm))
    if absmax is None:
        call("df_adam_update_f32", *args, _stream())
    else:
        assert absmax.numel() >= n and absmax.dtype == _torch().float32
        call("df_adam_update_absmax_f32", *args, _ptr(absmax), _stream())


# ----------------------------------------------------------------------------
# delayed scaling: scale from an amax history, absmax measured in the pass
# ----------------------------------------------------------------------------
class DelayedScale:
    """History and scale of one tensor role (fp32 device tensors)."""

    def __init__(self, fmt: Fmt, length: int, device, seed_amax=None):
        torch = _torch()
        self.fmt = Fmt(fmt)
        self.history = torch.empty(length, dtype=torch.float32, device=device)
        self.scale = torch.empty(1, dtype=torch.float32, device=device)
        call("df_amax_history_init", _ptr(seed_amax), int(self.fmt), _ptr(self.history), length,
             _ptr(self.scale), _stream())

    def quantize_2d(self, x, want_q=True, want_qt=False, colsum=False):
        """Like :func:`quantize_2d` with the current scale; returns
        (q, qt[, colsum]) and advances the history."""
        torch = _torch()
        rows, cols = x.shape
        q = torch.empty((rows, round16(cols)), dtype=torch.uint8, device=x.device) if want_q else None
        qt = torch.empty((cols, round16(rows)), dtype=torch.uint8, device=x.device) if want_qt else None
        ldq = q.shape[1] if q is not None else 0
        ldqt = qt.shape[1] if qt is not None else 0
        cs = torch.empty(cols, dtype=torch.float32, device=x.device) if colsum else None
        nbytes = lib().df_quantize_2d_delayed_workspace_bytes(rows, cols, ldq, ldqt, int(colsum))
        ws = _scratch(x.device, nbytes, "delayed")
        call("df_quantize_2d_delayed", int(_in_dtype(x)), _ptr(x), rows, cols, x.stride(0), int(self.fmt),
             _ptr(self.scale), _ptr(self.scale), _ptr(self.history), self.history.numel(), _ptr(q), ldq, _ptr(qt),
             ldqt, _ptr(cs), _ptr(ws), ws.numel(), _stream())
        return (q, qt, cs) if colsum else (q, qt)


# ----------------------------------------------------------------------------
# LayerNorm with the fused quantize (dnn/layers/layer_norm_layer.cu:26-63)
# ----------------------------------------------------------------------------
def layernorm(x, gamma=None, beta=None, eps=1e-5, fmt: Fmt | None = None, want_y=True, want_q=True,
              want_qt=False, delayed: "DelayedScale | None" = None):
    """LayerNorm over the last dim of a 2-D fp32/bf16 tensor.  fmt=None: y
    only.  Otherwise returns (y or None, q, qt, scale) with the codes of y at
    the just-in-time scale, or at ``delayed``'s history scale."""
    torch = _torch()
    rows, cols = x.shape
    dt = int(_in_dtype(x))
    y = torch.empty_like(x) if (want_y or fmt is None) else None
    ldy = cols if y is not None else 0
    if fmt is None:
        nbytes = lib().df_layernorm_workspace_bytes(rows, cols, 0, 0)
        ws = _scratch(x.device, nbytes, "layernorm")
        call("df_layernorm", dt, _ptr(x), rows, cols, x.stride(0), _ptr(gamma), _ptr(beta), float(eps), _ptr(y),
             ldy, _ptr(ws), ws.numel(), _stream())
        return y
    q = torch.empty((rows, round16(cols)), dtype=torch.uint8, device=x.device) if want_q else None
    qt = torch.empty((cols, round16(rows)), dtype=torch.uint8, device=x.device) if want_qt else None
    ldq = q.shape[1] if q is not None else 0
    ldqt = qt.shape[1] if qt is not None else 0
    nbytes = lib().df_layernorm_workspace_bytes(rows, cols, ldq, ldqt)
    ws = _scratch(x.device, nbytes, "layernorm")
    if delayed is None:
        scale = torch.empty(1, dtype=torch.float32, device=x.device)
        call("df_layernorm_quantize", dt, _ptr(x), rows, cols, x.stride(0), _ptr(gamma), _ptr(beta), float(eps),
             _ptr(y), ldy, int(fmt), _ptr(scale), None, _ptr(q), ldq, _ptr(qt), ldqt, _ptr(ws), ws.numel(),
             _stream())
    else:
        scale = delayed.scale.clone()
        call("df_layernorm_quantize_delayed", dt, _ptr(x), rows, cols, x.stride(0), _ptr(gamma), _ptr(beta),
             float(eps), _ptr(y), ldy, int(fmt), _ptr(scale), _ptr(delayed.scale), _ptr(delayed.history),
             delayed.history.numel(), _ptr(q), ldq, _ptr(qt), ldqt, _ptr(ws), ws.numel(), _stream())
    return y, q, qt, scale
