"""ctypes binding of the CPU oracle (oracle/libdf_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker, never as the thing
measured or shipped.  Arrays are numpy, C-contiguous.
"""
from __future__ import annotations

import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdf_oracle.so")

E4M3, E5M2 = 0, 1
FMAX = {E4M3: 448.0, E5M2: 57344.0}

_vp, _i64, _i, _f, _u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_uint32
_SIGS = {
    "dfo_encode": (ctypes.c_uint8, [_f, _i]),
    "dfo_decode": (_f, [ctypes.c_uint8, _i]),
    "dfo_fmax": (_f, [_i]),
    "dfo_f32_to_bf16": (ctypes.c_uint16, [_f]),
    "dfo_bf16_to_f32": (_f, [ctypes.c_uint16]),
    "dfo_f32_to_f16": (ctypes.c_uint16, [_f]),
    "dfo_f16_to_f32": (_f, [ctypes.c_uint16]),
    "dfo_narrow_bits_range": (None, [_u32, _i64, _i, _vp, _i]),
    "dfo_convert": (_i, [_i, _vp, _i, _vp, _i64]),
    "dfo_absmax_f32": (_f, [_vp, _i64]),
    "dfo_absmax_bf16": (_f, [_vp, _i64]),
    "dfo_scale": (_f, [_f, _i]),
    "dfo_quantize_f32": (None, [_vp, _i64, _f, _i, _vp]),
    "dfo_quantize_bf16": (None, [_vp, _i64, _f, _i, _vp]),
    "dfo_dequantize_f32": (None, [_vp, _i64, _f, _i, _vp]),
    "dfo_dequantize_bf16": (None, [_vp, _i64, _f, _i, _vp]),
    "dfo_encode_bits_range": (None, [_u32, _i64, _i, _vp, _i]),
    "dfo_encode_by_table": (ctypes.c_uint8, [_f, _i]),
    "dfo_sweep_compare": (_i64, [_u32, _i64, _i, ctypes.POINTER(_u32), _i]),
    "dfo_fc_forward": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "dfo_fc_forward_bias_first": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "dfo_fc_backward_input": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "dfo_fc_backward_weights": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "dfo_fc_backward_bias": (None, [_vp, _vp, _i, _i]),
    "dfo_sumsq": (ctypes.c_double, [_vp, _i64]),
    "dfo_grad_norm": (_f, [_vp, _vp, _i]),
    "dfo_grad_norm_ref_f32": (_f, [_vp, _vp, _i]),
    "dfo_clip_scale": (_i, [_vp, _i64, _f, _f]),
    "dfo_bias_correction": (_f, [_f, _i]),
    "dfo_adam_step": (None, [_vp, _vp, _vp, _vp, _i64, _f, _f, _f, _f, _f, _i, _f]),
    "dfo_history_push": (_f, [_vp, _i, _f, _i]),
    "dfo_layernorm": (None, [_vp, _i, _i, _vp, _vp, _f, _i, _vp]),
}

_lib = None


def load(path: str) -> ctypes.CDLL:
    """A build of df_oracle.c at `path` with every signature declared (the
    default build, or the CPU-baseline build of `make -C oracle native`)."""
    L = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run make -C oracle")
        _lib = load(LIB_PATH)
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def nthreads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def encode(v: float, fmt: int) -> int:
    return lib().dfo_encode(v, fmt)


def decode(q: int, fmt: int) -> float:
    return lib().dfo_decode(q, fmt)


def absmax(x: np.ndarray) -> float:
    if x.dtype == np.float32:
        return lib().dfo_absmax_f32(_p(x), x.size)
    assert x.dtype == np.uint16  # bf16 bit patterns
    return lib().dfo_absmax_bf16(_p(x), x.size)


def scale(am: float, fmt: int) -> float:
    return lib().dfo_scale(am, fmt)


def _chunks(n: int, parts: int):
    step = max(1, (n + parts - 1) // parts)
    return [(lo, min(n, lo + step)) for lo in range(0, n, step)]


def quantize(x: np.ndarray, s: float, fmt: int, threads: int | None = None) -> np.ndarray:
    """Codes of x (float32, or uint16 holding bf16 bits); chunked over threads."""
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, dtype=np.uint8)
    xf, qf = x.reshape(-1), q.reshape(-1)
    fn = lib().dfo_quantize_f32 if x.dtype == np.float32 else lib().dfo_quantize_bf16
    item = x.itemsize

    def run(r):
        lo, hi = r
        fn(_p(xf) + lo * item, hi - lo, s, fmt, _p(qf) + lo)

    parts = _chunks(xf.size, threads or nthreads())
    with ThreadPoolExecutor(len(parts) or 1) as ex:
        list(ex.map(run, parts))
    return q


def dequantize(q: np.ndarray, s: float, fmt: int, out: str = "f32") -> np.ndarray:
    q = np.ascontiguousarray(q)
    if out == "f32":
        o = np.empty(q.shape, dtype=np.float32)
        lib().dfo_dequantize_f32(_p(q), q.size, s, fmt, _p(o))
    else:
        o = np.empty(q.shape, dtype=np.uint16)
        lib().dfo_dequantize_bf16(_p(q), q.size, s, fmt, _p(o))
    return o


def encode_bits_range(first: int, count: int, fmt: int, threads: int | None = None) -> np.ndarray:
    out = np.empty(count, dtype=np.uint8)
    lib().dfo_encode_bits_range(first, count, fmt, _p(out), threads or nthreads())
    return out


def sweep_compare(first: int, count: int, fmt: int, threads: int | None = None):
    bad = _u32(0)
    n = lib().dfo_sweep_compare(first, count, fmt, ctypes.byref(bad), threads or nthreads())
    return n, bad.value


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """RNE float32 -> bf16 bit patterns (numpy, same rule as the oracle's)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) & 0x8000 | 0x7FC0).astype(np.uint16)
    return r


_CVT_NP = {0: np.float32, 1: np.uint16, 2: np.int8, 4: np.uint16}


def convert(x: np.ndarray, in_dtype: int, out_dtype: int) -> np.ndarray:
    """dfo_convert: DType 0 (f32), 1 (f16 bits), 2 (int8), 4 (bf16 bits)."""
    x = np.ascontiguousarray(x, _CVT_NP[in_dtype])
    out = np.empty(x.shape, _CVT_NP[out_dtype])
    if lib().dfo_convert(in_dtype, _p(x), out_dtype, _p(out), x.size) != 0:
        raise ValueError(f"unsupported conversion {in_dtype} -> {out_dtype}")
    return out


def narrow_bits_range(first: int, count: int, to_f16: bool, threads: int | None = None) -> np.ndarray:
    """bf16 (or binary16) bit patterns of every fp32 pattern in [first, first+count)."""
    out = np.empty(count, np.uint16)
    lib().dfo_narrow_bits_range(first, count, 1 if to_f16 else 0, _p(out), threads or nthreads())
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fc_forward(X, W, b, threads=None, bias_first=False):
    X, W = np.ascontiguousarray(X, np.float32), np.ascontiguousarray(W, np.float32)
    N, K = X.shape
    O = W.shape[0]
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    Y = np.empty((N, O), np.float32)
    fn = lib().dfo_fc_forward_bias_first if bias_first else lib().dfo_fc_forward
    fn(_p(X), _p(W), _p(bb) if bb is not None else None, _p(Y), N, K, O, threads or nthreads())
    return Y


def fc_backward_input(dY, W, threads=None):
    dY, W = np.ascontiguousarray(dY, np.float32), np.ascontiguousarray(W, np.float32)
    N, O = dY.shape
    K = W.shape[1]
    dX = np.empty((N, K), np.float32)
    lib().dfo_fc_backward_input(_p(dY), _p(W), _p(dX), N, K, O, threads or nthreads())
    return dX


def fc_backward_weights(dY, X, threads=None):
    dY, X = np.ascontiguousarray(dY, np.float32), np.ascontiguousarray(X, np.float32)
    N, O = dY.shape
    K = X.shape[1]
    dW = np.empty((O, K), np.float32)
    lib().dfo_fc_backward_weights(_p(dY), _p(X), _p(dW), N, K, O, threads or nthreads())
    return dW


def fc_backward_bias(dY):
    dY = np.ascontiguousarray(dY, np.float32)
    N, O = dY.shape
    db = np.empty(O, np.float32)
    lib().dfo_fc_backward_bias(_p(dY), _p(db), N, O)
    return db


def rel_err(y: np.ndarray, r: np.ndarray) -> float:
    """Normwise relative error max|y-r| / max|r| (contract D6)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    den = np.max(np.abs(r)) if r.size else 0.0
    num = np.max(np.abs(y - r)) if r.size else 0.0
    return float(num / den) if den > 0 else float(num)


# ---- consumer side: clip and Adam (dnn/utils/clip_grad_norm.cu,
# dnn/optimizers/adam_optimizer.cu) ----
def _list(arrays):
    for a in arrays:
        assert a.dtype == np.float32 and a.flags.c_contiguous
    ptrs = (_vp * max(len(arrays), 1))(*[a.ctypes.data for a in arrays])
    sizes = (_i64 * max(len(arrays), 1))(*[a.size for a in arrays])
    return ptrs, sizes


def grad_norm(arrays) -> float:
    """Product contract: binary32 squares, binary64 sum, one rounding."""
    ptrs, sizes = _list(arrays)
    return lib().dfo_grad_norm(ptrs, sizes, len(arrays))


def grad_norm_ref_f32(arrays) -> float:
    """The reference's host loop: binary32 running sums."""
    ptrs, sizes = _list(arrays)
    return lib().dfo_grad_norm_ref_f32(ptrs, sizes, len(arrays))


def clip_scale(g: np.ndarray, norm: float, max_norm: float) -> bool:
    assert g.dtype == np.float32
    return bool(lib().dfo_clip_scale(_p(g), g.size, norm, max_norm))


def bias_correction(beta: float, t: int) -> float:
    return lib().dfo_bias_correction(beta, t)


def adam_step(p, g, m, v, t, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.0, clip_factor=1.0):
    """In place on p, m, v (float32 arrays)."""
    for a in (p, g, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous and a.size == p.size
    lib().dfo_adam_step(_p(p), _p(g), _p(m), _p(v), p.size, lr, beta1, beta2, eps, wd, t, clip_factor)


def history_push(history: np.ndarray, amax: float, fmt: int) -> float:
    """Delayed scaling: newest amax first; returns the next pass's scale."""
    assert history.dtype == np.float32 and history.flags.c_contiguous
    return lib().dfo_history_push(_p(history), history.size, amax, fmt)


def layernorm(x: np.ndarray, gamma=None, beta=None, eps=1e-5, round_bf16=False) -> np.ndarray:
    """LayerNorm over rows of a float32 [rows, C] array (the reference's
    thread-0 loops); gamma/beta float32 [C] or None."""
    x = np.ascontiguousarray(x, np.float32)
    rows, C = x.shape
    y = np.empty_like(x)
    g = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
    b = None if beta is None else np.ascontiguousarray(beta, np.float32)
    lib().dfo_layernorm(_p(x), rows, C, None if g is None else _p(g), None if b is None else _p(b), eps,
                        int(round_bf16), _p(y))
    return y
