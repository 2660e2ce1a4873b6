"""TEST INFRASTRUCTURE ONLY -- ctypes binding of the C oracle (dq8_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product library never does.  Arrays are numpy on the
host.  Build with `make -C oracle` (also done by __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

GROUP = 64
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libdq8_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        L.dq8o_quantize_inputs.argtypes = [_f32p, _sz, _sz, _i8p, _f32p, ctypes.c_int]
        L.dq8o_quantize_inputs.restype = ctypes.c_int
        L.dq8o_quantize_weights.argtypes = [_f32p, _sz, _sz, _u8p, _f32p]
        L.dq8o_quantize_weights.restype = None
        L.dq8o_dot.argtypes = [_i8p, _u8p, _sz]
        L.dq8o_dot.restype = ctypes.c_int32
        L.dq8o_scaled_dot.argtypes = [_i8p, _f32p, _u8p, _f32p, _sz]
        L.dq8o_scaled_dot.restype = ctypes.c_float
        L.dq8o_group_dots.argtypes = [_i8p, _sz, _u8p, _sz, _sz, _i32p]
        L.dq8o_group_dots.restype = None
        L.dq8o_linear_int8.argtypes = [_i8p, _f32p, _sz, _u8p, _f32p, _sz, _sz, ctypes.c_void_p, _f32p, ctypes.c_int]
        L.dq8o_linear_int8.restype = None
        L.dq8o_silu.argtypes = [ctypes.c_float]
        L.dq8o_silu.restype = ctypes.c_float
        L.dq8o_silu_n.argtypes = [_f32p, _f32p, _sz, ctypes.c_int]
        L.dq8o_silu_n.restype = None
        L.dq8o_expf_restated.argtypes = [ctypes.c_float]
        L.dq8o_expf_restated.restype = ctypes.c_float
        L.dq8o_expf_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int]
        L.dq8o_expf_mismatches.restype = ctypes.c_size_t
        L.dq8o_write_columns.argtypes = [_f32p, _sz, _sz, _f32p, ctypes.c_int]
        L.dq8o_write_columns.restype = None
        L.dq8o_linear.argtypes = [_f32p, _sz, _sz, _u8p, _f32p, _sz, ctypes.c_void_p, _f32p, ctypes.c_int, ctypes.c_int]
        L.dq8o_linear.restype = ctypes.c_int
        L.dq8o_dot_scores.argtypes = [_f32p, _f32p, _sz]
        L.dq8o_dot_scores.restype = ctypes.c_float
        L.dq8o_linear_f32.argtypes = [_f32p, _sz, _sz, _f32p, _sz, ctypes.c_void_p, _f32p, ctypes.c_int]
        L.dq8o_linear_f32.restype = None
        L.dq8o_lora_mid.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _f32p, ctypes.c_int]
        L.dq8o_lora_mid.restype = None
        L.dq8o_lora_combine.argtypes = [ctypes.c_float, _f32p, _f32p, _sz, ctypes.c_float]
        L.dq8o_lora_combine.restype = ctypes.c_float
        L.dq8o_linear_lora.argtypes = [_f32p, _sz, _sz, _u8p, _f32p, _sz, ctypes.c_void_p, _f32p, _f32p, _sz,
                                       ctypes.c_float, _f32p, ctypes.c_int, ctypes.c_int]
        L.dq8o_linear_lora.restype = ctypes.c_int
        L.dq8o_dequantize_weights.argtypes = [_u8p, _f32p, _sz, _sz, _f32p]
        L.dq8o_dequantize_weights.restype = None
        L.dq8o_apply.argtypes = [_f32p, _sz, _sz, _u8p, _f32p, _sz, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, _sz, ctypes.c_float, _f32p, ctypes.c_int, ctypes.c_int]
        L.dq8o_apply.restype = ctypes.c_int
        _lib = L
    return _lib


def groups(k: int) -> int:
    return (k + GROUP - 1) // GROUP


def quantize_inputs(x: np.ndarray, threads: int = 1):
    """QuantizedInputs::new: (q [M][K] int8, scales [M][G]) or None if non-finite."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, groups(k)), np.float32)
    if lib().dq8o_quantize_inputs(x, rows, k, q, s, threads) != 0:
        return None
    return q, s


def quantize_weights(w: np.ndarray):
    """Data::quantize (8 bits): (values [N][K] uint8, scales [N][G])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    v = np.zeros((n, k), np.uint8)
    s = np.zeros((n, groups(k)), np.float32)
    lib().dq8o_quantize_weights(w, n, k, v, s)
    return v, s


def decode_weights(raw: np.ndarray, dtype: str) -> np.ndarray:
    """Data::row / Data::into_f32 of stored elements (weights.rs:35-46, 83-90).

    F32: unchanged.  BF16: f32::from_bits((v as u32) << 16).  F16: `half`
    (weights.rs:367-382) in float32 arithmetic: sign * m * 2^-24 for e = 0,
    +-inf / NaN for e = 31, else sign * (1 + m/1024) * 2^(e-15).
    """
    if dtype == "F32":
        return np.ascontiguousarray(raw, dtype=np.float32)
    v = np.ascontiguousarray(raw, dtype=np.uint16)
    if dtype == "BF16":
        return (v.astype(np.uint32) << np.uint32(16)).view(np.float32)
    if dtype != "F16":
        raise ValueError(f"unsupported weight dtype {dtype}")
    sign = np.where(v & 0x8000, np.float32(-1.0), np.float32(1.0))
    e = ((v >> 10) & 31).astype(np.int32)
    m = (v & 1023).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        sub = sign * m * np.float32(2.0 ** -24)
        norm = sign * ((np.float32(1.0) + m / np.float32(1024.0)) * np.ldexp(np.float32(1.0), e - 15).astype(np.float32))
        special = np.where(m == 0, sign * np.float32(np.inf), np.float32(np.nan))
    return np.where(e == 0, sub, np.where(e == 31, special, norm)).astype(np.float32)


def weights_finite(raw: np.ndarray, dtype: str) -> bool:
    """Data::read's check (weights.rs:170-187): F32 is_finite, or the 16-bit
    exponent mask (0x7f80 for BF16, 0x7c00 for F16) not all ones."""
    if dtype == "F32":  # float32 values, or their uint32 bit patterns
        raw = np.asarray(raw)
        return bool(np.all(np.isfinite(raw.view(np.float32) if raw.dtype == np.uint32 else raw.astype(np.float32))))
    mask = np.uint16(0x7F80 if dtype == "BF16" else 0x7C00)
    return bool(np.all((np.asarray(raw, dtype=np.uint16) & mask) != mask))


def dot(a: np.ndarray, b: np.ndarray) -> int:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    assert a.shape == b.shape and a.size <= GROUP
    return int(lib().dq8o_dot(a, b, a.size))


def scaled_dot(x, xs, w, ws) -> np.float32:
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    assert x.size == w.size and xs.size == ws.size == groups(x.size)
    return np.float32(lib().dq8o_scaled_dot(x, xs, w, ws, x.size))


def group_dots(q: np.ndarray, w: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rows, k = q.shape
    n = w.shape[0]
    out = np.zeros((rows, n, groups(k)), np.int32)
    lib().dq8o_group_dots(q, rows, w, n, k, out)
    return out


def _bias_ptr(bias):
    if bias is None:
        return None, None
    b = np.ascontiguousarray(bias, dtype=np.float32)
    return b, b.ctypes.data_as(ctypes.c_void_p)


def linear_int8(q, xs, w, ws, bias=None, threads: int = 1) -> np.ndarray:
    """linear_int8 on quantized inputs: columns [N][M]."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    rows, k = q.shape
    n = w.shape[0]
    cols = np.zeros((n, rows), np.float32)
    keep, bp = _bias_ptr(bias)
    lib().dq8o_linear_int8(q, xs, rows, w, ws, n, k, bp, cols, threads)
    return cols


def write_columns(columns: np.ndarray, result: np.ndarray, epilogue: int) -> np.ndarray:
    """write_columns + Epilogue (0 write, 1 add, 2 swiglu) into a copy of result."""
    columns = np.ascontiguousarray(columns, dtype=np.float32)
    out = np.array(result, dtype=np.float32, copy=True, order="C")
    n, rows = columns.shape
    lib().dq8o_write_columns(columns, rows, n, out, epilogue)
    return out


def silu(x: float) -> np.float32:
    return np.float32(lib().dq8o_silu(float(x)))


def silu_n(x: np.ndarray, threads: int = 1) -> np.ndarray:
    """dq8o_silu elementwise over a float32 array (any shape)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().dq8o_silu_n(x, y, x.size, threads)
    return y


def expf_restated(x: float) -> np.float32:
    """The restated glibc expf algorithm (the one the kernels run)."""
    return np.float32(lib().dq8o_expf_restated(float(x)))


def expf_mismatches(begin: int, end: int, threads: int = 1) -> int:
    """Bit patterns in [begin, end) where the restated expf differs from libm's."""
    return int(lib().dq8o_expf_mismatches(begin, end, threads))


def linear(x, w, ws, bias=None, result=None, epilogue: int = 0, threads: int = 1):
    """The x86 plan of Linear::apply_into (no LoRA): returns result [M][N], or None
    when the reference would fall back to FP32 (non-finite input)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    rows, k = x.shape
    n = w.shape[0]
    out = np.zeros((rows, n), np.float32) if result is None else np.array(result, np.float32, copy=True, order="C")
    keep, bp = _bias_ptr(bias)
    st = lib().dq8o_linear(x, rows, k, w, ws, n, bp, out, epilogue, threads)
    if st == 1:
        return None
    if st != 0:
        raise MemoryError("oracle allocation failed")
    return out


def dot_scores(a, b) -> np.float32:
    """dot_scores (tensor.rs:6-25), x86-64 order."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    assert a.shape == b.shape and a.ndim == 1
    return np.float32(lib().dq8o_dot_scores(a, b, a.size))


def linear_f32(x, w, bias=None, threads: int = 1) -> np.ndarray:
    """`linear` of FP32 weights w [N][K] (Epilogue::Write): result [M][N]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = x.shape
    n = w.shape[0]
    out = np.zeros((rows, n), np.float32)
    keep, bp = _bias_ptr(bias)
    lib().dq8o_linear_f32(x, rows, k, w, n, bp, out, threads)
    return out


def lora_mid(x, a, threads: int = 1) -> np.ndarray:
    """LoRA middle product mid [M][rank] = linear(x, A), A [rank][K]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    a = np.ascontiguousarray(a, dtype=np.float32)
    rows, k = x.shape
    rank = a.shape[0]
    mid = np.zeros((rows, rank), np.float32)
    lib().dq8o_lora_mid(x, rows, k, a, rank, mid, threads)
    return mid


def lora_combine(base: float, mid_row, b_row, scale: float) -> np.float32:
    """Adapter::combine (tensor.rs:109-117)."""
    mid_row = np.ascontiguousarray(mid_row, dtype=np.float32)
    b_row = np.ascontiguousarray(b_row, dtype=np.float32)
    return np.float32(lib().dq8o_lora_combine(float(base), mid_row, b_row, mid_row.size, float(scale)))


def linear_lora(x, w, ws, a, b, scale: float, bias=None, result=None, epilogue: int = 0, threads: int = 1):
    """The x86 plan of Linear::apply_into with a LoRA pair (A [rank][K], B [N][rank],
    FP32): result [M][N], or None when the base projection would fall back to FP32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    rows, k = x.shape
    n = w.shape[0]
    rank = a.shape[0]
    assert a.shape == (rank, k) and b.shape == (n, rank)
    out = np.zeros((rows, n), np.float32) if result is None else np.array(result, np.float32, copy=True, order="C")
    keep, bp = _bias_ptr(bias)
    st = lib().dq8o_linear_lora(x, rows, k, w, ws, n, bp, a, b, rank, float(scale), out, epilogue, threads)
    if st == 1:
        return None
    if st != 0:
        raise MemoryError("oracle allocation failed")
    return out


def dequantize_weights(w, ws) -> np.ndarray:
    """Data::row of 8-bit Quantized weights: (float)q * scale, [N][K] float32."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    n, k = w.shape
    out = np.zeros((n, k), np.float32)
    lib().dq8o_dequantize_weights(w, ws, n, k, out)
    return out


def apply(x, w, ws, bias=None, a=None, b=None, scale=0.0, result=None, epilogue: int = 0, threads: int = 1):
    """Projection::apply_quantized with the FP32 fallback for non-finite x.
    Returns (result [M][N], fp32_path_taken)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    rows, width = x.shape
    n = w.shape[0]
    out = np.zeros((rows, n), np.float32) if result is None else np.array(result, dtype=np.float32, copy=True, order="C")
    keep, bp = _bias_ptr(bias)
    rank = 0
    ap = bpp = None
    if a is not None:
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        rank = a.shape[0]
        ap, bpp = a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p)
    st = lib().dq8o_apply(x, rows, width, w, ws, n, bp, ap, bpp, rank, scale, out, epilogue, threads)
    if st == 2:
        raise MemoryError("dq8o_apply")
    return out, st == 1
