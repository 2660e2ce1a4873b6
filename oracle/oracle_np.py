"""TEST INFRASTRUCTURE ONLY -- an independent numpy restatement of the same
int8-compute arithmetic as dq8_oracle.c, used to cross-check the C oracle bit
for bit.  Written from the reference, not from the C file:

  quantize      tensor.rs:321-339 / weights.rs:117-136 (absmax, scale, round, clamp)
  group dots    int8.rs:149-154 (exact integer sums; here int64 einsum)
  rescale sum   int8.rs:53-61 / tensor.rs:427-437 (p = xs*ws, t = d*p, s = s + t
                in group order, then + bias or + 0.0)
  epilogues     tensor.rs:92-99, qwen.rs:194-199

Every float operation is a numpy float32 elementwise op (IEEE binary32, round
to nearest even, never contracted).  Round-half-away-from-zero is done in
float64 on the exact float32 quotient (np.round is half-to-even).
"""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np

GROUP = 64
F32 = np.float32
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def groups(k: int) -> int:
    return -(-k // GROUP)


def round_half_away(v: np.ndarray) -> np.ndarray:
    d = v.astype(np.float64)
    return (np.sign(d) * np.floor(np.abs(d) + 0.5)).astype(np.float32)


def quantize(x: np.ndarray):
    """(q int8 [R][K], scales float32 [R][G]); the caller checks finiteness."""
    x = np.asarray(x, dtype=np.float32)
    rows, k = x.shape
    g = groups(k)
    pad = np.zeros((rows, g * GROUP), np.float32)
    pad[:, :k] = x
    blocks = pad.reshape(rows, g, GROUP)
    m = np.abs(blocks).max(axis=2)
    scale = np.where(m == F32(0), F32(1), np.maximum(m / F32(127), FLT_MIN)).astype(np.float32)
    r = round_half_away(blocks / scale[:, :, None])
    q = np.clip(r, F32(-127), F32(127)).astype(np.int8).reshape(rows, g * GROUP)[:, :k]
    return np.ascontiguousarray(q), scale


def quantize_inputs(x: np.ndarray):
    x = np.asarray(x, dtype=np.float32)
    if not np.all(np.isfinite(x)):
        return None
    return quantize(x)


def group_dots(q: np.ndarray, w_u8: np.ndarray) -> np.ndarray:
    """[R][N][G] int64 exact dots of each 64-group (partial last group)."""
    rows, k = q.shape
    n = w_u8.shape[0]
    g = groups(k)
    qa = np.zeros((rows, g * GROUP), np.int64)
    wa = np.zeros((n, g * GROUP), np.int64)
    qa[:, :k] = q.astype(np.int64)
    wa[:, :k] = w_u8.view(np.int8).astype(np.int64)
    return np.einsum("rgk,ngk->rng", qa.reshape(rows, g, GROUP), wa.reshape(n, g, GROUP))


def rescale_sum(dots: np.ndarray, xs: np.ndarray, ws: np.ndarray, bias=None) -> np.ndarray:
    """Result [R][N]: s = 0; s = s + f32(d_g) * (xs_g * ws_g) in group order; + bias."""
    rows, n, g = dots.shape
    s = np.zeros((rows, n), np.float32)
    for gi in range(g):
        p = xs[:, gi][:, None] * ws[:, gi][None, :]
        t = dots[:, :, gi].astype(np.float32) * p
        s = s + t
    b = np.zeros(n, np.float32) if bias is None else np.asarray(bias, np.float32)
    return s + b[None, :]


def linear_rows(x_q, xs, w_u8, ws, bias=None) -> np.ndarray:
    return rescale_sum(group_dots(x_q, w_u8), xs, ws, bias)


_libm = None


def expf(v: np.ndarray) -> np.ndarray:
    """Platform libm expf elementwise (what Rust's f32::exp calls on Linux)."""
    global _libm
    if _libm is None:
        _libm = ctypes.CDLL(ctypes.util.find_library("m"))
        _libm.expf.argtypes = [ctypes.c_float]
        _libm.expf.restype = ctypes.c_float
    flat = np.asarray(v, np.float32).ravel()
    out = np.array([_libm.expf(float(e)) for e in flat], dtype=np.float32)
    return out.reshape(np.shape(v))


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float32)
    return x * (F32(1) / (F32(1) + expf(-x)))


def store(dst: np.ndarray, value: np.ndarray, epilogue: int) -> np.ndarray:
    dst = np.asarray(dst, np.float32)
    if epilogue == 0:
        return value.astype(np.float32)
    if epilogue == 1:
        return dst + value
    return silu(dst) * value
