"""Python binding of libdq8.so (include/dq8.h) over ctypes.

Device buffers are torch tensors on a ROCm device (torch is only memory and
stream plumbing here; every computation runs in the HIP kernels of libdq8.so).
Work is enqueued on torch's current stream of the tensors' device.

The names mirror decider-engine's int8 path:
  Weights.from_f32       Data::quantize(Precision::Int8Compute)   weights.rs:98-146
  Weights.from_quantized Data::Quantized { values, scales, .. }   weights.rs:16-23
  Context.quantize       QuantizedInputs::new (None -> NonFinite) tensor.rs:315-353
  Context.linear         linear_int8 + write_columns/Epilogue     tensor.rs:379-456, 272-288
  Context.linear_f32in   linear (quantize + multiply)             tensor.rs:290-308
  Context.weights_from_raw / weights_upload
                         Data::read + Data::quantize              weights.rs:147-195, 98-146
  SafeTensors            read_tensors' checkpoint reader          weights.rs:298-365
There is no CPU fallback: without libdq8.so, or without a GPU, calls raise.
"""
from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
# DQ8_LIBRARY selects another build of the library (for comparing kernel variants)
LIB_PATH = os.environ.get("DQ8_LIBRARY") or os.path.join(_HERE, "libdq8.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "dq8.h")

OK, ERR_SHAPE, ERR_NONFINITE, ERR_ARG, ERR_DEVICE, ERR_NOMEM, ERR_FORMAT, ERR_IO, ERR_CAPTURE, ERR_LIMIT = range(10)
F32, BF16, F16 = 0, 1, 2  # dq8_dtype
WRITE, ADD, SWIGLU = 0, 1, 2
ROWS, COLUMNS = 0, 1
GROUP = 64


class Dq8Error(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {status_string(status)} ({status})")
        self.status = status


class NonFinite(Dq8Error):
    """The reference's `None` from QuantizedInputs::new: the input holds NaN or +-inf."""


class _Lora(ctypes.Structure):
    _fields_ = [
        ("mid", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("rank", ctypes.c_size_t),
        ("scale", ctypes.c_float),
    ]


class _FfnWeights(ctypes.Structure):
    _fields_ = [
        ("gate", ctypes.c_void_p),
        ("up", ctypes.c_void_p),
        ("down", ctypes.c_void_p),
        ("gate_bias", ctypes.c_void_p),
        ("up_bias", ctypes.c_void_p),
        ("down_bias", ctypes.c_void_p),
        ("gate_lora", ctypes.POINTER(_Lora)),
        ("up_lora", ctypes.POINTER(_Lora)),
        ("down_lora_a", ctypes.c_void_p),
        ("down_lora_b", ctypes.c_void_p),
        ("down_lora_rank", ctypes.c_size_t),
        ("down_lora_scale", ctypes.c_float),
    ]


class _MidItem(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("m", ctypes.c_size_t),
        ("k", ctypes.c_size_t),
        ("a", ctypes.c_void_p),
        ("rank", ctypes.c_size_t),
        ("mid", ctypes.c_void_p),
    ]


class _Item(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("m", ctypes.c_size_t),
        ("bias", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("layout", ctypes.c_int),
        ("epilogue", ctypes.c_int),
        ("lora", ctypes.POINTER(_Lora)),
    ]


_lib = None
_vp, _sz, _i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int


def header_functions() -> list[str]:
    """Every function that include/dq8.h declares."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"^\s*(?:dq8_status|const char \*)\s*(dq8_\w+)\s*\(", text, re.M)))


def lib() -> ctypes.CDLL:
    """Load libdq8.so (no GPU needed to load it)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libdq8.so is not built: {LIB_PATH} (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    sig = {
        "dq8_create": ([_i, ctypes.POINTER(_vp)], _i),
        "dq8_destroy": ([_vp], _i),
        "dq8_reserve": ([_vp, _sz, _sz, _sz], _i),
        "dq8_weights_from_f32": ([_vp, _vp, _sz, _sz, _vp, ctypes.POINTER(_vp)], _i),
        "dq8_weights_from_quantized": ([_vp, _vp, _vp, _sz, _sz, _vp, ctypes.POINTER(_vp)], _i),
        "dq8_weights_export": ([_vp, _vp, _vp, _vp, _vp], _i),
        "dq8_weights_shape": ([_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz)], _i),
        "dq8_weights_free": ([_vp], _i),
        "dq8_quantize": ([_vp, _vp, _sz, _sz, _vp, _vp, _vp, _vp], _i),
        "dq8_linear": ([_vp, _vp, _vp, _vp, _sz, _vp, _vp, _i, _i, _vp], _i),
        "dq8_linear_f32in": ([_vp, _vp, _vp, _sz, _vp, _vp, _i, _i, _vp], _i),
        "dq8_linear_batch": ([_vp, ctypes.POINTER(_Item), _sz, _vp], _i),
        "dq8_lora_mid": ([_vp, _vp, _sz, _sz, _vp, _sz, _vp, _vp], _i),
        "dq8_lora_mid_batch": ([_vp, ctypes.POINTER(_MidItem), _sz, _vp], _i),
        "dq8_linear_lora": ([_vp, _vp, _vp, _vp, _sz, _vp, ctypes.POINTER(_Lora), _vp, _i, _i, _vp], _i),
        "dq8_linear_q": ([_vp, _vp, _vp, _vp, _sz, _vp, ctypes.POINTER(_Lora), _vp, _i, _vp, _vp, _vp, _vp], _i),
        "dq8_ffn": ([_vp, ctypes.POINTER(_FfnWeights), _vp, _vp, _sz, _vp, _vp, _vp, _vp], _i),
        "dq8_ffn_gate_up": ([_vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
        "dq8_ffn_gate_up_lora": ([_vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
        "dq8_group_dots": ([_vp, _vp, _vp, _sz, _vp, _vp], _i),
        "dq8_status_string": ([_i], ctypes.c_char_p),
        "dq8_linear_fp32": ([_vp, _vp, _vp, _sz, _vp, ctypes.POINTER(_Lora), _vp, _i, _i, _vp], _i),
        "dq8_apply": ([_vp, _vp, _vp, _sz, _vp, ctypes.POINTER(_Lora), _vp, _i, _i, _vp], _i),
        "dq8_apply_noalloc": ([_vp, _vp, _vp, _sz, _vp, ctypes.POINTER(_Lora), _vp, _i, _i, _vp], _i),
        "dq8_weights_from_raw": ([_vp, _vp, _i, _sz, _sz, _vp, ctypes.POINTER(_vp)], _i),
        "dq8_weights_upload": ([_vp, _vp, _i, _sz, _sz, _vp, ctypes.POINTER(_vp)], _i),
        "dq8_st_open": ([ctypes.c_char_p, ctypes.POINTER(_vp)], _i),
        "dq8_st_close": ([_vp], _i),
        "dq8_st_count": ([_vp, ctypes.POINTER(_sz)], _i),
        "dq8_st_info": ([_vp, _sz, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                         ctypes.POINTER(_sz), ctypes.POINTER(ctypes.POINTER(_sz)), ctypes.POINTER(_sz)], _i),
        "dq8_st_find": ([_vp, ctypes.c_char_p, ctypes.POINTER(_sz)], _i),
        "dq8_st_read_host": ([_vp, _sz, _vp, _sz], _i),
        "dq8_st_read_f32_host": ([_vp, _sz, _vp, _sz], _i),
        "dq8_st_load_weights": ([_vp, _vp, _sz, _vp, ctypes.POINTER(_vp)], _i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def status_string(status: int) -> str:
    try:
        return lib().dq8_status_string(status).decode()
    except RuntimeError:
        return "unknown"


def _check(status: int, what: str) -> None:
    if status == ERR_NONFINITE:
        raise NonFinite(status, what)
    if status != OK:
        raise Dq8Error(status, what)


def _torch():
    import torch

    return torch


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device).cuda_stream


def groups(k: int) -> int:
    return (k + GROUP - 1) // GROUP


class Weights:
    """A repacked int8 weight matrix [n][k] resident on the device."""

    def __init__(self, ctx: "Context", handle: int, n: int, k: int):
        self.ctx, self.handle, self.n, self.k = ctx, handle, n, k

    @property
    def groups(self) -> int:
        return groups(self.k)

    def export(self):
        """(values uint8 [n][k], scales float32 [n][G]) in the Data::Quantized layout."""
        torch = _torch()
        dev = self.ctx.device
        values = torch.empty((self.n, self.k), dtype=torch.uint8, device=dev)
        scales = torch.empty((self.n, self.groups), dtype=torch.float32, device=dev)
        _check(lib().dq8_weights_export(self.ctx.handle, self.handle, values.data_ptr(), scales.data_ptr(),
                                        _stream(dev)), "dq8_weights_export")
        return values, scales

    def free(self) -> None:
        if self.handle:
            _check(lib().dq8_weights_free(self.handle), "dq8_weights_free")
            self.handle = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class Lora:
    """A projection's LoRA pair as the reference's Adapter holds it (tensor.rs:102-108):
    mid [m][rank] (Context.lora_mid of x and lora_A), b = lora_B [n][rank], scale."""

    mid: object
    b: object
    scale: float


@dataclass
class Item:
    """One projection of Context.linear_batch."""

    w: Weights
    q: object
    scales: object
    out: object
    bias: object = None
    layout: int = ROWS
    epilogue: int = WRITE
    lora: Lora | None = None


class Context:
    def __init__(self, device: int = 0):
        torch = _torch()
        if not torch.cuda.is_available():
            raise RuntimeError("dq8 needs a ROCm GPU; none is visible")
        self.index = device
        self.device = torch.device("cuda", device)
        h = ctypes.c_void_p()
        _check(lib().dq8_create(device, ctypes.byref(h)), "dq8_create")
        self.handle = h.value

    def reserve(self, m: int, k: int, rank: int = 0) -> None:
        """Pre-size the context workspace for calls of up to m rows of width k
        (and an FFN down adapter of rank `rank`), so that later calls can be
        graph-captured without growing it."""
        _check(lib().dq8_reserve(self.handle, m, k, rank), "dq8_reserve")

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().dq8_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _dev(self, t, dtype, shape=None, name="tensor"):
        torch = _torch()
        if t.device != self.device or t.dtype != dtype or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dtype} tensor on {self.device}")
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        return t

    # -- weights -------------------------------------------------------
    def weights_from_f32(self, w) -> Weights:
        torch = _torch()
        self._dev(w, torch.float32, name="w")
        n, k = w.shape
        h = ctypes.c_void_p()
        _check(lib().dq8_weights_from_f32(self.handle, w.data_ptr(), n, k, _stream(self.device), ctypes.byref(h)),
               "dq8_weights_from_f32")
        return Weights(self, h.value, n, k)

    def weights_from_quantized(self, values, scales) -> Weights:
        torch = _torch()
        self._dev(values, torch.uint8, name="values")
        n, k = values.shape
        self._dev(scales, torch.float32, (n, groups(k)), "scales")
        h = ctypes.c_void_p()
        _check(lib().dq8_weights_from_quantized(self.handle, values.data_ptr(), scales.data_ptr(), n, k,
                                                _stream(self.device), ctypes.byref(h)), "dq8_weights_from_quantized")
        return Weights(self, h.value, n, k)

    def weights_from_raw(self, data, dtype: int | None = None) -> Weights:
        """Data::read + Data::quantize of stored elements already on the device:
        a [n][k] float32, bfloat16 or float16 tensor, or uint16 bit patterns
        with dtype BF16 or F16.  Raises NonFinite for non-finite weights."""
        torch = _torch()
        code = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}.get(data.dtype, dtype)
        if code is None or (data.dtype == torch.uint16 and dtype not in (BF16, F16)):
            raise ValueError("weights_from_raw: float32/bfloat16/float16 data, or uint16 with dtype BF16/F16")
        self._dev(data, data.dtype, name="data")
        n, k = data.shape
        h = ctypes.c_void_p()
        _check(lib().dq8_weights_from_raw(self.handle, data.data_ptr(), code, n, k, _stream(self.device),
                                          ctypes.byref(h)), "dq8_weights_from_raw")
        return Weights(self, h.value, n, k)

    def weights_upload(self, data, dtype: int) -> Weights:
        """weights_from_raw from host memory: a C-contiguous 2-D numpy array of
        stored elements (float32 for F32, uint16 bit patterns for BF16/F16),
        streamed through the context's pinned staging buffers."""
        import numpy as np

        want = np.float32 if dtype == F32 else np.uint16
        if not isinstance(data, np.ndarray) or data.dtype != want or data.ndim != 2 or not data.flags.c_contiguous:
            raise ValueError(f"weights_upload: a C-contiguous 2-D {np.dtype(want).name} array")
        n, k = data.shape
        h = ctypes.c_void_p()
        _check(lib().dq8_weights_upload(self.handle, data.ctypes.data, dtype, n, k, _stream(self.device),
                                        ctypes.byref(h)), "dq8_weights_upload")
        return Weights(self, h.value, n, k)

    # -- activations ---------------------------------------------------
    def quantize(self, x, q=None, scales=None, nonfinite=None):
        """QuantizedInputs::new.  Raises NonFinite like the reference's None,
        unless `nonfinite` (a zeroed int32 device scalar) is given: then the
        call does not synchronize and the flag is ORed on the device."""
        torch = _torch()
        self._dev(x, torch.float32, name="x")
        m, k = x.shape
        if q is None:
            q = torch.empty((m, k), dtype=torch.int8, device=self.device)
        if scales is None:
            scales = torch.empty((m, groups(k)), dtype=torch.float32, device=self.device)
        self._dev(q, torch.int8, (m, k), "q")
        self._dev(scales, torch.float32, (m, groups(k)), "scales")
        _check(lib().dq8_quantize(self.handle, x.data_ptr(), m, k, q.data_ptr(), scales.data_ptr(),
                                  _ptr(nonfinite), _stream(self.device)), "dq8_quantize")
        return q, scales

    # -- projections ---------------------------------------------------
    def linear(self, w: Weights, q, scales, out=None, bias=None, layout=ROWS, epilogue=WRITE):
        torch = _torch()
        self._dev(q, torch.int8, name="q")
        m, k = q.shape
        if k != w.k:
            raise Dq8Error(ERR_SHAPE, "dq8_linear: input width differs from the weights")
        self._dev(scales, torch.float32, (m, groups(k)), "scales")
        shape = (m, w.n) if layout == ROWS else (w.n, m)
        if out is None:
            out = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self._dev(out, torch.float32, shape, "out")
        if bias is not None:
            self._dev(bias, torch.float32, (w.n,), "bias")
        _check(lib().dq8_linear(self.handle, w.handle, q.data_ptr(), scales.data_ptr(), m, _ptr(bias),
                                out.data_ptr(), layout, epilogue, _stream(self.device)), "dq8_linear")
        return out

    # -- LoRA ----------------------------------------------------------
    def lora_mid(self, x, a, mid=None):
        """mid [m][rank] = linear(x, lora_A) in the reference's FP32 order (weights.rs:480, 495)."""
        torch = _torch()
        self._dev(x, torch.float32, name="x")
        self._dev(a, torch.float32, name="lora_A")
        m, k = x.shape
        rank, ka = a.shape
        if ka != k:
            raise Dq8Error(ERR_SHAPE, "dq8_lora_mid: lora_A width differs from the input")
        if mid is None:
            mid = torch.zeros((m, rank), dtype=torch.float32, device=self.device)
        self._dev(mid, torch.float32, (m, rank), "mid")
        _check(lib().dq8_lora_mid(self.handle, x.data_ptr(), m, k, a.data_ptr(), rank, mid.data_ptr(),
                                  _stream(self.device)), "dq8_lora_mid")
        return mid

    def lora_mid_batch(self, pairs, mids=None):
        """dq8_lora_mid of every (x, lora_A) pair, grouped into as few launches as
        possible; returns the middle products (the given `mids`, or new tensors)."""
        torch = _torch()
        arr = (_MidItem * max(1, len(pairs)))()
        out = []
        for i, (x, a) in enumerate(pairs):
            self._dev(x, torch.float32, name="x")
            self._dev(a, torch.float32, name="lora_A")
            m, k = x.shape
            rank, ka = a.shape
            if ka != k:
                raise Dq8Error(ERR_SHAPE, "dq8_lora_mid_batch: lora_A width differs from the input")
            mid = mids[i] if mids is not None else torch.zeros((m, rank), dtype=torch.float32, device=self.device)
            self._dev(mid, torch.float32, (m, rank), "mid")
            arr[i] = _MidItem(x.data_ptr(), m, k, a.data_ptr(), rank, mid.data_ptr())
            out.append(mid)
        _check(lib().dq8_lora_mid_batch(self.handle, arr, len(pairs), _stream(self.device)), "dq8_lora_mid_batch")
        return out

    def _lora(self, lora: Lora, m: int, n: int) -> _Lora:
        torch = _torch()
        rank = lora.b.shape[1]
        self._dev(lora.mid, torch.float32, (m, rank), "lora mid")
        self._dev(lora.b, torch.float32, (n, rank), "lora_B")
        return _Lora(lora.mid.data_ptr(), lora.b.data_ptr(), rank, lora.scale)

    def linear_lora(self, w: Weights, q, scales, lora: Lora, out=None, bias=None, layout=ROWS, epilogue=WRITE):
        torch = _torch()
        self._dev(q, torch.int8, name="q")
        m, k = q.shape
        if k != w.k:
            raise Dq8Error(ERR_SHAPE, "dq8_linear_lora: input width differs from the weights")
        self._dev(scales, torch.float32, (m, groups(k)), "scales")
        shape = (m, w.n) if layout == ROWS else (w.n, m)
        if out is None:
            out = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self._dev(out, torch.float32, shape, "out")
        if bias is not None:
            self._dev(bias, torch.float32, (w.n,), "bias")
        lo = self._lora(lora, m, w.n)
        _check(lib().dq8_linear_lora(self.handle, w.handle, q.data_ptr(), scales.data_ptr(), m, _ptr(bias),
                                     ctypes.byref(lo), out.data_ptr(), layout, epilogue, _stream(self.device)),
               "dq8_linear_lora")
        return out

    def linear_q(self, w: Weights, q, scales, out=None, bias=None, lora: Lora | None = None, epilogue=WRITE,
                 nonfinite=None):
        """The projection (rows layout) plus QuantizedInputs::new of its stored result:
        returns (out, q_out, scales_out).  Raises NonFinite like dq8_quantize unless
        `nonfinite` (a zeroed int32 device scalar) is given."""
        torch = _torch()
        self._dev(q, torch.int8, name="q")
        m, k = q.shape
        if k != w.k:
            raise Dq8Error(ERR_SHAPE, "dq8_linear_q: input width differs from the weights")
        self._dev(scales, torch.float32, (m, groups(k)), "scales")
        if out is None:
            out = torch.zeros((m, w.n), dtype=torch.float32, device=self.device)
        self._dev(out, torch.float32, (m, w.n), "out")
        if bias is not None:
            self._dev(bias, torch.float32, (w.n,), "bias")
        qo = torch.empty((m, w.n), dtype=torch.int8, device=self.device)
        so = torch.empty((m, groups(w.n)), dtype=torch.float32, device=self.device)
        lo = None if lora is None else ctypes.byref(self._lora(lora, m, w.n))
        _check(lib().dq8_linear_q(self.handle, w.handle, q.data_ptr(), scales.data_ptr(), m, _ptr(bias), lo,
                                  out.data_ptr(), epilogue, qo.data_ptr(), so.data_ptr(), _ptr(nonfinite),
                                  _stream(self.device)), "dq8_linear_q")
        return out, qo, so

    def ffn(self, gate: Weights, up: Weights, down: Weights, q, scales, residual, h=None, biases=(None, None, None),
            gate_lora: Lora | None = None, up_lora: Lora | None = None, down_lora=None, nonfinite=None):
        """One layer's FFN chain (qwen.rs:486-492): h = silu(gate(x)) * up(x); residual += down(h).
        down_lora = (lora_A [rank][inter], lora_B [hidden][rank], scale) or None.  Returns h.
        A non-finite h sends down through the FP32 path, as in the crate; `nonfinite`
        (a uint32 device scalar) then gets 1 ORed into it."""
        torch = _torch()
        self._dev(q, torch.int8, name="q")
        m, k = q.shape
        self._dev(scales, torch.float32, (m, groups(k)), "scales")
        if h is None:
            h = torch.zeros((m, up.n), dtype=torch.float32, device=self.device)
        self._dev(h, torch.float32, (m, up.n), "h")
        self._dev(residual, torch.float32, (m, down.n), "residual")
        fw = _FfnWeights(gate.handle, up.handle, down.handle, *[_ptr(b) for b in biases])
        keep = []
        if gate_lora is not None:
            keep.append(self._lora(gate_lora, m, gate.n))
            fw.gate_lora = ctypes.pointer(keep[-1])
        if up_lora is not None:
            keep.append(self._lora(up_lora, m, up.n))
            fw.up_lora = ctypes.pointer(keep[-1])
        if down_lora is not None:
            a, b, sc = down_lora
            self._dev(a, torch.float32, (a.shape[0], up.n), "down lora_A")
            self._dev(b, torch.float32, (down.n, a.shape[0]), "down lora_B")
            fw.down_lora_a, fw.down_lora_b, fw.down_lora_rank, fw.down_lora_scale = a.data_ptr(), b.data_ptr(), \
                a.shape[0], sc
        _check(lib().dq8_ffn(self.handle, ctypes.byref(fw), q.data_ptr(), scales.data_ptr(), m, h.data_ptr(),
                             residual.data_ptr(), _ptr(nonfinite), _stream(self.device)), "dq8_ffn")
        return h

    def ffn_gate_up(self, gate: Weights, up: Weights, q, scales, h=None, biases=(None, None), quantize=False,
                    nonfinite=None, loras=(None, None)):
        """h = silu(gate(x) + gate_bias) * (up(x) + up_bias) (qwen.rs:489-490), the gate Write and up SwiGlu
        stores of one FFN in one call, each projection with its LoRA adapter when loras gives one (Lora, with
        the adapter's middle product computed).  Returns h [m][n], or with quantize=True (h, h_q, h_scales): h
        also quantized for the down projection, as dq8_quantize(h) would; raises NonFinite like dq8_quantize
        unless `nonfinite` (a zeroed uint32 device scalar) is given."""
        torch = _torch()
        self._dev(q, torch.int8, name="q")
        m, k = q.shape
        self._dev(scales, torch.float32, (m, groups(k)), "scales")
        if h is None:
            h = torch.empty((m, up.n), dtype=torch.float32, device=self.device)
        self._dev(h, torch.float32, (m, up.n), "h")
        hq = hs = None
        if quantize:
            hq = torch.empty((m, up.n), dtype=torch.int8, device=self.device)
            hs = torch.empty((m, groups(up.n)), dtype=torch.float32, device=self.device)
        lo = [self._lora(lr, m, w.n) if lr is not None else None for lr, w in zip(loras, (gate, up))]
        lp = [ctypes.byref(x) if x is not None else None for x in lo]
        _check(lib().dq8_ffn_gate_up_lora(self.handle, gate.handle, up.handle, q.data_ptr(), scales.data_ptr(), m,
                                          _ptr(biases[0]), _ptr(biases[1]), lp[0], lp[1], h.data_ptr(), _ptr(hq),
                                          _ptr(hs), _ptr(nonfinite), _stream(self.device)), "dq8_ffn_gate_up_lora")
        return (h, hq, hs) if quantize else h

    def linear_f32in(self, w: Weights, x, out=None, bias=None, layout=ROWS, epilogue=WRITE):
        torch = _torch()
        self._dev(x, torch.float32, name="x")
        m, k = x.shape
        if k != w.k:
            raise Dq8Error(ERR_SHAPE, "dq8_linear_f32in: input width differs from the weights")
        shape = (m, w.n) if layout == ROWS else (w.n, m)
        if out is None:
            out = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self._dev(out, torch.float32, shape, "out")
        if bias is not None:
            self._dev(bias, torch.float32, (w.n,), "bias")
        _check(lib().dq8_linear_f32in(self.handle, w.handle, x.data_ptr(), m, _ptr(bias), out.data_ptr(), layout,
                                      epilogue, _stream(self.device)), "dq8_linear_f32in")
        return out

    def _fp32_call(self, fn: str, w: Weights, x, out, bias, lora, layout, epilogue):
        torch = _torch()
        self._dev(x, torch.float32, name="x")
        m, k = x.shape
        if k != w.k:
            raise Dq8Error(ERR_SHAPE, f"{fn}: input width differs from the weights")
        shape = (m, w.n) if layout == ROWS else (w.n, m)
        if out is None:
            out = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self._dev(out, torch.float32, shape, "out")
        if bias is not None:
            self._dev(bias, torch.float32, (w.n,), "bias")
        lo = self._lora(lora, m, w.n) if lora is not None else None
        _check(getattr(lib(), fn)(self.handle, w.handle, x.data_ptr(), m, _ptr(bias),
                                  ctypes.byref(lo) if lo is not None else None, out.data_ptr(), layout, epilogue,
                                  _stream(self.device)), fn)
        return out

    def linear_fp32(self, w: Weights, x, out=None, bias=None, lora: Lora | None = None, layout=ROWS, epilogue=WRITE):
        """Projection::columns_tiled: the FP32 path over dequantized weights."""
        return self._fp32_call("dq8_linear_fp32", w, x, out, bias, lora, layout, epilogue)

    def apply(self, w: Weights, x, out=None, bias=None, lora: Lora | None = None, layout=ROWS, epilogue=WRITE):
        """Projection::apply_quantized on fp32 x: the int8 path, or the FP32 path
        if x holds a non-finite value, chosen on the device."""
        return self._fp32_call("dq8_apply", w, x, out, bias, lora, layout, epilogue)

    def apply_noalloc(self, w: Weights, x, out=None, bias=None, lora: Lora | None = None, layout=ROWS,
                      epilogue=WRITE):
        """apply() through dq8_apply_noalloc: no device allocation, inputs limited
        by the library's fixed 16 MiB scratch (ERR_LIMIT beyond it)."""
        return self._fp32_call("dq8_apply_noalloc", w, x, out, bias, lora, layout, epilogue)

    def linear_batch(self, items: list[Item]) -> None:
        torch = _torch()
        arr = (_Item * max(1, len(items)))()
        keep = []  # the _Lora structs must outlive the call
        for i, it in enumerate(items):
            self._dev(it.q, torch.int8, name="q")
            m, k = it.q.shape
            if k != it.w.k:
                raise Dq8Error(ERR_SHAPE, "dq8_linear_batch: input width differs from the weights")
            self._dev(it.scales, torch.float32, (m, groups(k)), "scales")
            shape = (m, it.w.n) if it.layout == ROWS else (it.w.n, m)
            self._dev(it.out, torch.float32, shape, "out")
            lp = None
            if it.lora is not None:
                keep.append(self._lora(it.lora, m, it.w.n))
                lp = ctypes.pointer(keep[-1])
            arr[i] = _Item(it.w.handle, it.q.data_ptr(), it.scales.data_ptr(), m, _ptr(it.bias), it.out.data_ptr(),
                           it.layout, it.epilogue, lp)
        _check(lib().dq8_linear_batch(self.handle, arr, len(items), _stream(self.device)), "dq8_linear_batch")

    def group_dots(self, w: Weights, q):
        torch = _torch()
        self._dev(q, torch.int8, name="q")
        m, k = q.shape
        if k != w.k:
            raise Dq8Error(ERR_SHAPE, "dq8_group_dots: input width differs from the weights")
        dots = torch.zeros((m, w.n, groups(k)), dtype=torch.int32, device=self.device)
        _check(lib().dq8_group_dots(self.handle, w.handle, q.data_ptr(), m, dots.data_ptr(), _stream(self.device)),
               "dq8_group_dots")
        return dots


def is_projection(name: str, shape) -> bool:
    """read_tensors' rule for weights quantized at load (weights.rs:346-351),
    applied to a name with the file's prefix already removed."""
    return name.startswith("layers.") and "_proj" in name and name.endswith(".weight") and len(shape) == 2


class SafeTensors:
    """One safetensors file through dq8_st_* (the checks of read_tensors,
    weights.rs:298-365).  Opening and reading need no GPU; load_weights does."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _check(lib().dq8_st_open(os.fsencode(path), ctypes.byref(h)), f"dq8_st_open({path})")
        self.handle = h.value
        n = ctypes.c_size_t()
        _check(lib().dq8_st_count(self.handle, ctypes.byref(n)), "dq8_st_count")
        self.tensors = []  # (name, dtype, shape, bytes) in file order
        for i in range(n.value):
            name, dt = ctypes.c_char_p(), ctypes.c_char_p()
            nd, nb = ctypes.c_size_t(), ctypes.c_size_t()
            shp = ctypes.POINTER(ctypes.c_size_t)()
            _check(lib().dq8_st_info(self.handle, i, ctypes.byref(name), ctypes.byref(dt), ctypes.byref(nd),
                                     ctypes.byref(shp), ctypes.byref(nb)), "dq8_st_info")
            self.tensors.append((name.value.decode(), dt.value.decode(), tuple(shp[j] for j in range(nd.value)),
                                 nb.value))
        self._index = {t[0]: i for i, t in enumerate(self.tensors)}

    def reserve(self, m: int, k: int, rank: int = 0) -> None:
        """Pre-size the context workspace for calls of up to m rows of width k
        (and an FFN down adapter of rank `rank`), so that later calls can be
        graph-captured without growing it."""
        _check(lib().dq8_reserve(self.handle, m, k, rank), "dq8_reserve")

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().dq8_st_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def names(self):
        return [t[0] for t in self.tensors]

    def info(self, name: str):
        """(dtype, shape, bytes) of a tensor."""
        return self.tensors[self._index[name]][1:]

    def read(self, name: str):
        """Data::read: the stored elements (float32, or uint16 bit patterns for
        BF16/F16), shaped.  Raises NonFinite for non-finite weights."""
        import numpy as np

        i = self._index[name]
        _, dt, shape, nbytes = self.tensors[i]
        out = np.empty(shape, dtype=np.float32 if dt == "F32" else np.uint16)
        if out.nbytes != nbytes and dt in ("F32", "BF16", "F16"):
            raise Dq8Error(ERR_SHAPE, "read")
        _check(lib().dq8_st_read_host(self.handle, i, out.ctypes.data, nbytes), f"dq8_st_read_host({name})")
        return out

    def read_f32(self, name: str):
        """Data::into_f32 of a tensor, shaped."""
        import numpy as np

        i = self._index[name]
        shape = self.tensors[i][2]
        out = np.empty(shape, dtype=np.float32)
        _check(lib().dq8_st_read_f32_host(self.handle, i, out.ctypes.data, out.size), f"dq8_st_read_f32_host({name})")
        return out

    def load_weights(self, ctx: "Context", name: str) -> "Weights":
        """A projection weight [n][k] from the file to the device, quantized and repacked."""
        i = self._index[name]
        _, _, shape, _ = self.tensors[i]
        h = ctypes.c_void_p()
        _check(lib().dq8_st_load_weights(ctx.handle, self.handle, i, _stream(ctx.device), ctypes.byref(h)),
               f"dq8_st_load_weights({name})")
        return Weights(ctx, h.value, shape[0], shape[1])
