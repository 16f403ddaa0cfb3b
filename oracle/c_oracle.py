"""ctypes binding of ``oracle/liboracle.so`` (built from ``tkv_oracle.c``).

Test infrastructure only.  Arrays cross as numpy buffers; fp16 values cross as
their uint16 bit patterns so the C side owns every rounding decision.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build() -> str:
    subprocess.run([os.path.join(_HERE, "build_oracle.sh")], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        p = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.tkvo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.tkvo_f16_to_f32.restype = f32
        L.tkvo_f32_to_f16.argtypes = [f32]
        L.tkvo_f32_to_f16.restype = ctypes.c_uint16
        L.tkvo_quantize.argtypes = [p, i64, i32, i32, i32, p, p, p]
        L.tkvo_quantize.restype = i32
        L.tkvo_dequantize.argtypes = [p, p, p, i64, i32, i32, i32, p]
        L.tkvo_dequantize.restype = None
        L.tkvo_decode_attention.argtypes = [p, p, p, i32, i32, i32, i32, i32, f32, p, p]
        L.tkvo_decode_attention.restype = i32
        L.tkvo_quantized_decode_attention.argtypes = (
            [p] * 7 + [i32] * 7 + [f32, p])
        L.tkvo_quantized_decode_attention.restype = i32
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    f = lib().tkvo_f32_to_f16
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


def quantize(x: np.ndarray, nbits: int, gs: int):
    """Returns (packed u8 (..., D/P), scale f16 (..., D/gs), zero f16 (..., D/gs))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D
    P = 8 // nbits
    packed = np.empty(x.shape[:-1] + (D // P,), dtype=np.uint8)
    scale = np.empty(x.shape[:-1] + (D // gs,), dtype=np.uint16)
    zero = np.empty_like(scale)
    rc = lib().tkvo_quantize(_ptr(x), rows, D, nbits, gs, _ptr(packed), _ptr(scale), _ptr(zero))
    if rc:
        raise ValueError(f"tkvo_quantize rejected nbits={nbits} gs={gs} D={D}")
    return packed, scale.view(np.float16), zero.view(np.float16)


def dequantize(packed, scale, zero, nbits: int, gs: int, D: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(scale, dtype=np.float16).view(np.uint16)
    z = np.ascontiguousarray(zero, dtype=np.float16).view(np.uint16)
    rows = packed.size // packed.shape[-1]
    out = np.empty(packed.shape[:-1] + (D,), dtype=np.float32)
    lib().tkvo_dequantize(_ptr(packed), _ptr(s), _ptr(z), rows, D, nbits, gs, _ptr(out))
    return out


def decode_attention(q, k, v, sm_scale: float, seq_lens=None) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, HQ, D = q.shape
    HKV, S = k.shape[1], k.shape[2]
    out = np.empty((B, HQ, D), dtype=np.float32)
    lens = None if seq_lens is None else np.ascontiguousarray(seq_lens, dtype=np.int64)
    rc = lib().tkvo_decode_attention(_ptr(q), _ptr(k), _ptr(v), B, HQ, HKV, S, D, sm_scale,
                                     None if lens is None else _ptr(lens), _ptr(out))
    if rc:
        raise ValueError("tkvo_decode_attention rejected the shapes")
    return out


def quantized_decode_attention(q, kq, vq, sm_scale: float) -> np.ndarray:
    """kq / vq: (packed, scale, zero, nbits, gs) tuples with (B,HKV,S,*) arrays."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, HQ, D = q.shape
    kp, ks, kz, nbits, gs = kq
    vp, vs, vz, _, _ = vq
    HKV, S = kp.shape[1], kp.shape[2]
    arrs = [np.ascontiguousarray(a) for a in (kp, ks.view(np.uint16), kz.view(np.uint16),
                                               vp, vs.view(np.uint16), vz.view(np.uint16))]
    out = np.empty((B, HQ, D), dtype=np.float32)
    rc = lib().tkvo_quantized_decode_attention(_ptr(q), *[_ptr(a) for a in arrs], B, HQ, HKV,
                                               S, D, nbits, gs, sm_scale, _ptr(out))
    if rc:
        raise ValueError("tkvo_quantized_decode_attention rejected the shapes")
    return out
