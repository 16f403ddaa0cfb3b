"""numpy restatement of the reference quantizer -- test infrastructure only.

Follows ``quantize.py`` of the reference:

* split-P layout ``quantize.py:40-54``: with ``P = 8 // nbits`` codes per byte and
  ``DP = D // P`` bytes per row, bits ``[p*nbits, (p+1)*nbits)`` of byte ``j``
  hold the code of dim ``j + p*DP``;
* ``pack_codes`` ``quantize.py:149-169``; ``unpack_codes`` ``:172-183``;
* ``quantize_groupwise`` ``:186-236`` (fp32 min/max per group, scale =
  range/qmax with a degenerate group getting scale 1, scale and zero rounded to
  fp16 *before* the codes are computed, codes = round-half-even of
  ``(x - zero) / scale`` clamped to ``[0, qmax]``);
* ``dequantize_groupwise`` ``:239-246`` (``code * scale + zero`` in fp32).

Every operation below is an IEEE-754 binary32 operation (numpy float32
arithmetic is correctly rounded), ``np.rint`` rounds half to even like
``torch.round``, and ``astype(np.float16)`` rounds to nearest even like
``Tensor.half()``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SUPPORTED_BITS = (2, 4)
META_BITS_PER_GROUP = 2 * 16  # fp16 scale + fp16 zero, quantize.py:64-65


def _check_bits(nbits: int) -> None:
    if nbits not in SUPPORTED_BITS:
        raise ValueError(f"nbits must be one of {SUPPORTED_BITS}, got {nbits}")


@dataclass
class QuantNP:
    """numpy mirror of ``QuantizedTensor`` (``quantize.py:73-146``)."""

    packed: np.ndarray  # uint8 (..., D // P)
    scale: np.ndarray   # float16 (..., D // gs)
    zero: np.ndarray    # float16 (..., D // gs)
    nbits: int
    group_size: int
    head_dim: int

    @property
    def n_groups(self) -> int:
        return self.head_dim // self.group_size

    def nbytes(self) -> int:
        return self.packed.nbytes + self.scale.nbytes + self.zero.nbytes

    def effective_bits_per_element(self) -> float:
        return self.nbits + META_BITS_PER_GROUP / self.group_size


def pack_codes(codes: np.ndarray, nbits: int) -> np.ndarray:
    """Split-P pack, ``quantize.py:149-169``: byte j = OR_p code[j + p*DP] << p*nbits."""
    _check_bits(nbits)
    if codes.dtype != np.uint8:
        raise TypeError(f"codes must be uint8, got {codes.dtype}")
    P = 8 // nbits
    D = codes.shape[-1]
    if D % P != 0:
        raise ValueError(f"head_dim {D} must be divisible by {P} for {nbits}-bit packing")
    DP = D // P
    out = np.zeros(codes.shape[:-1] + (DP,), dtype=np.uint8)
    for p in range(P):
        out |= (codes[..., p * DP:(p + 1) * DP] << np.uint8(p * nbits)).astype(np.uint8)
    return out


def unpack_codes(packed: np.ndarray, nbits: int, head_dim: int) -> np.ndarray:
    """Inverse of :func:`pack_codes`, ``quantize.py:172-183``."""
    _check_bits(nbits)
    P = 8 // nbits
    DP = head_dim // P
    if packed.shape[-1] != DP:
        raise ValueError(f"packed last dim {packed.shape[-1]} != head_dim//P = {DP}")
    mask = np.uint8((1 << nbits) - 1)
    parts = [(packed >> np.uint8(p * nbits)) & mask for p in range(P)]
    return np.concatenate(parts, axis=-1).astype(np.uint8)


def quantize_groupwise(x: np.ndarray, nbits: int, group_size: int) -> QuantNP:
    """Group-wise asymmetric quantization, ``quantize.py:186-236``."""
    _check_bits(nbits)
    D = x.shape[-1]
    if group_size <= 0 or D % group_size != 0:
        raise ValueError(f"group_size {group_size} must divide head_dim {D}")
    P = 8 // nbits
    if D % P != 0:
        raise ValueError(f"head_dim {D} must be divisible by {P} for {nbits}-bit packing")
    qmax = (1 << nbits) - 1
    ng = D // group_size

    xg = np.asarray(x).astype(np.float32).reshape(*x.shape[:-1], ng, group_size)
    # numpy's min/max propagate a NaN, as torch's amin/amax do (quantize.py:209-210)
    with np.errstate(invalid="ignore", over="ignore"):
        gmin = xg.min(axis=-1)
        gmax = xg.max(axis=-1)
        scale = (gmax - gmin) / np.float32(qmax)
        scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
        scale16 = scale.astype(np.float16)
        zero16 = gmin.astype(np.float16)
    # torch's amin returns the canonical quiet NaN whatever the NaN's sign or
    # payload (golden cases nan_one_*, f32_range_*), so a NaN group's zero is
    # fp16 0x7E00; numpy would keep the sign and payload bits.
    zero16 = np.where(np.isnan(gmin), np.uint16(0x7E00).view(np.float16), zero16)
    scale_f = scale16.astype(np.float32)
    zero_f = zero16.astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        codes = np.rint((xg - zero_f[..., None]) / scale_f[..., None])
    # A scale that rounds to fp16 zero makes 0/0 = NaN (torch.clamp keeps it and the
    # uint8 cast then yields 0 -- pinned by the golden vectors) and c/0 = +inf -> qmax.
    # The same holds for a NaN zero, inf/inf and (inf - inf): code 0.
    codes = np.where(np.isnan(codes), np.float32(0.0), codes)
    codes = np.clip(codes, 0, qmax).astype(np.uint8).reshape(*x.shape[:-1], D)
    return QuantNP(pack_codes(codes, nbits), scale16, zero16, nbits, group_size, D)


def dequantize_groupwise(qt: QuantNP) -> np.ndarray:
    """fp32 ``code * scale + zero``, ``quantize.py:239-246``."""
    codes = unpack_codes(qt.packed, qt.nbits, qt.head_dim)
    cg = codes.reshape(*codes.shape[:-1], qt.n_groups, qt.group_size).astype(np.float32)
    with np.errstate(invalid="ignore"):  # code 0 times an infinite scale is NaN
        out = cg * qt.scale.astype(np.float32)[..., None] + qt.zero.astype(np.float32)[..., None]
    return out.reshape(*codes.shape[:-1], qt.head_dim).astype(np.float32)


def dequantize_fp16(qt: QuantNP) -> np.ndarray:
    """The reference baseline's dequant into fp16, ``reference.py:96-108``:
    codes, scale and zero as fp16, ``code * scale`` then ``+ zero``, each
    operation rounded to fp16 (numpy's float16 arithmetic computes in fp32 and
    rounds the result, as half arithmetic on the GPU does)."""
    codes = unpack_codes(qt.packed, qt.nbits, qt.head_dim)
    cg = codes.reshape(*codes.shape[:-1], qt.n_groups, qt.group_size).astype(np.float16)
    with np.errstate(invalid="ignore", over="ignore"):
        out = cg * qt.scale[..., None] + qt.zero[..., None]
    return out.reshape(*codes.shape[:-1], qt.head_dim)


def quantize_kv(k: np.ndarray, v: np.ndarray, nbits: int, group_size: int):
    """``quantize.py:249-256``: K and V quantized independently."""
    return quantize_groupwise(k, nbits, group_size), quantize_groupwise(v, nbits, group_size)


def row_bytes(head_dim: int, nbits: int, group_size: int) -> int:
    """Bytes per token per KV head per tensor: codes plus fp16 scale and zero."""
    if nbits == 16:
        return 2 * head_dim
    return head_dim * nbits // 8 + 4 * (head_dim // group_size)
