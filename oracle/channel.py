"""numpy restatement of per-channel (KIVI-style) key quantization with an fp16
residual window -- test infrastructure only.

The reference plans this format as its next step for keys
(``docs/future_work.md:229-293``) and has no implementation of it, so there are
no reference outputs to compare with.  Its arithmetic is the reference's own
group-wise quantizer (``quantize.py:186-236``) applied along the other axis:

* keys are cut into blocks of ``block`` consecutive tokens; within a block,
  every channel (head dim) d is one group of ``block`` values -- fp32 min and
  max, scale = range / qmax (1 when not positive), scale and zero rounded to
  fp16 before the codes, code = round-half-even((x - zero) / scale) clamped to
  [0, qmax];
* codes are packed per token row in the split-P layout of ``quantize.py:40-54``
  (byte j of a row holds the codes of dims j + p * D/P), exactly as per-token
  codes are;
* scale and zero are stored per (block, channel): ``(..., S / block, D)`` fp16;
* values keep the reference's per-token groups;
* the most recent tokens (fewer than one block per row) stay in fp16: the
  residual window.  Attention runs over the dequantized blocks followed by the
  window.

Pinned by: ``quantize_keys_per_channel(x)`` equals the reference quantizer
(``quant.quantize_groupwise``, itself pinned by the golden vectors) run on each
block transposed to ``(D, block)`` with ``group_size = block``; the split-P
packing is the pinned ``quant.pack_codes``; dequantization is checked against
float64 ``code * scale + zero``; the attention is the pinned fp32 attention on
the concatenated history (tests/test_oracle.py).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import quant as oq

BLOCK = 32  # tokens per key block: the decode kernel's chunk


@dataclass
class ChannelKeysNP:
    """Per-channel quantized keys: codes per token row, metadata per block."""

    packed: np.ndarray  # uint8 (..., S, D // P)
    scale: np.ndarray   # float16 (..., S // block, D)
    zero: np.ndarray    # float16 (..., S // block, D)
    nbits: int
    block: int
    head_dim: int


def quantize_keys_per_channel(x: np.ndarray, nbits: int, block: int = BLOCK) -> ChannelKeysNP:
    """x: (..., S, D) with S a multiple of ``block``."""
    oq._check_bits(nbits)
    *lead, S, D = x.shape
    if block <= 0 or S % block:
        raise ValueError(f"token count {S} must be a multiple of the block {block}")
    nb = S // block
    # (..., nb, block, D) -> (..., nb, D, block): each channel's block is one group
    xt = np.swapaxes(np.asarray(x).reshape(*lead, nb, block, D), -1, -2)
    qmax = (1 << nbits) - 1
    xf = xt.astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        gmin = xf.min(axis=-1)  # NaN-propagating, as torch's amin / amax
        gmax = xf.max(axis=-1)
        scale = (gmax - gmin) / np.float32(qmax)
        scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
        scale16 = scale.astype(np.float16)
        zero16 = gmin.astype(np.float16)
    # a NaN channel's zero is the canonical fp16 NaN, as in oracle.quant
    zero16 = np.where(np.isnan(gmin), np.uint16(0x7E00).view(np.float16), zero16)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        codes = np.rint((xf - zero16.astype(np.float32)[..., None])
                        / scale16.astype(np.float32)[..., None])
    codes = np.where(np.isnan(codes), np.float32(0.0), codes)
    codes = np.clip(codes, 0, qmax).astype(np.uint8)          # (..., nb, D, block)
    rows = np.swapaxes(codes, -1, -2).reshape(*lead, S, D)     # per token row
    return ChannelKeysNP(oq.pack_codes(rows, nbits), scale16, zero16, nbits, block, D)


def dequantize_keys_per_channel(ck: ChannelKeysNP) -> np.ndarray:
    """fp32 ``code * scale + zero``, scale and zero of the token's block."""
    codes = oq.unpack_codes(ck.packed, ck.nbits, ck.head_dim).astype(np.float32)
    *lead, S, D = codes.shape
    nb = S // ck.block
    cg = codes.reshape(*lead, nb, ck.block, D)
    with np.errstate(invalid="ignore"):  # 0 * inf of an infinite scale is NaN, as intended
        out = cg * ck.scale.astype(np.float32)[..., None, :] + ck.zero.astype(np.float32)[..., None, :]
    return out.reshape(*lead, S, D).astype(np.float32)


def history(ck: ChannelKeysNP, vq: oq.QuantNP, k_res: np.ndarray, v_res: np.ndarray,
            q_lens, r_lens):
    """Per batch row b: the fp32 K and V of its first q_lens[b] quantized tokens
    followed by its first r_lens[b] residual tokens, padded to a common length.
    Returns (k, v, lens) with k, v: (B, HKV, L, D)."""
    kd = dequantize_keys_per_channel(ck)
    vd = oq.dequantize_groupwise(vq)
    B, HKV, _, D = kd.shape
    lens = [int(a) + int(r) for a, r in zip(q_lens, r_lens)]
    L = max(1, max(lens))
    k = np.zeros((B, HKV, L, D), np.float32)
    v = np.zeros((B, HKV, L, D), np.float32)
    for b in range(B):
        a, r = int(q_lens[b]), int(r_lens[b])
        k[b, :, :a] = kd[b, :, :a]
        v[b, :, :a] = vd[b, :, :a]
        k[b, :, a:a + r] = np.asarray(k_res[b, :, :r], np.float32)
        v[b, :, a:a + r] = np.asarray(v_res[b, :, :r], np.float32)
    return k, v, np.asarray(lens)


def channel_row_bytes(head_dim: int, nbits: int, block: int = BLOCK) -> float:
    """Key bytes per token per KV head: codes plus the block's metadata share."""
    return head_dim * nbits / 8 + 4 * head_dim / block
