"""Pins of the per-channel key oracle (``oracle/channel.py``), on the CPU.

The format has no reference implementation (the reference plans it in
``docs/future_work.md:229-293``), so it is pinned through what it is built
from: the golden-pinned per-token quantizer applied to transposed blocks, the
pinned split-P packing, float64 dequantization and the pinned fp32 attention.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import channel as och
from oracle import inputs as oinp
from oracle import quant as oq


def _rand(shape, seed, scale=2.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape) * scale).astype(np.float16)


@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("D", [64, 128])
def test_per_channel_equals_per_token_quantizer_on_transposed_blocks(nbits, D, f32):
    B, H, S, T = 2, 3, 96, 32
    x = _rand((B, H, S, D), seed=nbits + D)
    x[0, 1, 40:50, 7] = 1.25                                  # a constant stretch
    x[1, 2, 64:96, 5] = 0.5                                   # a constant group
    x[0, 0, 3, 9] = np.nan                                    # non-finite input, which
    x[0, 2, 70, 11] = np.inf                                  # the per-token quantizer's
    x[1, 0, 33, 2] = -np.inf                                  # golden cases pin
    x.view(np.uint16)[1, 1, 90, 4] = 0xFE00                   # a NaN with the sign bit
    if f32:                                                   # fp32 input beyond the
        x = x.astype(np.float32)                              # fp16 range
        x[1, 0, 40, 7], x[1, 0, 41, 7] = 1.0e6, -7.0e4
    ck = och.quantize_keys_per_channel(x, nbits, T)
    codes = oq.unpack_codes(ck.packed, nbits, D)              # (B, H, S, D)
    assert ck.scale.shape == (B, H, S // T, D) and ck.scale.dtype == np.float16
    for blk in range(S // T):
        xt = np.swapaxes(x[:, :, blk * T:(blk + 1) * T, :], -1, -2)   # (B, H, D, T)
        ref = oq.quantize_groupwise(xt, nbits, T)
        ref_codes = oq.unpack_codes(ref.packed, nbits, T)               # (B, H, D, T)
        assert np.array_equal(np.swapaxes(codes[:, :, blk * T:(blk + 1) * T], -1, -2), ref_codes)
        assert np.array_equal(ck.scale[:, :, blk].view(np.uint16), ref.scale[..., 0].view(np.uint16))
        assert np.array_equal(ck.zero[:, :, blk].view(np.uint16), ref.zero[..., 0].view(np.uint16))
    # the constant group: scale 1, zero = the value, codes 0
    assert float(ck.scale[1, 2, 2, 5]) == 1.0 and float(ck.zero[1, 2, 2, 5]) == 0.5
    assert not codes[1, 2, 64:96, 5].any()
    # a NaN channel block: scale 1, the canonical NaN zero, codes 0
    assert ck.zero[0, 0, 0, 9].view(np.uint16) == 0x7E00 == ck.zero[1, 1, 2, 4].view(np.uint16)
    assert float(ck.scale[0, 0, 0, 9]) == 1.0 and not codes[0, 0, 0:32, 9].any()


@pytest.mark.parametrize("nbits", [2, 4])
def test_per_channel_dequant_is_code_times_scale_plus_zero(nbits):
    x = _rand((1, 2, 64, 128), seed=3)
    ck = och.quantize_keys_per_channel(x, nbits)
    got = och.dequantize_keys_per_channel(ck)
    codes = oq.unpack_codes(ck.packed, nbits, 128).astype(np.float64)
    s = np.repeat(ck.scale.astype(np.float64), 32, axis=2)
    z = np.repeat(ck.zero.astype(np.float64), 32, axis=2)
    want = codes * s + z                      # exact: c <= 15, s has 11 bits
    assert np.array_equal(got, want.astype(np.float32))
    # within half a step (plus the fp16 rounding of zero) of the input
    err = np.abs(got - x.astype(np.float32))
    assert (err <= 0.5 * s + np.abs(z) * 2.0 ** -10 + 1e-6).all()


def test_per_channel_keys_beat_per_token_on_outlier_channels():
    """The point of the format: keys whose large values sit in fixed channels."""
    _, k, _, _ = oinp.make_outlier_channel_kv(1, 8, 2, 256, 128, seed=5)
    k = k.numpy()
    kf = k.astype(np.float32)
    ch = och.dequantize_keys_per_channel(och.quantize_keys_per_channel(k, 2))
    tok = oq.dequantize_groupwise(oq.quantize_groupwise(k, 2, 32))
    e_ch = np.linalg.norm(ch - kf) / np.linalg.norm(kf)
    e_tok = np.linalg.norm(tok - kf) / np.linalg.norm(kf)
    assert e_ch < 0.75 * e_tok, (e_ch, e_tok)  # measured 0.40 vs 0.58


def test_history_attention_matches_float64_brute_force():
    B, HQ, HKV, D, T = 2, 4, 2, 64, 32
    q = _rand((B, HQ, D), seed=1, scale=1.0)
    k = _rand((B, HKV, 64, D), seed=2, scale=1.0)
    v = _rand((B, HKV, 64, D), seed=3, scale=1.0)
    kres = _rand((B, HKV, T, D), seed=4, scale=1.0)
    vres = _rand((B, HKV, T, D), seed=5, scale=1.0)
    ck = och.quantize_keys_per_channel(k, 4)
    vq = oq.quantize_groupwise(v, 4, 32)
    q_lens, r_lens = [64, 32], [5, 0]
    kh, vh, lens = och.history(ck, vq, kres, vres, q_lens, r_lens)
    assert list(lens) == [69, 32]
    got = oatt.reference_grouped(q, lambda s, e: kh[:, :, s:e], lambda s, e: vh[:, :, s:e],
                                 kh.shape[2], HKV, seq_lens=lens)
    kd = och.dequantize_keys_per_channel(ck)
    vd = oq.dequantize_groupwise(vq)
    for b in range(B):
        kk = np.concatenate([kd[b:b + 1, :, :q_lens[b]], kres[b:b + 1, :, :r_lens[b]]], axis=2)
        vv = np.concatenate([vd[b:b + 1, :, :q_lens[b]], vres[b:b + 1, :, :r_lens[b]]], axis=2)
        want = oatt.reference_decode_attention_f64(q[b:b + 1], kk, vv)
        assert np.abs(got[b] - want[0]).max() < 1e-5


def test_channel_row_bytes():
    assert och.channel_row_bytes(128, 4) == 64 + 16
    assert och.channel_row_bytes(128, 2) == 32 + 16
    with pytest.raises(ValueError):
        och.quantize_keys_per_channel(np.zeros((1, 1, 40, 64), np.float16), 4)
