"""CPU tests of the per-channel key surface: validation and the C ABI's
argument checks (nothing is launched)."""

from __future__ import annotations

import ctypes

import pytest
import torch


def test_channel_keys_container():
    from tritonkv_amd.channel import empty_channel_keys

    ck = empty_channel_keys(2, 3, 64, 128, 2, device="cpu")
    assert ck.shape == (2, 3, 64, 128)
    assert ck.packed.shape == (2, 3, 64, 32) and ck.scale.shape == (2, 3, 2, 128)
    assert ck.effective_bits_per_element() == 3.0
    assert ck.nbytes() == 2 * 3 * (64 * 32 + 2 * 2 * 128 * 2)
    with pytest.raises(ValueError):
        empty_channel_keys(1, 1, 40, 128, 4, device="cpu")
    with pytest.raises(ValueError):
        empty_channel_keys(1, 1, 64, 128, 3, device="cpu")


def test_channel_decode_validates_before_the_backend_check():
    from tritonkv_amd.channel import channel_decode_attention, empty_channel_keys
    from tritonkv_amd.quantize import empty_cache

    ck = empty_channel_keys(1, 2, 64, 128, 4, device="cpu")
    q = torch.zeros(1, 8, 128, dtype=torch.float16)
    kr = torch.zeros(1, 2, 32, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="group_size"):
        channel_decode_attention(q, ck, empty_cache(1, 2, 64, 128, 4, 64, "cpu"), kr, kr)
    with pytest.raises(ValueError, match="inconsistent"):
        channel_decode_attention(q, ck, empty_cache(1, 2, 32, 128, 4, 32, "cpu"), kr, kr)
    with pytest.raises(ValueError, match="k_res"):
        channel_decode_attention(q, ck, empty_cache(1, 2, 64, 128, 4, 32, "cpu"), kr.float(), kr)


def test_channel_c_entry_points_reject_bad_arguments_without_a_gpu():
    from tritonkv_amd import _lib

    lib = _lib.load()
    d = 0x1000
    # token count not a multiple of 32 / capacity not a multiple of 32
    assert lib.tkv_quantize_keys_channel(d, 0, 1, 1, 40, 128, 4, None, 64, d, d, d, None) == \
        _lib.TKV_EINVAL
    assert lib.tkv_quantize_keys_channel(d, 0, 1, 1, 32, 128, 4, None, 48, d, d, d, None) == \
        _lib.TKV_EINVAL
    assert lib.tkv_quantize_keys_channel(d, 0, 1, 1, 32, 128, 3, None, 64, d, d, d, None) == \
        _lib.TKV_EINVAL
    a = _lib.DecodeArgs(q=d, k=d, v=d, k_scale=d, k_zero=d, v_scale=d, v_zero=d, out=d, acc=d,
                        maxs=d, sums=d, B=1, HQ=8, HKV=2, S=64, D=128, k_nbits=4, v_nbits=4,
                        group_size=32, sm_scale=0.1, split_size=64, num_splits=1, key_block=0)
    # the channel entry needs key_block == 32 and a window
    assert lib.tkv_channel_decode_attention(ctypes.byref(a), d, d, None, 32, None) == _lib.TKV_EINVAL
    a.key_block = 32
    assert lib.tkv_channel_decode_attention(ctypes.byref(a), None, d, None, 32, None) == \
        _lib.TKV_EINVAL
    a.key_block = 16
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EINVAL
    # partials placement: the window's row must fit, the whole-attention entry owns all splits
    a.key_block, a.split_base, a.num_splits_total = 0, 1, 1
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.split_base, a.num_splits_total = 0, 2
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    # per-channel keys need V groups of 16 or 32, and no paged cache
    a.num_splits_total, a.key_block, a.group_size = 0, 32, 64
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.group_size, a.page_size, a.block_table, a.block_table_stride, a.num_pages = 32, 32, d, 2, 4
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EINVAL


def test_channel_window_entry_points_reject_bad_arguments_without_a_gpu():
    from tritonkv_amd import _lib

    lib = _lib.load()
    d, lens = 0x1000, 0x2000
    # window capacity must be 32, D 64 or 128, pointers 16-byte aligned
    assert lib.tkv_channel_window_append(d, d, 2, 2, 128, d, d, 16, lens, None) == _lib.TKV_EINVAL
    assert lib.tkv_channel_window_append(d, d, 2, 2, 96, d, d, 32, lens, None) == _lib.TKV_EINVAL
    assert lib.tkv_channel_window_append(d + 2, d, 2, 2, 128, d, d, 32, lens, None) == \
        _lib.TKV_EINVAL
    assert lib.tkv_channel_window_append(d, d, 2, 2, 128, d, d, 32, None, None) == _lib.TKV_EINVAL
    args = [d, d, 2, 2, 128, 4, 2, 32, 32, lens, lens, 256, d, d, d, d, d, d, None]
    bad_cap = list(args)
    bad_cap[11] = 250
    assert lib.tkv_channel_window_flush(*bad_cap) == _lib.TKV_EINVAL
    bad_bits = list(args)
    bad_bits[5] = 3
    assert lib.tkv_channel_window_flush(*bad_bits) == _lib.TKV_EINVAL
    bad_gs = list(args)
    bad_gs[7] = 64
    assert lib.tkv_channel_window_flush(*bad_gs) == _lib.TKV_EUNSUPPORTED


def test_channel_cache_checks_token_shapes_before_any_launch():
    from tritonkv_amd.channel import ChannelKVCache

    c = ChannelKVCache(2, 2, 64, 128, device="cpu")
    good = torch.zeros(2, 2, 3, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="one shape"):
        c.extend(torch.zeros(1, 2, 3, 128, dtype=torch.float16), good)   # would broadcast
    with pytest.raises(ValueError, match="one shape"):
        c.extend(good, torch.zeros(2, 2, 4, 128, dtype=torch.float16))
    with pytest.raises(ValueError, match="one shape"):
        c.step(good, good, torch.zeros(2, 8, 128, dtype=torch.float16))  # 3 tokens, not 1
    with pytest.raises(TypeError):
        c.extend(None, good)
    assert len(c) == 0
    c.quantized, c.window = 32, 5
    c._qlens.fill_(32)
    c._rlens.fill_(5)
    c.reset()
    assert len(c) == 0 and not c._qlens.any() and not c._rlens.any()
