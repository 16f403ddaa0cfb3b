"""Host-side argument checks of the paged cache and fused-append surface (no
GPU): they must raise before any backend call."""

from __future__ import annotations

import pytest
import torch


def _pool(num_pages=4, HKV=2, page=32, D=128, nbits=4, gs=32):
    from tritonkv_amd.quantize import QuantizedTensor

    P = 8 // nbits
    return QuantizedTensor(torch.zeros(num_pages, HKV, page, D // P, dtype=torch.uint8),
                           torch.ones(num_pages, HKV, page, D // gs, dtype=torch.float16),
                           torch.zeros(num_pages, HKV, page, D // gs, dtype=torch.float16),
                           nbits, gs, D)


def test_pool_shape_rules():
    from tritonkv_amd.paged import empty_paged_pool

    with pytest.raises(ValueError, match="multiple of 32"):
        empty_paged_pool(4, 2, 48, 128, 4, 32, device="cpu")
    with pytest.raises(ValueError, match="num_pages"):
        empty_paged_pool(0, 2, 32, 128, 4, 32, device="cpu")
    p = empty_paged_pool(3, 2, 64, 128, 2, 32, device="cpu")
    assert p.packed.shape == (3, 2, 64, 32) and p.scale.shape == (3, 2, 64, 4)


def test_paged_decode_validates_before_the_backend():
    from tritonkv_amd.paged import paged_decode_attention

    q = torch.zeros(2, 8, 128, dtype=torch.float16)
    kp, vp = _pool(), _pool()
    table = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match="block_table"):
        paged_decode_attention(q, kp, vp, table.long())
    with pytest.raises(ValueError, match="block_table"):
        paged_decode_attention(q, kp, vp, table[:1])
    with pytest.raises(ValueError, match="same nbits"):
        paged_decode_attention(q, kp, _pool(nbits=2), table)
    with pytest.raises(ValueError, match="multiple of HKV"):
        paged_decode_attention(torch.zeros(2, 7, 128, dtype=torch.float16), kp, vp, table)
    with pytest.raises(ValueError, match="seq_lens"):
        paged_decode_attention(q, kp, vp, table, seq_lens=torch.ones(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="k_new and v_new"):
        paged_decode_attention(q, kp, vp, table, k_new=torch.zeros(2, 2, 128))
    with pytest.raises(ValueError, match="shape"):
        paged_decode_attention(q, kp, vp, table, k_new=torch.zeros(2, 2, 64),
                               v_new=torch.zeros(2, 2, 64))
    with pytest.raises(TypeError, match="same dtype"):
        paged_decode_attention(q, kp, vp, table, k_new=torch.zeros(2, 2, 128),
                               v_new=torch.zeros(2, 2, 128, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="HIP"):
        paged_decode_attention(q, kp, vp, table)


def test_fused_append_arguments_of_the_contiguous_decode():
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import QuantizedTensor

    def qt(nbits=4):
        P = 8 // nbits
        return QuantizedTensor(torch.zeros(1, 2, 64, 128 // P, dtype=torch.uint8),
                               torch.ones(1, 2, 64, 4, dtype=torch.float16),
                               torch.zeros(1, 2, 64, 4, dtype=torch.float16), nbits, 32, 128)

    q = torch.zeros(1, 8, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="k_new and v_new"):
        fused_decode_attention(q, qt(), qt(), v_new=torch.zeros(1, 2, 128))
    with pytest.raises(TypeError, match="float16 or float32"):
        fused_decode_attention(q, qt(), qt(), k_new=torch.zeros(1, 2, 128, dtype=torch.int32),
                               v_new=torch.zeros(1, 2, 128, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="HIP"):
        fused_decode_attention(q, qt(), qt(), k_new=torch.zeros(1, 2, 1, 128),
                               v_new=torch.zeros(1, 2, 1, 128))


def test_paged_append_requires_a_gpu_tensor():
    from tritonkv_amd.paged import paged_append

    with pytest.raises(RuntimeError, match="GPU"):
        paged_append(_pool(), torch.zeros(1, 2, 1, 128), torch.zeros(1, 2, dtype=torch.int32),
                     torch.zeros(1, dtype=torch.int32))


def test_wave_count_policy():
    from tritonkv_amd.kernels.fused_decode_attn import (TWELVE_WAVES_MIN_SPLIT, choose_waves,
                                                        twelve_wave_format)

    fmt = dict(D=128, k_nbits=2, v_nbits=2, group_size=32)
    # Llama-3-8B shape, 2-bit gs32 (G = 4): one 32768-token split per unit -> 12 waves
    assert choose_waves(32, 8, 4, 32768, 1, **fmt) == 12
    # the same format below the split threshold, or in a wider GQA group, or paged -> 8
    assert choose_waves(32, 8, 4, TWELVE_WAVES_MIN_SPLIT - 64, 1, **fmt) == 8
    assert choose_waves(1, 2, 6, 32768, 1, **fmt) == 8
    assert choose_waves(32, 8, 4, 32768, 1, paged=True, **fmt) == 8
    # gs128 with equal bits, any group -> 12; the 4-bit gs32 headline, mixed
    # bits, head_dim 64 and the fp16 control (the default format) -> 8
    assert choose_waves(32, 8, 4, 32768, 1, D=128, k_nbits=4, v_nbits=4, group_size=128) == 12
    assert choose_waves(32, 8, 4, 32768, 1, D=128, k_nbits=4, v_nbits=4, group_size=32) == 8
    assert choose_waves(64, 8, 8, 65536, 2, D=128, k_nbits=4, v_nbits=2, group_size=32) == 8
    assert choose_waves(32, 8, 4, 32768, 1, D=64, k_nbits=2, v_nbits=2, group_size=32) == 8
    assert choose_waves(32, 8, 4, 32768, 1) == 8
    assert not twelve_wave_format(128, 4, 4, 2, 128)
    # short splits keep the 4 / 8 rule
    assert choose_waves(1, 2, 6, 128, 16, **fmt) == 4


def test_split_policy_fills_the_device_at_mid_batches():
    from tritonkv_amd.kernels.fused_decode_attn import (TOKENS_PER_WORKGROUP_FP16, choose_waves,
                                                        plan_splits)

    # Llama-3-8B (256 units) and long histories stay unsplit, 8 waves
    assert plan_splits(32768, 64, None, 32, 8, 4)[1] == 1
    # mid-size batch: about one workgroup per CU, >= 512 tokens each
    _, ns, size = plan_splits(32768, 64, None, 16, 2, 6)
    assert ns * 16 * 2 == 256 and size >= 512 and choose_waves(16, 2, 6, size, ns) == 8
    # Qwen2.5-1.5B B=1: at least 32 workgroups, never more than the history allows
    _, ns, size = plan_splits(2048, 64, None, 1, 2, 6)
    assert ns * 2 >= 32 and size >= 128
    assert plan_splits(512, 64, None, 1, 2, 6)[1] == 1
    # the fp16 control cuts shorter (its tokens are larger)
    assert plan_splits(16384, 64, None, 1, 2, 6, TOKENS_PER_WORKGROUP_FP16)[1] > \
        plan_splits(16384, 64, None, 1, 2, 6)[1]
    # an explicit num_splits is honoured after the reference's clamp and tighten
    assert plan_splits(1000, 64, 5, 1, 2, 6)[1] == 4
