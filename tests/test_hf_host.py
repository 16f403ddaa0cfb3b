"""Host-side checks of the transformers integration (no GPU): registration,
the prefill path (SDPA over the prompt, cache bookkeeping) against stock SDPA,
and a clean backend error at the first decode step."""

from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")


def _model():
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=256, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=1024)
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).eval()


def test_prefill_through_tkv_matches_stock_sdpa():
    from tritonkv_amd import hf

    assert hf.register() == "tkv"
    model = _model()
    ids = torch.randint(0, 256, (2, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        model.set_attn_implementation("sdpa")
        ref = model(input_ids=ids).logits
        model.set_attn_implementation("tkv")
        cache = hf.TkvCache(model.config, capacity=32, nbits=16)
        got = model(input_ids=ids, past_key_values=cache, use_cache=True).logits
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)
    assert cache.get_seq_length() == 12
    assert [layer.length for layer in cache.layers] == [12, 12]
    assert cache.layers[0].get_mask_sizes(1) == (13, 0)


def test_capacity_and_decode_errors_without_a_gpu():
    from tritonkv_amd import hf

    hf.register()
    model = _model()
    model.set_attn_implementation("tkv")
    ids = torch.randint(0, 256, (1, 8), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        with pytest.raises(ValueError, match="capacity"):
            model(input_ids=ids, past_key_values=hf.TkvCache(model.config, capacity=4, nbits=16))
        cache = hf.TkvCache(model.config, capacity=16, nbits=16)
        model(input_ids=ids, past_key_values=cache, use_cache=True)
        with pytest.raises(RuntimeError, match="HIP"):
            model(input_ids=ids[:, :1], past_key_values=cache, use_cache=True)
    with pytest.raises(ValueError, match="nbits"):
        hf.TkvLayer(16, nbits=8)


def test_channel_key_mode_arguments():
    from tritonkv_amd import hf

    with pytest.raises(ValueError):
        hf.TkvLayer(64, nbits=16, keys="channel")
    with pytest.raises(ValueError):
        hf.TkvLayer(64, nbits=4, keys="block")
    assert hf.TkvLayer(64, nbits=2, keys="channel").key_format == "channel"


def test_padded_prefill_into_a_tkv_cache_is_refused():
    """A left-padded batch (its mask hides key positions) cannot be stored with
    one shared length: the prefill raises instead of letting decode attend to
    the pad tokens.  An unpadded mask still prefills."""
    from tritonkv_amd import hf

    hf.register()
    model = _model()
    ids = torch.randint(0, 256, (2, 10), generator=torch.Generator().manual_seed(2))
    mask = torch.ones(2, 10, dtype=torch.long)
    mask[1, :3] = 0  # row 1 left-padded by 3 tokens
    model.set_attn_implementation("tkv")
    with torch.no_grad():
        cache = hf.TkvCache(model.config, capacity=32, nbits=16)
        with pytest.raises(NotImplementedError, match="padded batch"):
            model(input_ids=ids, attention_mask=mask, past_key_values=cache, use_cache=True)
        cache = hf.TkvCache(model.config, capacity=32, nbits=16)
        model(input_ids=ids, attention_mask=torch.ones_like(mask), past_key_values=cache,
              use_cache=True)
    assert cache.get_seq_length() == 10
    # the mask test itself: bool and additive forms, causal masking alone never counts
    causal = torch.ones(4, 4, dtype=torch.bool).tril()[None, None]
    assert not hf._masks_keys(None)
    assert not hf._masks_keys(causal)
    padded = causal.clone()
    padded[..., :, 0] = False
    assert hf._masks_keys(padded)
    additive = torch.zeros(1, 1, 4, 4).masked_fill(~padded, float("-inf"))
    assert hf._masks_keys(additive)
    assert not hf._masks_keys(torch.zeros(1, 1, 4, 4).masked_fill(~causal, float("-inf")))
