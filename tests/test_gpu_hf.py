"""The kernels inside a ``transformers`` model (``tritonkv_amd.hf``).

A small random-initialised Qwen2 model (head_dim 64, GQA 4) runs prefill and
greedy decode three ways: stock SDPA with ``DynamicCache``, ``"tkv"`` over an
fp16 :class:`TkvCache` (the fp16 control kernel), and ``"tkv"`` over a 4-bit
one (the fused kernel with the append fused into each decode step).  Every
quantized decode attention call made inside the model is checked against the
oracle's dequantise-then-attend on the cache it ran on, and the row the fused
append wrote against the oracle quantizer.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant as oq
from tests.helpers import assert_close_to_reference, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
transformers = pytest.importorskip("transformers")

PROMPT, STEPS = 40, 8


def _model():
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=4096)
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).half().to(DEV).eval()


def _run(model, cache, ids, forced=None):
    """Prefill, then STEPS decode steps; tokens are the model's greedy choice
    unless ``forced`` gives them.  Returns (tokens, per-step logits)."""
    logits, toks = [], []
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        for s in range(STEPS):
            lg = out.logits[:, -1].float()
            logits.append(lg)
            nxt = lg.argmax(-1, keepdim=True) if forced is None else forced[s]
            toks.append(nxt)
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
    return toks, logits


def test_fp16_control_inside_the_model_matches_stock_sdpa():
    from transformers import DynamicCache

    from tritonkv_amd import hf

    hf.register()
    model = _model()
    ids = torch.randint(0, 512, (2, PROMPT), generator=torch.Generator().manual_seed(1)).to(DEV)
    model.set_attn_implementation("sdpa")
    toks, ref = _run(model, DynamicCache(config=model.config), ids)
    model.set_attn_implementation(hf.ATTN_NAME)
    cache = hf.TkvCache(model.config, capacity=128, nbits=16)
    _, got = _run(model, cache, ids, forced=toks)
    assert cache.get_seq_length() == PROMPT + STEPS
    for s, (a, b) in enumerate(zip(got, ref)):
        err = (a - b).abs().max().item() / b.abs().max().item()
        assert err < 2e-2, (s, err)


def test_quantized_decode_inside_the_model_matches_the_oracle(monkeypatch):
    from tritonkv_amd import hf

    hf.register()
    model = _model()
    model.set_attn_implementation(hf.ATTN_NAME)
    calls = []
    orig = hf.TkvLayer.decode

    def checked(self, module, query, key, value, scaling):
        out = orig(self, module, query, key, value, scaling)
        q = query[:, :, 0].to(torch.float16)
        ref = oracle_attention_on_quant(q, self.kc, self.vc, sm_scale=scaling,
                                        seq_lens=self.lens.cpu().numpy())
        assert_close_to_reference(self.out, ref, f"layer decode at length {self.length}")
        pos = self.length - 1  # the row the fused append wrote
        for cache, x in ((self.kc, key), (self.vc, value)):
            want = oq.quantize_groupwise(x.to(torch.float16).cpu().numpy(), cache.nbits,
                                         cache.group_size)
            assert np.array_equal(cache.packed[:, :, pos].cpu().numpy(), want.packed[:, :, 0])
            assert np.array_equal(cache.scale[:, :, pos].cpu().numpy().view(np.uint16),
                                  want.scale[:, :, 0].view(np.uint16))
        calls.append(self.length)
        return out

    monkeypatch.setattr(hf.TkvLayer, "decode", checked)
    ids = torch.randint(0, 512, (2, PROMPT), generator=torch.Generator().manual_seed(2)).to(DEV)
    cache = hf.TkvCache(model.config, capacity=128, nbits=4)
    toks, got = _run(model, cache, ids)
    assert len(calls) == STEPS * model.config.num_hidden_layers
    assert cache.get_seq_length() == PROMPT + STEPS
    assert cache.nbytes > 0
    # against the fp16 control on the same tokens: same model, a 4-bit cache
    cache16 = hf.TkvCache(model.config, capacity=128, nbits=16)
    monkeypatch.setattr(hf.TkvLayer, "decode", orig)
    _, ref = _run(model, cache16, ids, forced=toks)
    for a, b in zip(got, ref):
        assert torch.isfinite(a).all()
        cos = torch.nn.functional.cosine_similarity(a, b, dim=-1).min().item()
        assert cos > 0.99, cos


def test_generate_with_tkv_cache():
    from tritonkv_amd import hf

    hf.register()
    model = _model()
    model.set_attn_implementation(hf.ATTN_NAME)
    ids = torch.randint(0, 512, (1, 16), generator=torch.Generator().manual_seed(3)).to(DEV)
    cache = hf.TkvCache(model.config, capacity=64, nbits=4)
    out = model.generate(ids, past_key_values=cache, max_new_tokens=6, do_sample=False)
    assert out.shape == (1, 22)
    assert cache.get_seq_length() == 21  # the last generated token is never fed back


def test_channel_keys_inside_the_model():
    """keys="channel": per-channel keys plus an fp16 window; the window flushes
    into the quantized history during decode (60-token prompt, 8 steps)."""
    from tritonkv_amd import hf

    hf.register()
    model = _model()
    model.set_attn_implementation(hf.ATTN_NAME)
    ids = torch.randint(0, 512, (2, 60), generator=torch.Generator().manual_seed(4)).to(DEV)
    cache16 = hf.TkvCache(model.config, capacity=128, nbits=16)
    toks, ref = _run(model, cache16, ids)
    cache = hf.TkvCache(model.config, capacity=128, nbits=4, keys="channel")
    _, got = _run(model, cache, ids, forced=toks)
    layer = cache.layers[0]
    assert cache.get_seq_length() == 68
    assert (layer.cc.quantized, layer.cc.window) == (64, 4)
    assert cache.nbytes > 0
    for a, b in zip(got, ref):
        assert torch.isfinite(a).all()
        cos = torch.nn.functional.cosine_similarity(a, b, dim=-1).min().item()
        assert cos > 0.99, cos
