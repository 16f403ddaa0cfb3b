"""Hugging Face ``transformers`` integration: decode through the fused kernel.

The reference plans this as its next step (``docs/future_work.md:187-210``):
a custom ``Cache`` that quantizes each new token as it is appended, and an
attention function registered with ``AttentionInterface`` that keeps prefill on
fp16 SDPA and runs decode (``q_len == 1``) on the fused kernel.  Here:

* :class:`TkvCache` -- a ``transformers`` ``Cache`` made of :class:`TkvLayer`,
  one preallocated contiguous cache per layer (capacity fixed up front),
  either quantized (``nbits`` 2 or 4: split-P codes with fp16 scale/zero) or
  fp16 (``nbits=16``: the control).  Prefill puts the prompt's K/V into it
  (the GPU quantize/pack append for 2/4 bits).  A decode step only advances
  the length: the new token's K/V reach the attention call, which appends them
  inside the split kernel (``k_new``/``v_new``), so a quantized decode step is
  one launch per layer.  ``keys="channel"`` instead keeps per-channel
  (KIVI-style) keys with an fp16 window (:class:`~tritonkv_amd.channel.ChannelKVCache`,
  the key format of ``docs/future_work.md:229-293``); its decode step keeps
  the window fill and the flush decision on the device, so it is
  graph-capturable too.
* ``"tkv"`` -- the attention function (:func:`register`): SDPA over the prompt
  for prefill; for decode, :func:`~tritonkv_amd.kernels.fused_decode_attention`
  over the quantized cache, or the fp16 control
  :func:`~tritonkv_amd.kernels.fp16_decode_attention` over the fp16 one.

Usage::

    from tritonkv_amd import hf
    hf.register()
    model.set_attn_implementation("tkv")
    cache = hf.TkvCache(model.config, capacity=8192, nbits=4)
    out = model.generate(input_ids, past_key_values=cache, max_new_tokens=64)

All rows of a batch share one length: a prefill whose mask hides key
positions (a left-padded batch) raises ``NotImplementedError`` rather than
letting decode attend to the pad tokens.  Chunked prefill into a non-empty
cache is not supported.  ``transformers`` is imported lazily, so the
rest of the package does not depend on it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .channel import ChannelKVCache
from .kernels import fp16_decode_attention, fused_decode_attention
from .quantize import append_kv, empty_cache

ATTN_NAME = "tkv"

try:  # the base classes exist only when transformers is importable
    from transformers.cache_utils import Cache as _Cache
    from transformers.cache_utils import CacheLayerMixin as _LayerBase
except ImportError:  # pragma: no cover - transformers is part of this image
    _Cache = object
    _LayerBase = object


class TkvLayer(_LayerBase):
    """One decoder layer's KV cache: ``(B, HKV, capacity, ...)``, preallocated."""

    is_compileable = False
    is_sliding = False

    def __init__(self, capacity: int, nbits: int = 4, group_size: int = 32, keys: str = "token"):
        if _LayerBase is not object:
            super().__init__()
        self.keys = self.values = None
        self.is_initialized = False
        if nbits not in (2, 4, 16):
            raise ValueError(f"nbits must be 2, 4 or 16, got {nbits}")
        if keys not in ("token", "channel") or (keys == "channel" and nbits == 16):
            raise ValueError(f"keys must be 'token' or (2/4 bits) 'channel', got {keys!r}")
        self.capacity, self.nbits, self.group_size = capacity, nbits, group_size
        self.key_format = keys
        self.length = 0  # tokens held (the same for every row)

    # -- storage ---------------------------------------------------------------
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, HKV, _, D = key_states.shape
        self.dtype, self.device = key_states.dtype, key_states.device
        if self.key_format == "channel":
            self.cc = ChannelKVCache(B, HKV, self.capacity, D, k_nbits=self.nbits,
                                     v_nbits=self.nbits, group_size=self.group_size,
                                     device=self.device)
            self.keys, self.values = self.cc.keys.packed, self.cc.values.packed
        elif self.nbits == 16:
            self.kc = torch.zeros(B, HKV, self.capacity, D, dtype=torch.float16, device=self.device)
            self.vc = torch.zeros_like(self.kc)
            self.keys, self.values = self.kc, self.vc
        else:
            self.kc = empty_cache(B, HKV, self.capacity, D, self.nbits, self.group_size, self.device)
            self.vc = empty_cache(B, HKV, self.capacity, D, self.nbits, self.group_size, self.device)
            for t in (self.kc.packed, self.kc.scale, self.kc.zero, self.vc.packed, self.vc.scale,
                      self.vc.zero):
                t.zero_()
            self.keys, self.values = self.kc.packed, self.vc.packed
        self.lens = torch.zeros(B, dtype=torch.int32, device=self.device)
        self.workspace: dict = {}
        self.out = None  # (B, HQ, D) float32, allocated at the first decode step
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.shape[-2]
        if self.length + n > self.capacity:
            raise ValueError(f"cache capacity {self.capacity} exceeded ({self.length} + {n} tokens)")
        if n == 1 and self.length > 0:
            # decode: the attention call appends the token (fused append).  The
            # device-side length is advanced on the device, so a captured
            # decode step stays right when its graph is replayed.
            self.length += 1
            self.lens.add_(1)
            key_states._tkv_layer = self
            return key_states, value_states
        if self.length:
            raise NotImplementedError("prefill into a non-empty TkvCache (chunked prefill)")
        if self.key_format == "channel":
            self.cc.extend(key_states, value_states)
        elif self.nbits == 16:
            self.kc[:, :, :n] = key_states
            self.vc[:, :, :n] = value_states
        else:
            append_kv(self.kc, key_states.to(torch.float16).contiguous())
            append_kv(self.vc, value_states.to(torch.float16).contiguous())
        self.length = n
        self.lens.fill_(n)
        key_states._tkv_prefill = self
        return key_states, value_states

    # -- sizes -------------------------------------------------------------------
    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_seq_length(self) -> int:
        return self.length

    def get_max_length(self) -> int:
        return self.capacity

    def reset(self) -> None:
        self.length = 0
        if self.is_initialized:
            self.lens.zero_()
            if self.key_format == "channel":
                self.cc.reset()

    def decode(self, module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
               scaling: float) -> torch.Tensor:
        """Attention of the single new query over the cache (with the new token)."""
        B, HQ, _, D = query.shape
        if self.out is None:
            self.out = torch.empty(B, HQ, D, dtype=torch.float32, device=query.device)
        q = query[:, :, 0].to(torch.float16)
        if self.key_format == "channel":
            out = self.cc.step(key, value, q, sm_scale=scaling, out=self.out)
        elif self.nbits == 16:
            pos = (self.lens[:1] - 1).long()  # all rows share one length
            self.kc.index_copy_(2, pos, key.to(torch.float16))
            self.vc.index_copy_(2, pos, value.to(torch.float16))
            out = fp16_decode_attention(q, self.kc, self.vc, sm_scale=scaling, out=self.out,
                                        _workspace=self.workspace, seq_lens=self.lens,
                                        equal_lengths=True)
        else:
            # every row holds the same length: the split plan of an unragged
            # batch, and no uneven tail for a dispatch order to fix
            out = fused_decode_attention(q, self.kc, self.vc, sm_scale=scaling, out=self.out,
                                         _workspace=self.workspace, seq_lens=self.lens,
                                         k_new=key[:, :, 0].to(torch.float16),
                                         v_new=value[:, :, 0].to(torch.float16),
                                         equal_lengths=True)
        return out.to(query.dtype).view(B, 1, HQ, D)


class TkvCache(_Cache):
    """A ``transformers`` cache of :class:`TkvLayer`, one per decoder layer."""

    def __init__(self, config, capacity: int, nbits: int = 4, group_size: int = 32,
                 keys: str = "token"):
        cfg = config.get_text_config() if hasattr(config, "get_text_config") else config
        layers = [TkvLayer(capacity, nbits, group_size, keys) for _ in range(cfg.num_hidden_layers)]
        super().__init__(layers=layers)

    @property
    def nbytes(self) -> int:
        """Device bytes held by the caches of all layers."""
        total = 0
        for layer in self.layers:
            if layer.is_initialized and layer.key_format == "channel":
                total += layer.cc.nbytes()
            elif layer.is_initialized:
                cs = (layer.kc, layer.vc)
                if layer.nbits == 16:
                    total += sum(c.numel() * c.element_size() for c in cs)
                else:
                    total += sum(c.nbytes() for c in cs)
        return total


def _masks_keys(mask) -> bool:
    """Whether a prefill mask hides any key position from the prompt's last
    query (padding; causal masking never hides a key from the last query).
    ``mask``: None, bool (True = attend) or additive float, (..., q_len, kv_len)."""
    if mask is None:
        return False
    last = mask[..., -1, :]
    if last.dtype == torch.bool:
        return not bool(last.all())
    return bool((last < 0).any())


def tkv_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """``AttentionInterface`` entry: (B, HQ, q_len, D) query -> (B, q_len, HQ, D)."""
    layer = getattr(key, "_tkv_layer", None)
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    if layer is not None and query.shape[2] == 1:
        return layer.decode(module, query, key, value, scaling), None
    # prefill (or no TkvCache): fp16 SDPA over the given keys and values
    if getattr(key, "_tkv_prefill", None) is not None and _masks_keys(attention_mask):
        raise NotImplementedError(
            "TkvCache keeps one length for every row of the batch, and decode attends to "
            "every cached token: a prompt mask that hides key positions (a padded batch) "
            "would put the pad tokens into every decode step. Prefill rows of equal length.")
    groups = query.shape[1] // key.shape[1]
    if groups > 1:
        key = key.repeat_interleave(groups, dim=1)
        value = value.repeat_interleave(groups, dim=1)
    if attention_mask is None:
        out = F.scaled_dot_product_attention(query, key, value, is_causal=query.shape[2] > 1,
                                             scale=scaling)
    else:
        out = F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask,
                                             scale=scaling)
    return out.transpose(1, 2).contiguous(), None


def register() -> str:
    """Register ``"tkv"`` with ``transformers``' attention and mask interfaces."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

    AttentionInterface.register(ATTN_NAME, tkv_attention)
    AttentionMaskInterface.register(ATTN_NAME, sdpa_mask)
    return ATTN_NAME


__all__ = ["ATTN_NAME", "TkvLayer", "TkvCache", "tkv_attention", "register"]
