"""tritonkv_amd: MI355X-native fused quantized-KV decode attention.

A from-scratch gfx950 implementation of tritonkv's hot path -- the 2/4-bit
split-P fused decode-attention kernel, its fp16 control, the split-combine
kernel and a GPU quantize/pack append kernel -- behind the reference's own call
surface:

* ``tritonkv_amd.kernels``: ``fused_decode_attention``, ``fp16_decode_attention``,
  ``pick_num_splits``, ``triton_available`` (reference ``kernels/__init__.py``);
* ``tritonkv_amd.quantize``: ``QuantizedTensor`` and the split-P
  pack/scale/zero layout (reference ``quantize.py``), plus ``append_kv``;
* ``tritonkv_amd.paged``: the same cache format in page pools addressed
  through a block table (``paged_append``, ``paged_decode_attention``);
* ``tritonkv_amd.channel``: per-channel (KIVI-style) keys with an fp16
  residual window, the key format the reference plans
  (``ChannelKVCache``, ``channel_decode_attention``);
* ``tritonkv_amd.hf``: a ``transformers`` cache and attention function.

The kernels live in ``libtkv_hip.so`` (C ABI in ``include/tkv.h``), built by
``python -m tritonkv_amd.build``.  There is no CPU or Triton fallback.
"""

from .quantize import (  # noqa: F401
    QuantizedTensor,
    append_kv,
    dequantize_groupwise,
    empty_cache,
    pack_codes,
    quantize_groupwise,
    quantize_kv,
    unpack_codes,
)

__version__ = "0.1.0"
