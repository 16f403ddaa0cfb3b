"""Seeded synthetic inputs of the large decode configurations, drawn on the GPU.

The Llama-3-8B and 70B-style workloads hold 4-17 GB of fp16 K/V.  Drawing that
from a CPU generator takes about a minute per cache, so these inputs come from
the device's own generator (torch's Philox) in a fixed order: a seed always
gives the same tensors on the same device type.  ``bench.py`` times exactly
these inputs, and the GPU tests check the kernels on them -- sampled (batch
row, kv head) units against the CPU oracle on the very same values copied back
to the host.

* :func:`outlier_channel_kv` -- the Llama-3-8B configuration: q, K, V fp16
  N(0,1), with ``n_outlier_channels`` channel indices per KV head (drawn once,
  shared by every batch row and token) scaled by ``outlier_scale``.
* :func:`ragged_lengths` -- per-sequence context lengths uniform in
  ``[lo, hi]`` (a CPU generator: B numbers).
* :func:`ragged_row_kv` -- the fp16 history of one batch row of the 70B-style
  configuration, from a generator of its own, so any row can be redrawn alone.
* :func:`ragged_batch` -- that configuration's quantized caches (K and V bit
  widths of the caller's choice, per-row lengths, fixed capacity), q and the
  step's new K/V token per sequence.
"""

from __future__ import annotations

import torch


def outlier_channel_kv(B, HQ, HKV, S, D, seed=0, n_outlier_channels=4, outlier_scale=8.0,
                       device="cuda", dtype=torch.float16):
    """``(q, k, v, chans)``: q ``(B, HQ, D)``, k and v ``(B, HKV, S, D)``, chans
    ``(HKV, n_outlier_channels)`` the scaled channels of each KV head.  Draw
    order: q, the channel permutations (one per KV head), k, then v."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, HQ, D, device=device, generator=g, dtype=torch.float32).to(dtype)
    chans = torch.stack([torch.randperm(D, device=device, generator=g)[:n_outlier_channels]
                         for _ in range(HKV)])
    mult = torch.ones(HKV, D, device=device, dtype=dtype)
    mult.scatter_(1, chans, outlier_scale)
    out = []
    for _ in range(2):
        x = torch.randn(B, HKV, S, D, device=device, generator=g, dtype=dtype)
        x.mul_(mult[None, :, None, :])
        out.append(x)
    return q, out[0], out[1], chans


def ragged_lengths(B, lo, hi, seed=0):
    """int32 ``(B,)`` lengths uniform in ``[lo, hi]`` (CPU generator)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)


def _row_seed(seed: int, b: int) -> int:
    # batch row b >= 0; b = -1 is the generator of q and the new tokens
    return seed * 1_000_003 + 7919 * (b + 1) + 1


def ragged_row_kv(seed, b, HKV, L, D, device="cuda", dtype=torch.float16):
    """fp16 ``(k, v)``, each ``(HKV, L, D)`` N(0,1): the first L tokens of batch
    row b (draw order k then v, from the row's own generator)."""
    g = torch.Generator(device=device).manual_seed(_row_seed(seed, b))
    k = torch.randn(HKV, L, D, device=device, generator=g, dtype=dtype)
    v = torch.randn(HKV, L, D, device=device, generator=g, dtype=dtype)
    return k, v


def ragged_batch(B, HQ, HKV, D, lengths, capacity, k_nbits, v_nbits, group_size, seed=0,
                 device="cuda"):
    """The 70B-style decode step's inputs: ``(q, kc, vc, k_new, v_new)``.

    ``kc`` / ``vc`` are quantized caches of ``capacity`` tokens per (b, kv
    head); row b holds its ``lengths[b]`` tokens (:func:`ragged_row_kv`,
    quantized on the GPU) and the rest of the row is never written.  q is
    ``(B, HQ, D)``, ``k_new`` / ``v_new`` are ``(B, HKV, 1, D)``, all fp16 N(0,1)
    from one more generator (draw order q, k_new, v_new)."""
    from .quantize import QuantizedTensor, append_kv, empty_cache

    lens = [int(x) for x in lengths]
    if max(lens) > capacity:
        raise ValueError(f"a length exceeds the capacity {capacity}")
    kc = empty_cache(B, HKV, capacity, D, k_nbits, group_size, device)
    vc = empty_cache(B, HKV, capacity, D, v_nbits, group_size, device)
    for b in range(B):
        k, v = ragged_row_kv(seed, b, HKV, lens[b], D, device)
        for cache, x in ((kc, k), (vc, v)):
            row = QuantizedTensor(cache.packed[b:b + 1], cache.scale[b:b + 1],
                                  cache.zero[b:b + 1], cache.nbits, group_size, D)
            append_kv(row, x[None])
        del k, v
    g = torch.Generator(device=device).manual_seed(_row_seed(seed, -1))
    q = torch.randn(B, HQ, D, device=device, generator=g, dtype=torch.float16)
    k_new = torch.randn(B, HKV, 1, D, device=device, generator=g, dtype=torch.float16)
    v_new = torch.randn(B, HKV, 1, D, device=device, generator=g, dtype=torch.float16)
    return q, kc, vc, k_new, v_new
