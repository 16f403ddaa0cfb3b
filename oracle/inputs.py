"""Seeded synthetic inputs -- test infrastructure only.

``make_random_kv`` restates ``reference.py:361-392``: one CPU
``torch.Generator`` seeded with ``seed``; for q ``(B, HQ, D)``, then k and v
``(B, HKV, S, D)`` in that order, ``randn`` in fp32, and -- only when
``outlier_frac > 0`` -- a second ``rand`` draw of the same shape whose entries
below ``outlier_frac`` scale the value by ``outlier_scale``; then cast to
``dtype``.  It uses torch's own CPU generator because "the same seeded inputs"
means the reference's RNG stream, which only torch reproduces.  It returns CPU
tensors; callers move them to the device.

``make_outlier_channel_kv`` is the Llama-3-8B benchmark configuration's input:
N(0,1) K/V with, per KV head, ``n_outlier_channels`` seeded channel indices
scaled by ``outlier_scale`` for every batch row and token.  The reference has
no generator for it (its generator draws element-wise outliers), so this one is
defined here.

``ragged_lengths`` draws the 70B-style configuration's per-sequence context
lengths, uniform in ``[lo, hi]`` from a seeded generator.
"""

from __future__ import annotations

import torch


def make_random_kv(B, HQ, HKV, S, D, dtype=torch.float16, seed=0,
                   outlier_frac=0.01, outlier_scale=8.0):
    g = torch.Generator(device="cpu").manual_seed(seed)

    def _rand(*shape):
        x = torch.randn(*shape, generator=g, dtype=torch.float32)
        if outlier_frac > 0:
            m = torch.rand(*shape, generator=g) < outlier_frac
            x = torch.where(m, x * outlier_scale, x)
        return x.to(dtype=dtype)

    q = _rand(B, HQ, D)
    k = _rand(B, HKV, S, D)
    v = _rand(B, HKV, S, D)
    return q, k, v


def make_outlier_channel_kv(B, HQ, HKV, S, D, dtype=torch.float16, seed=0,
                            n_outlier_channels=4, outlier_scale=8.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, HQ, D, generator=g, dtype=torch.float32).to(dtype)
    chans = torch.stack([torch.randperm(D, generator=g)[:n_outlier_channels]
                         for _ in range(HKV)])            # (HKV, n)
    mult = torch.ones(HKV, D)
    mult.scatter_(1, chans, outlier_scale)

    def _rand():
        x = torch.randn(B, HKV, S, D, generator=g, dtype=torch.float32)
        return (x * mult[None, :, None, :]).to(dtype)

    k = _rand()
    v = _rand()
    return q, k, v, chans


def ragged_lengths(B, lo, hi, seed=0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int64)
