"""Restatement of the reference's host-side split arithmetic -- test infrastructure.

``kernels/fused_decode_attn.py``:

* ``_next_pow2`` ``:398-399``;
* ``pick_num_splits`` ``:402-416``: ``want = max(1, target // max(1, B*HKV))``,
  clamped to ``[1, n_blocks]``;
* the block/split tightening in ``fused_decode_attention`` ``:486-499``:
  ``block_n = min(block_n, max(16, next_pow2(S)))``; ``n_blocks = cdiv(S,
  block_n)``; ``ns = clamp(ns, 1, n_blocks)``; ``bps = cdiv(n_blocks, ns)``;
  ``ns = cdiv(n_blocks, bps)``; ``split_size = bps * block_n``.
"""

from __future__ import annotations


def next_pow2(x: int) -> int:
    return 1 << (x - 1).bit_length()


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def pick_num_splits(B: int, HKV: int, n_blocks: int, target_programs: int) -> int:
    want = max(1, target_programs // max(1, B * HKV))
    return max(1, min(n_blocks, want))


def split_plan(S: int, block_n: int, num_splits: int):
    """Return (block_n, num_splits, split_size) after the reference's tightening."""
    block_n = min(block_n, max(16, next_pow2(S)))
    n_blocks = cdiv(S, block_n)
    ns = max(1, min(num_splits, n_blocks))
    bps = cdiv(n_blocks, ns)
    ns = cdiv(n_blocks, bps)
    return block_n, ns, bps * block_n
