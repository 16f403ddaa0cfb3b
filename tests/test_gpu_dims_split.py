"""GPU parity of the dims-split kernels.

A small grid (at most half as many workgroups as the GPU has CUs) of a
format with 8 head columns (GQA groups of 5-8 heads, groups of 32, equal K/V
bits) runs every (unit, split) as two workgroups, each computing all scores
but the V products and the merge of half the head dim.  Each part performs
the one-workgroup kernel's own operations on its dims, so the output must be
*bit-identical* to the same step through a page pool, which never splits the
dims (same kernel arithmetic, one workgroup).  Shapes are the Qwen2.5-1.5B
batch-1 shape (HQ=12, HKV=2): rows of hi/lo probabilities (<= 256 tokens), one
unsplit row, split rows with a tail chunk, ragged lengths with empty splits,
and the fused append.
"""

from __future__ import annotations

import pytest
import torch

from oracle import inputs as oinp
from tests.helpers import assert_close_to_reference, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
PAGE = 64


def _pool(qt, table, num_pages):
    from tritonkv_amd.paged import empty_paged_pool

    B, H, S, _ = qt.packed.shape
    mp = S // PAGE
    pool = empty_paged_pool(num_pages, H, PAGE, qt.head_dim, qt.nbits, qt.group_size, DEV)
    for src, dst in ((qt.packed, pool.packed), (qt.scale, pool.scale), (qt.zero, pool.zero)):
        dst.view(torch.uint8).fill_(0xFF)
        dst[table.long()] = src.reshape(B, H, mp, PAGE, src.shape[-1]).permute(0, 2, 1, 3, 4)
    return pool


def _table(B, mp, num_pages, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(num_pages, generator=g)[:B * mp].reshape(B, mp).to(torch.int32).to(DEV)


@pytest.mark.parametrize("nbits", [4, 2])
@pytest.mark.parametrize("S", [192, 512, 2048, 9024])
def test_dims_split_is_bit_identical_to_one_workgroup(nbits, S):
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.paged import paged_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D = 1, 12, 2, 128
    print(f"dims split nbits={nbits} S={S}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=S + nbits)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, nbits, 32), quantize_groupwise(v, nbits, 32)
    mp = S // PAGE
    num_pages = B * mp + 3
    table = _table(B, mp, num_pages, seed=S)
    kp, vp = _pool(kq, table, num_pages), _pool(vq, table, num_pages)
    for ns in (None, 1, 3):
        got = fused_decode_attention(q, kq, vq, num_splits=ns)
        want = paged_decode_attention(q, kp, vp, table, None, num_splits=ns)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), (ns, (got - want).abs().max().item())
    assert_close_to_reference(got, oracle_attention_on_quant(q, kq, vq), f"nbits={nbits} S={S}")


def test_dims_split_ragged_rows_and_empty_splits():
    """Rows of different lengths, so that some splits of the short rows are
    empty (the empty partial is written by both halves of the dims)."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.paged import paged_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, S = 3, 12, 2, 128, 4096
    print("dims split ragged", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=77)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, 4, 32), quantize_groupwise(v, 4, 32)
    lens = torch.tensor([S, 100, 1500], dtype=torch.int32, device=DEV)
    mp = S // PAGE
    num_pages = B * mp + 5
    table = _table(B, mp, num_pages, seed=78)
    kp, vp = _pool(kq, table, num_pages), _pool(vq, table, num_pages)
    for ns in (4, 8):
        got = fused_decode_attention(q, kq, vq, num_splits=ns, seq_lens=lens)
        want = paged_decode_attention(q, kp, vp, table, lens, num_splits=ns)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (ns, (got - want).abs().max().item())
    assert_close_to_reference(got, oracle_attention_on_quant(q, kq, vq, seq_lens=lens.cpu()),
                              "ragged dims split")


def test_dims_split_fused_append():
    """The decode step with the new token appended inside the launch: the
    output and every cache byte must equal the paged step's (part 0 of the
    first head block stores the row; both parts patch their own copy)."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.paged import paged_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, S = 2, 12, 2, 128, 1024
    print("dims split fused append", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=91)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, 4, 32), quantize_groupwise(v, 4, 32)
    mp = S // PAGE
    num_pages = B * mp + 2
    table = _table(B, mp, num_pages, seed=92)
    kp, vp = _pool(kq, table, num_pages), _pool(vq, table, num_pages)
    g = torch.Generator().manual_seed(93)
    for step in range(3):
        lens = torch.tensor([S - 10 + step, 700 + step], dtype=torch.int32, device=DEV)
        kn = torch.randn(B, HKV, D, generator=g).half().to(DEV)
        vn = torch.randn(B, HKV, D, generator=g).half().to(DEV)
        got = fused_decode_attention(q, kq, vq, seq_lens=lens, k_new=kn, v_new=vn)
        want = paged_decode_attention(q, kp, vp, table, lens, k_new=kn, v_new=vn)
        torch.cuda.synchronize()
        assert torch.equal(got, want), step
    idx = table.long()
    for c, p in ((kq, kp), (vq, vp)):
        for src, dst in ((c.packed, p.packed), (c.scale, p.scale), (c.zero, p.zero)):
            assert torch.equal(dst[idx], src.reshape(B, HKV, mp, PAGE, src.shape[-1]).permute(0, 2, 1, 3, 4))
