"""GPU parity of the paged cache: page pools addressed through a block table.

The paged decode must be *bit-identical* to the contiguous decode on a cache
holding the same logical tokens (same kernel arithmetic, only the addressing
differs), and the paged append must write exactly the rows the contiguous
append writes.  Pools are filled with 0xFF (fp16 NaN) first and pages are
scattered in random order, so a wrong page, slot or head lands on NaN garbage
or on another sequence's data and breaks equality.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs as oinp
from oracle import quant as oq
from tests.helpers import assert_close_to_reference, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _scatter_to_pool(qt, table, num_pages, page_size):
    """A NaN-filled pool holding contiguous cache ``qt`` in the pages of ``table``."""
    from tritonkv_amd.paged import empty_paged_pool

    B, H, S, _ = qt.packed.shape
    mp = S // page_size
    pool = empty_paged_pool(num_pages, H, page_size, qt.head_dim, qt.nbits, qt.group_size, DEV)
    idx = table.long()
    for src, dst in ((qt.packed, pool.packed), (qt.scale, pool.scale), (qt.zero, pool.zero)):
        dst.view(torch.uint8).fill_(0xFF)
        F = src.shape[-1]
        dst[idx] = src.reshape(B, H, mp, page_size, F).permute(0, 2, 1, 3, 4)
    return pool


def _random_table(B, max_pages, num_pages, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(num_pages, generator=g)[:B * max_pages].reshape(B, max_pages) \
        .to(torch.int32).to(DEV)


@pytest.mark.parametrize("page_size", [32, 64, 256])
@pytest.mark.parametrize("kbits,vbits,gs", [(4, 4, 32), (2, 2, 32), (4, 2, 32), (4, 4, 128)])
def test_paged_decode_is_bit_identical_to_contiguous(page_size, kbits, vbits, gs):
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.paged import paged_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, max_pages = 3, 16, 2, 128, 2048 // page_size + 1
    S = max_pages * page_size
    print(f"case page={page_size} K{kbits}/V{vbits} gs={gs} S={S}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=page_size + kbits)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, kbits, gs), quantize_groupwise(v, vbits, gs)
    num_pages = B * max_pages + 7
    table = _random_table(B, max_pages, num_pages, seed=page_size)
    kp = _scatter_to_pool(kq, table, num_pages, page_size)
    vp = _scatter_to_pool(vq, table, num_pages, page_size)
    for lens in (None, torch.tensor([S, 1, S - page_size - 5], dtype=torch.int32)):
        lens_d = lens.to(DEV) if lens is not None else None
        for ns in (None, 1, 5):
            want = fused_decode_attention(q, kq, vq, num_splits=ns, seq_lens=lens_d,
                                          allow_mixed_bits=True)
            got = paged_decode_attention(q, kp, vp, table, lens_d, num_splits=ns,
                                         allow_mixed_bits=True)
            torch.cuda.synchronize()
            assert torch.isfinite(got).all()
            assert torch.equal(got, want), (lens, ns, (got - want).abs().max().item())


def test_unused_table_entries_are_never_read():
    """Entries past each row's length may hold anything, even out-of-range
    page numbers: the kernel looks a page up only for chunks it streams."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.paged import paged_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, page, mp = 2, 8, 1, 128, 64, 10
    S = mp * page
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=41)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, 4, 32), quantize_groupwise(v, 4, 32)
    table = _random_table(B, mp, B * mp, seed=3)
    kp = _scatter_to_pool(kq, table, B * mp, page)
    vp = _scatter_to_pool(vq, table, B * mp, page)
    lens = torch.tensor([3 * page + 1, 7 * page], dtype=torch.int32, device=DEV)
    bad = table.clone()
    bad[0, 4:] = -5
    bad[1, 7:] = 1 << 30
    for ns in (None, 1, 4):
        want = fused_decode_attention(q, kq, vq, num_splits=ns, seq_lens=lens)
        got = paged_decode_attention(q, kp, vp, bad, lens, num_splits=ns)
        torch.cuda.synchronize()
        assert torch.equal(got, want), ns


@pytest.mark.parametrize("page_size", [32, 128])
def test_paged_append_then_decode_ragged(page_size):
    """Prefill each row through the paged append, append one token per row at
    its own position, then decode: the pool's rows must equal the contiguous
    append's bit for bit, and attention must match the oracle."""
    from tritonkv_amd.paged import empty_paged_pool, gather_pages, paged_append, \
        paged_decode_attention
    from tritonkv_amd.quantize import QuantizedTensor, append_kv, empty_cache

    B, HQ, HKV, D, gs = 4, 32, 4, 128, 32
    lens = torch.tensor([1500, 1, 617, page_size * 3 - 1], dtype=torch.int32)
    mp = (int(lens.max()) + 1 + page_size - 1) // page_size
    cap = mp * page_size
    print(f"case page={page_size} cap={cap}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, cap, D, seed=53)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    num_pages = B * mp + 3
    table = _random_table(B, mp, num_pages, seed=page_size + 1)
    pools, contig = [], []
    for nbits in (4, 2):
        p = empty_paged_pool(num_pages, HKV, page_size, D, nbits, gs, DEV)
        c = empty_cache(B, HKV, cap, D, nbits, gs, DEV)
        for t in (p.packed, p.scale, p.zero, c.packed, c.scale, c.zero):
            t.view(torch.uint8).fill_(0xFF)
        pools.append(p)
        contig.append(c)
    zero1 = torch.zeros(1, dtype=torch.int32, device=DEV)
    for b in range(B):
        L = int(lens[b])
        for p, c, x in ((pools[0], contig[0], k), (pools[1], contig[1], v)):
            xb = x[b:b + 1, :, :L].contiguous()
            paged_append(p, xb, table[b:b + 1], zero1)
            view = QuantizedTensor(c.packed[b:b + 1], c.scale[b:b + 1], c.zero[b:b + 1],
                                   c.nbits, gs, D)
            append_kv(view, xb)
    k_new, v_new = k[:, :, -1:].contiguous(), v[:, :, -1:].contiguous()
    pos = lens.to(DEV)
    for p, c, x in ((pools[0], contig[0], k_new), (pools[1], contig[1], v_new)):
        paged_append(p, x, table, pos)
        append_kv(c, x, pos)
    torch.cuda.synchronize()
    lens1 = lens + 1
    for p, c in zip(pools, contig):
        g = gather_pages(p, table)
        for b in range(B):
            L = int(lens1[b])
            for a, w in ((g.packed, c.packed), (g.scale, c.scale), (g.zero, c.zero)):
                assert torch.equal(a[b, :, :L].view(torch.uint8), w[b, :, :L].view(torch.uint8)), b
    # the appended token is the oracle quantizer's
    for p, x in ((pools[0], k_new), (pools[1], v_new)):
        g = gather_pages(p, table)
        want = oq.quantize_groupwise(x.cpu().numpy(), p.nbits, gs)
        for b in range(B):
            L = int(lens[b])
            assert np.array_equal(g.packed[b, :, L].cpu().numpy(), want.packed[b, :, 0])
            assert np.array_equal(g.scale[b, :, L].cpu().numpy().view(np.uint16),
                                  want.scale[b, :, 0].view(np.uint16))
    for ns in (None, 1, 6):
        got = paged_decode_attention(q, pools[0], pools[1], table, lens1.to(DEV), num_splits=ns,
                                     allow_mixed_bits=True)
        assert torch.isfinite(got).all(), ns
        clean = []
        for p in pools:
            g = gather_pages(p, table)
            for b in range(B):
                L = int(lens1[b])
                g.packed[b, :, L:] = 0
                g.scale[b, :, L:] = 0
                g.zero[b, :, L:] = 0
            clean.append(g)
        ref = oracle_attention_on_quant(q, clean[0], clean[1], seq_lens=lens1.numpy())
        assert_close_to_reference(got, ref, f"paged append + decode page={page_size} ns={ns}")


def test_paged_append_skips_positions_outside_the_table():
    from tritonkv_amd.paged import empty_paged_pool, paged_append

    HKV, D, page = 2, 64, 32
    pool = empty_paged_pool(4, HKV, page, D, 4, 32, DEV)
    for t in (pool.packed, pool.scale, pool.zero):
        t.view(torch.uint8).fill_(0xAB)
    before = [t.clone() for t in (pool.packed, pool.scale, pool.zero)]
    table = torch.tensor([[2, 9], [-1, 0]], dtype=torch.int32, device=DEV)
    x = torch.randn(2, HKV, 1, D, device=DEV, dtype=torch.float16)
    # row 0 at position 40 -> table entry 9 (out of pool); row 1 at 5 -> entry -1;
    paged_append(pool, x, table, torch.tensor([40, 5], dtype=torch.int32, device=DEV))
    # row 0 at 64 -> past the table; row 1 at 2000 -> past the table
    paged_append(pool, x, table, torch.tensor([64, 2000], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    for a, b in zip((pool.packed, pool.scale, pool.zero), before):
        assert torch.equal(a, b)
    # valid positions write exactly one slot of one page per (row, kv head):
    # row 0 at 5 -> page 2 slot 5; row 1 at 40 -> page 0 slot 8
    paged_append(pool, x, table, torch.tensor([5, 40], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    changed = sorted((pool.packed != before[0]).any(dim=-1).nonzero().tolist())
    assert changed == sorted([[2, h, 5] for h in range(HKV)] + [[0, h, 8] for h in range(HKV)])


def test_paged_step_replays_in_a_graph():
    """Append + decode captured once and replayed with new positions and
    lengths (the serving loop), against the eager calls."""
    from tritonkv_amd.paged import empty_paged_pool, paged_append, paged_decode_attention

    B, HQ, HKV, D, page, mp = 2, 16, 2, 128, 64, 8
    num_pages = B * mp
    table = _random_table(B, mp, num_pages, seed=11)
    kp = empty_paged_pool(num_pages, HKV, page, D, 4, 32, DEV)
    vp = empty_paged_pool(num_pages, HKV, page, D, 4, 32, DEV)
    for t in (kp.packed, kp.scale, kp.zero, vp.packed, vp.scale, vp.zero):
        t.zero_()
    g = torch.Generator(device="cpu").manual_seed(5)
    steps = 4
    xs = [torch.randn(B, HKV, 1, D, generator=g).half().to(DEV) for _ in range(2 * steps)]
    q = torch.randn(B, HQ, D, generator=g).half().to(DEV)
    pos = torch.tensor([100, 300], dtype=torch.int32, device=DEV)
    lens = pos + 1
    xk = torch.empty(B, HKV, 1, D, dtype=torch.float16, device=DEV)
    xv = torch.empty_like(xk)
    out = torch.empty(B, HQ, D, dtype=torch.float32, device=DEV)
    ws = {}

    def step():
        paged_append(kp, xk, table, pos)
        paged_append(vp, xv, table, pos)
        paged_decode_attention(q, kp, vp, table, lens, num_splits=3, out=out, _workspace=ws)

    xk.copy_(xs[0])
    xv.copy_(xs[1])
    step()  # warm-up: allocates the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    kp2 = [t.clone() for t in (kp.packed, kp.scale, kp.zero)]
    vp2 = [t.clone() for t in (vp.packed, vp.scale, vp.zero)]
    for i in range(steps):
        pos.add_(1)
        lens.copy_(pos + 1)
        xk.copy_(xs[2 * i])
        xv.copy_(xs[2 * i + 1])
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        # eager on copies of the pools as they were before this step
        from tritonkv_amd.quantize import QuantizedTensor
        ke = QuantizedTensor(*kp2, 4, 32, D)
        ve = QuantizedTensor(*vp2, 4, 32, D)
        paged_append(ke, xk, table, pos)
        paged_append(ve, xv, table, pos)
        want = paged_decode_attention(q, ke, ve, table, lens, num_splits=3)
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
        for a, b in zip((kp.packed, kp.scale, kp.zero, vp.packed, vp.scale, vp.zero),
                        (*kp2, *vp2)):
            assert torch.equal(a, b), i
