"""GPU tests of the longest-piece-first dispatch order of ragged batches.

``work_order`` only changes which workgroup runs which (unit, split): every
piece still runs once and writes its own partial row.  So the decode with the
order must be *bit-identical* to the decode without it, under every path that
reads the order (plain, counters merge, fused append, paged, 12-wave, query
heads in several 16-head blocks).  The order buffer itself is checked against
a brute-force sort of the pieces: length under ``seq_lens`` descending, ties
in the natural ``s * B + b`` order, the HKV units of a piece consecutive,
each slot carrying its row's length.
"""

from __future__ import annotations

import pytest
import torch

from tests.helpers import assert_close_to_reference, make_case, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lengths(B, S, split_size, seed):
    """Ragged lengths in [1, S] with rows ending exactly on a split boundary,
    rows of the full history and one-token rows among them."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, S + 1, (B,), generator=g)
    lens[0] = S
    if B > 1:
        lens[1] = 1
    if B > 2:
        lens[2] = split_size
    if B > 3:
        lens[3] = min(S, 2 * split_size)
    return lens.to(torch.int32)


def _expected_order(lens, B, HKV, num_splits, split_size, S):
    """(s * B * HKV + unit, row length) per slot, by a sort of the pieces."""
    pieces = []
    for s in range(num_splits):
        for b in range(B):
            L = min(int(lens[b]), S)
            pieces.append((-max(0, min(L - s * split_size, split_size)), s * B + b, s, b, L))
    pieces.sort()
    out = []
    for _, _, s, b, L in pieces:
        out += [(s * B * HKV + b * HKV + hk, L) for hk in range(HKV)]
    return torch.tensor(out, dtype=torch.int32)


def _both(fn, **kw):
    ws_on, ws_off = {}, {}
    on = fn(dispatch_order=True, _workspace=ws_on, **kw)
    off = fn(dispatch_order=False, _workspace=ws_off, **kw)
    torch.cuda.synchronize()
    return on, off, ws_on


@pytest.mark.parametrize("B,HQ,HKV,S,kbits,vbits,gs,ns", [
    (12, 16, 4, 4096, 4, 4, 32, 4),
    (12, 16, 4, 4096, 2, 2, 32, 7),
    (9, 64, 8, 2048, 4, 2, 32, 3),    # the 70B-style format, G = 8
    (5, 32, 1, 3072, 4, 4, 128, 5),   # G = 32: two blocks of 16 query heads
    (16, 8, 2, 1024, 2, 2, 128, None),
    (10, 16, 4, 2048, 4, 2, 32, 1),   # unsplit: whole rows in order, out written directly
])
def test_ordered_dispatch_is_bit_identical(B, HQ, HKV, S, kbits, vbits, gs, ns):
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import plan_splits
    from tritonkv_amd.quantize import quantize_groupwise

    print(f"ordered dispatch B={B} HQ={HQ} HKV={HKV} S={S} K{kbits}V{vbits} gs{gs} ns={ns}",
          flush=True)
    q, k, v, kq, _ = make_case(B, HQ, HKV, 128, S, kbits, gs, seed=B + S)
    vq = quantize_groupwise(v, vbits, gs)
    _, n_s, split = plan_splits(S, 64, ns, B, HKV, HQ // HKV, ragged=True)
    assert (n_s > 1) == (ns != 1)
    lens = _lengths(B, S, split, seed=S + 3)
    for fused_combine in (False, True):
        on, off, ws = _both(fused_decode_attention, q=q, kq=kq, vq=vq, num_splits=ns,
                            seq_lens=lens.to(DEV), allow_mixed_bits=True,
                            fused_combine=fused_combine)
        assert torch.equal(on, off), f"fused_combine={fused_combine}"
        order = ws["work_order"][:2 * B * HKV * n_s].cpu().view(-1, 2)
        assert torch.equal(order, _expected_order(lens, B, HKV, n_s, split, S))
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
    assert_close_to_reference(on, ref, f"ordered K{kbits}V{vbits} gs{gs}")


def test_ordered_dispatch_with_fused_append_writes_the_same_cache():
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, S, ns = 8, 32, 8, 2048, 4
    print(f"ordered dispatch + fused append B={B} S={S} ns={ns}", flush=True)
    q, k, v, kq, _ = make_case(B, HQ, HKV, 128, S, 4, 32, seed=11)
    vq = quantize_groupwise(v, 2, 32)
    lens = _lengths(B, S, S // ns, seed=5)
    g = torch.Generator(device=DEV).manual_seed(9)
    kn = torch.randn(B, HKV, 128, device=DEV, generator=g).half()
    vn = torch.randn(B, HKV, 128, device=DEV, generator=g).half()
    res = []
    for order in (True, False):
        kc = type(kq)(kq.packed.clone(), kq.scale.clone(), kq.zero.clone(), kq.nbits,
                      kq.group_size, kq.head_dim)
        vc = type(vq)(vq.packed.clone(), vq.scale.clone(), vq.zero.clone(), vq.nbits,
                      vq.group_size, vq.head_dim)
        out = fused_decode_attention(q, kc, vc, num_splits=ns, seq_lens=lens.to(DEV),
                                     allow_mixed_bits=True, k_new=kn, v_new=vn,
                                     dispatch_order=order, _workspace={})
        torch.cuda.synchronize()
        res.append((out, kc, vc))
    (o1, k1, v1), (o2, k2, v2) = res
    assert torch.equal(o1, o2)
    for a, b in ((k1, k2), (v1, v2)):
        assert torch.equal(a.packed, b.packed)
        assert torch.equal(a.scale, b.scale) and torch.equal(a.zero, b.zero)


def test_ordered_dispatch_paged_and_twelve_waves():
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import choose_waves
    from tritonkv_amd.paged import empty_paged_pool, paged_decode_attention

    # 12-wave workgroups: gs128 with equal bits, at least 8192 tokens per split.
    B, HQ, HKV, S, ns = 4, 8, 2, 32768, 2
    assert choose_waves(B, HKV, HQ // HKV, S // ns, ns, k_nbits=2, v_nbits=2,
                        group_size=128) == 12
    print(f"ordered dispatch 12 waves B={B} S={S}", flush=True)
    q, k, v, kq, vq = make_case(B, HQ, HKV, 128, S, 2, 128, seed=21)
    lens = torch.tensor([S, 9000, 20000, 100], dtype=torch.int32)
    on, off, _ = _both(fused_decode_attention, q=q, kq=kq, vq=vq, num_splits=ns,
                       seq_lens=lens.to(DEV))
    assert torch.equal(on, off)

    # Paged pools: pages of 64 tokens scattered through the pool.
    B, HQ, HKV, S, page, ns = 6, 16, 4, 2048, 64, 4
    print(f"ordered dispatch paged B={B} S={S} page={page}", flush=True)
    q, k, v, kq, vq = make_case(B, HQ, HKV, 128, S, 4, 32, seed=31)
    mp = S // page
    num_pages = B * mp + 5
    table = torch.randperm(num_pages, generator=torch.Generator().manual_seed(3))[:B * mp] \
        .reshape(B, mp).to(torch.int32).to(DEV)
    pools = []
    for qt in (kq, vq):
        pool = empty_paged_pool(num_pages, HKV, page, 128, qt.nbits, qt.group_size, DEV)
        for src, dst in ((qt.packed, pool.packed), (qt.scale, pool.scale), (qt.zero, pool.zero)):
            dst.view(torch.uint8).fill_(0xFF)
            dst[table.long()] = src.reshape(B, HKV, mp, page, src.shape[-1]).permute(0, 2, 1, 3, 4)
        pools.append(pool)
    lens = _lengths(B, S, S // ns, seed=8).to(DEV)
    on, off, _ = _both(paged_decode_attention, q=q, k_pool=pools[0], v_pool=pools[1],
                       block_table=table, seq_lens=lens, num_splits=ns)
    assert torch.equal(on, off)
    contiguous = fused_decode_attention(q, kq, vq, num_splits=ns, seq_lens=lens)
    assert torch.equal(on, contiguous)


@pytest.mark.parametrize("ns", [1, 3])
def test_ordered_dispatch_with_empty_and_overlong_rows(ns):
    """Rows of length 0 and lengths past the cache's capacity reach the split
    kernel as the same L either way (the order's slots carry min(len, S)), so
    whatever those rows produce, both orders produce it bit for bit."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import plan_splits

    B, HQ, HKV, S = 20, 16, 4, 2048
    print(f"ordered dispatch empty/overlong rows B={B} S={S} ns={ns}", flush=True)
    q, k, v, kq, vq = make_case(B, HQ, HKV, 128, S, 4, 32, seed=41)
    _, n_s, split = plan_splits(S, 64, ns, B, HKV, HQ // HKV, ragged=True)
    lens = _lengths(B, S, split, seed=12)
    lens[5] = 0
    lens[6] = S + 1000
    lens[7] = 0
    on, off, ws = _both(fused_decode_attention, q=q, kq=kq, vq=vq, num_splits=ns,
                        seq_lens=lens.to(DEV))
    torch.testing.assert_close(on, off, rtol=0, atol=0, equal_nan=True)
    order = ws["work_order"][:2 * B * HKV * n_s].cpu().view(-1, 2)
    assert torch.equal(order, _expected_order(lens, B, HKV, n_s, split, S))
    keep = [i for i in range(B) if i not in (5, 7)]
    kd = torch.tensor(keep, device=DEV)
    sub = [type(t)(t.packed[kd], t.scale[kd], t.zero[kd], 4, 32, 128) for t in (kq, vq)]
    ref = oracle_attention_on_quant(q[kd], sub[0], sub[1],
                                    seq_lens=lens[keep].clamp(max=S).numpy())
    assert_close_to_reference(on[kd], ref, f"ordered rows with empty neighbours ns={ns}")


@pytest.mark.parametrize("length", [16384, 15000])
def test_equal_lengths_take_the_unragged_plan(monkeypatch, length):
    """``equal_lengths=True`` with ``seq_lens``: the split plan of a batch
    without lengths (here one workgroup per unit, where the ragged rule cuts
    histories of >= 16384 tokens into two pieces), still stopping each row at
    its length.  At the full length the output is bit-identical to the call
    without ``seq_lens``; both plans match the oracle."""
    from tritonkv_amd.kernels import fused_decode_attn as fda

    monkeypatch.setattr(fda, "compute_units", lambda device=None: 8)  # B * HKV units fill the GPU
    B, HQ, HKV, D, S = 2, 8, 4, 128, 16384
    print(f"equal lengths {length} of S={S}", flush=True)
    q, _, _, kq, vq = make_case(B, HQ, HKV, D, S, 4, 32, 77)
    lens = torch.full((B,), length, dtype=torch.int32, device=DEV)
    ws_eq, ws_rag = {}, {}
    out_eq = fda.fused_decode_attention(q, kq, vq, seq_lens=lens, equal_lengths=True,
                                        _workspace=ws_eq)
    out_rag = fda.fused_decode_attention(q, kq, vq, seq_lens=lens, _workspace=ws_rag)
    torch.cuda.synchronize()
    assert "acc" not in ws_eq and "work_order" not in ws_eq  # one split, no order
    assert ws_rag["key"][2] == 2                            # the ragged rule's two pieces
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.cpu().numpy())
    assert_close_to_reference(out_eq, ref, "equal lengths")
    assert_close_to_reference(out_rag, ref, "ragged plan")
    if length == S:
        out_none = fda.fused_decode_attention(q, kq, vq)
        torch.cuda.synchronize()
        assert torch.equal(out_eq, out_none)
