"""GPU parity of the paired-tile score path.

With at most 8 query heads per GQA group and at least 8192 tokens per
workgroup, the split kernel scores both 16-token tiles of a chunk in one set
of MFMAs (a block-diagonal q operand, column = 8 * tile + head).  These cases
use ``num_splits=1`` on histories of >= 8192 tokens so that path runs, and
check it against the oracle, with NaN garbage past each row's length (a row
of one tile shares an MFMA row with the other tile's token), ragged lengths,
every group size, both bit widths, mixed K/V widths, head_dim 64, a paged
pool and the fused append.
"""

from __future__ import annotations

import pytest
import torch

from oracle import inputs as oinp
from tests.helpers import assert_close_to_reference, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
S_PT = 8192 + 40  # > the paired-tile threshold, and not a multiple of 32


def _nan_past(qt, lens):
    from tritonkv_amd.quantize import QuantizedTensor

    c = QuantizedTensor(qt.packed.clone(), qt.scale.clone(), qt.zero.clone(), qt.nbits,
                        qt.group_size, qt.head_dim)
    for b, L in enumerate(lens):
        for t in (c.packed, c.scale, c.zero):
            t[b, :, L:].view(torch.uint8).fill_(0xFF)
    return c


def _zero_past(qt, lens):
    from tritonkv_amd.quantize import QuantizedTensor

    c = QuantizedTensor(qt.packed.clone(), qt.scale.clone(), qt.zero.clone(), qt.nbits,
                        qt.group_size, qt.head_dim)
    for b, L in enumerate(lens):
        c.packed[b, :, L:] = 0
        c.scale[b, :, L:] = 0
        c.zero[b, :, L:] = 0
    return c


CASES = [
    # (kbits, vbits, gs, D, HQ, HKV): G = HQ / HKV <= 8
    (4, 4, 32, 128, 8, 2),
    (2, 2, 32, 128, 8, 2),
    (4, 2, 32, 128, 16, 2),
    (2, 4, 16, 128, 12, 2),
    (4, 4, 128, 128, 6, 1),
    (2, 2, 64, 128, 2, 2),
    (4, 4, 64, 64, 8, 8),
    (2, 2, 16, 64, 4, 1),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "K{}V{}-gs{}-D{}-G{}".format(
    c[0], c[1], c[2], c[3], c[4] // c[5]))
def test_paired_tiles_match_the_oracle(case):
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    kbits, vbits, gs, D, HQ, HKV = case
    lens = [S_PT, S_PT - 37]
    print(f"case {case} lens={lens}", flush=True)
    q, k, v = oinp.make_random_kv(2, HQ, HKV, S_PT, D, seed=kbits + 3 * vbits + gs + D)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, kbits, gs), quantize_groupwise(v, vbits, gs)
    kn, vn = _nan_past(kq, lens), _nan_past(vq, lens)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=DEV)
    got = fused_decode_attention(q, kn, vn, num_splits=1, seq_lens=lens_d, allow_mixed_bits=True)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    ref = oracle_attention_on_quant(q, _zero_past(kq, lens), _zero_past(vq, lens),
                                    seq_lens=lens)
    assert_close_to_reference(got, ref, f"paired tiles {case}")


def test_paired_tiles_paged_and_fused_append_are_bit_identical():
    """Paged pool vs contiguous cache, and fused append vs append-then-decode,
    on the paired-tile path (the same kernel arithmetic on both sides)."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.paged import empty_paged_pool, paged_decode_attention
    from tritonkv_amd.quantize import QuantizedTensor, append_kv, quantize_groupwise

    B, HQ, HKV, D, page = 2, 8, 2, 128, 256
    S = 8192 + 256
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=77)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, 4, 32), quantize_groupwise(v, 4, 32)
    lens = torch.tensor([S, S - 100], dtype=torch.int32, device=DEV)
    mp = S // page
    gen = torch.Generator().manual_seed(9)
    table = torch.randperm(B * mp, generator=gen).reshape(B, mp).to(torch.int32).to(DEV)
    pools = []
    for qt in (kq, vq):
        p = empty_paged_pool(B * mp, HKV, page, D, 4, 32, DEV)
        for src, dst in ((qt.packed, p.packed), (qt.scale, p.scale), (qt.zero, p.zero)):
            dst[table.long()] = src.reshape(B, HKV, mp, page, -1).permute(0, 2, 1, 3, 4)
        pools.append(p)
    want = fused_decode_attention(q, kq, vq, num_splits=1, seq_lens=lens)
    got = paged_decode_attention(q, pools[0], pools[1], table, lens, num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # fused append on the same path
    k_new, v_new = k[:, :, -1].contiguous(), v[:, :, -1].contiguous()

    def clone(c):
        return QuantizedTensor(c.packed.clone(), c.scale.clone(), c.zero.clone(), c.nbits,
                               c.group_size, c.head_dim)

    ka, va = clone(kq), clone(vq)
    append_kv(ka, k_new[:, :, None], lens - 1)
    append_kv(va, v_new[:, :, None], lens - 1)
    want = fused_decode_attention(q, ka, va, num_splits=1, seq_lens=lens)
    kb, vb = clone(kq), clone(vq)
    got = fused_decode_attention(q, kb, vb, num_splits=1, seq_lens=lens, k_new=k_new, v_new=v_new)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    for a, b in ((ka, kb), (va, vb)):
        assert torch.equal(a.packed, b.packed) and torch.equal(a.scale, b.scale)
