"""GPU parity of the quad-tile kernel (``csrc/quant_quad.h``): 2-bit K/V codes,
one scale/zero group per row (group size 128), GQA groups of at most 4 query
heads, contiguous caches, 8- and 12-wave workgroups.

Every case calls the C ABI with an explicit wave count on splits of at least
8192 tokens -- 8 or 12 waves take the quad-tile kernel, 4 the paired-tile
kernel -- and checks the output against
the oracle's fp32 dequantise-then-attend at the north-star tolerance, and the
two kernels against each other.  The lengths cover rows of a single token,
rows that end inside a step's first chunk (an odd number of chunks: the TAIL
step's second chunk past the end), rows of at most 256 tokens (hi/lo
probabilities) and longer ones (P * s remainders), ragged batches, splits
with both combine modes, and fp32 queries.
"""

from __future__ import annotations

import pytest
import torch

from oracle import inputs as oinp
from tests.helpers import assert_close_to_reference, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _call(q, kq, vq, lens, waves, num_splits=1, fused_combine=False):
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits

    B, HQ, D = q.shape
    _, HKV, S, _ = kq.packed.shape
    _, ns, size = plan_splits(S, 64, num_splits, B, HKV, HQ // HKV)
    out = torch.full((B, HQ, D), float("nan"), device=DEV)
    acc = torch.empty(B, HQ, ns, D, device=DEV)
    mx = torch.empty(B, HQ, ns, device=DEV)
    sm = torch.empty(B, HQ, ns, device=DEV)
    cnt = torch.zeros(B * HKV, dtype=torch.int32, device=DEV)
    a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                        v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                        seq_lens=lens.data_ptr(), acc=acc.data_ptr(), maxs=mx.data_ptr(),
                        sums=sm.data_ptr(), out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D,
                        k_nbits=2, v_nbits=2, group_size=128, sm_scale=D ** -0.5,
                        split_size=size, num_splits=ns,
                        counters=cnt.data_ptr() if fused_combine else None, waves=waves,
                        q_is_fp32=int(q.dtype == torch.float32))
    _lib.check(_lib.load().tkv_fused_decode_attention(a, _lib.stream_handle(q.device)), "fused")
    torch.cuda.synchronize()
    assert int(cnt.abs().sum()) == 0  # the tickets reset
    return out


def _case(B, HQ, HKV, S, lens, seed, q_fp32=False):
    from tritonkv_amd.quantize import quantize_groupwise

    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, 128, seed=seed)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, 2, 128), quantize_groupwise(v, 2, 128)
    if q_fp32:
        q = q.float()
    return q, kq, vq, torch.tensor(lens, dtype=torch.int32)


# Both kernels run where a workgroup streams at least 8192 tokens (paired tiles'
# threshold), so the short rows sit in a cache of 8200 tokens: a single token,
# rows that end in a step's first chunk, rows of at most 256 tokens (hi/lo
# probabilities), full-length rows and rows one token short of a chunk edge.
CASES = [
    # (B, HQ, HKV, lens): G = 4, 3, 1, 4
    (2, 8, 2, [8200, 33]),
    (3, 6, 2, [1, 250, 4133]),
    (2, 2, 2, [700, 8200]),
    (1, 4, 1, [257]),
    (4, 8, 2, [8200, 8199, 8168, 8137]),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}-G{}-{}".format(c[0], c[1] // c[2], c[3][0]))
def test_quad_tiles_match_the_oracle_and_the_paired_kernel(case):
    B, HQ, HKV, lens = case
    S = 8200
    print(f"quad case B={B} HQ={HQ} HKV={HKV} lens={lens}", flush=True)
    q, kq, vq, lens = _case(B, HQ, HKV, S, lens, seed=100 + B + HQ)
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
    paired = _call(q, kq, vq, lens.to(DEV), waves=4)
    assert_close_to_reference(paired, ref, f"paired B={B} HQ={HQ}")
    for waves in (8, 12):
        got = _call(q, kq, vq, lens.to(DEV), waves=waves)
        assert_close_to_reference(got, ref, f"quad waves={waves} B={B} HQ={HQ}")
        assert (got - paired).abs().max().item() < 2e-3


@pytest.mark.parametrize("fused_combine", [False, True])
@pytest.mark.parametrize("waves", [8, 12])
def test_quad_tile_splits_and_combine_modes(waves, fused_combine):
    """Three splits of ragged rows (the short row's later splits are empty),
    merged by the combine kernel or by the last workgroup, three calls in a row."""
    B, HQ, HKV, S = 3, 8, 2, 25000
    print(f"quad splits waves={waves} fused={fused_combine}", flush=True)
    q, kq, vq, lens = _case(B, HQ, HKV, S, [S, 9001, 40], seed=7)
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
    for rep in range(3):
        got = _call(q, kq, vq, lens.to(DEV), waves=waves, num_splits=3, fused_combine=fused_combine)
        assert_close_to_reference(got, ref, f"quad splits waves={waves} fused={fused_combine} rep={rep}")


def test_quad_tiles_take_fp32_queries():
    B, HQ, HKV, S = 2, 8, 2, 8200
    q, kq, vq, lens = _case(B, HQ, HKV, S, [S, 3001], seed=11, q_fp32=True)
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
    for waves in (8, 12):
        got = _call(q, kq, vq, lens.to(DEV), waves=waves)
        assert_close_to_reference(got, ref, f"quad fp32 q waves={waves}")


def test_quad_tiles_leave_wider_groups_and_other_formats_to_paired_tiles():
    """G = 6 (and 4-bit codes at G = 4) never take the quad kernel: the same
    call at 8 and 12 waves then runs the paired-tile kernels, still within the
    tolerance of the oracle."""
    from tritonkv_amd import _lib
    from tritonkv_amd.quantize import quantize_groupwise

    B, S, D = 2, 8200, 128
    for HQ, HKV, nb in ((12, 2, 2), (8, 2, 4)):
        q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=5)
        q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
        kq, vq = quantize_groupwise(k, nb, 128), quantize_groupwise(v, nb, 128)
        lens = torch.tensor([S, 700], dtype=torch.int32)
        ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
        dl = lens.to(DEV)
        for waves in (8, 12):
            got = torch.full((B, HQ, D), float("nan"), device=DEV)
            a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                                k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                                v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                                seq_lens=dl.data_ptr(), out=got.data_ptr(), B=B, HQ=HQ, HKV=HKV,
                                S=S, D=D, k_nbits=nb, v_nbits=nb, group_size=128,
                                sm_scale=D ** -0.5, split_size=S, num_splits=1, waves=waves)
            _lib.check(_lib.load().tkv_fused_decode_attention(a, _lib.stream_handle(q.device)),
                       "fused")
            torch.cuda.synchronize()
            assert_close_to_reference(got, ref, f"HQ={HQ} nbits={nb} waves={waves}")
