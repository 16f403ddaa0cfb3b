"""GPU parity on non-finite input: NaN, +-Inf and fp32 values past fp16's range.

The reference quantizes with torch's ``amin``/``amax`` (``quantize.py:209-226``),
which propagate a NaN: a group holding one gets scale 1, codes 0 and the
canonical fp16 NaN 0x7E00 as its zero.  An infinite value makes the scale
infinite (codes 0, so the group dequantizes to ``0 * inf = NaN``), and fp32
input past 65504 rounds to an infinite fp16 scale or zero.  The golden cases
``nan_*``, ``inf_*`` and ``f32_range_*`` of ``tests/golden/quantize_golden.npz``
were written by the reference's own ``quantize_groupwise``; every GPU writer of
cache rows must reproduce them bit for bit: the wide and row quantize kernels,
the append at positions, the paged append, the decode step's fused append and
the per-channel key quantizer.

Decode over such a cache (per-token or per-channel keys) must be NaN exactly where the fp32
dequantise-then-attend oracle is NaN (a NaN key poisons every head of its KV
head, a NaN value group the dims of that group), and within the north-star
tolerance everywhere else.  That includes a split whose every score is NaN,
which the combine must merge rather than skip as an empty split.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import channel as och
from oracle import inputs as oinp
from oracle import quant as oq
from tests.helpers import (assert_close_to_reference, oracle_attention_on_quant, qt_to_np,
                           same_float_bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quantize_golden.npz")


def _nonfinite_names():
    return [str(n) for n in np.load(GOLDEN)["names"]
            if str(n).startswith(("nan_", "inf_", "f32_range_"))]


def _bits16(t):
    return t.detach().cpu().numpy().view(np.uint16)


def _assert_quant_equal(qt, ref: oq.QuantNP, what: str):
    assert np.array_equal(qt.packed.cpu().numpy(), ref.packed), f"{what}: packed"
    assert np.array_equal(_bits16(qt.scale), ref.scale.view(np.uint16)), f"{what}: scale"
    assert np.array_equal(_bits16(qt.zero), ref.zero.view(np.uint16)), f"{what}: zero"


def _sprinkle(x: torch.Tensor, seed: int, frac: float = 0.004) -> torch.Tensor:
    """x with NaN, +inf and -inf at random places (and whole NaN rows)."""
    g = torch.Generator().manual_seed(seed)
    x = x.clone()
    u = torch.rand(x.shape, generator=g)
    x[u < frac] = float("nan")
    x[(u >= frac) & (u < 2 * frac)] = float("inf")
    x[(u >= 2 * frac) & (u < 3 * frac)] = -float("inf")
    flat = x.view(-1, x.shape[-1])
    flat[torch.randint(0, flat.shape[0], (3,), generator=g)] = float("nan")
    return x


def test_golden_set_holds_the_nonfinite_cases():
    names = _nonfinite_names()
    assert len(names) == 16
    z = np.load(GOLDEN)
    zeros = np.concatenate([z[f"{n}__zero"].view(np.uint16).ravel() for n in names])
    scales = np.concatenate([z[f"{n}__scale"].view(np.uint16).ravel() for n in names])
    assert (zeros == 0x7E00).any() and (zeros == 0xFC00).any() and (zeros == 0x7C00).any()
    assert (scales == 0x7C00).any()


@pytest.mark.parametrize("name", _nonfinite_names())
def test_row_kernel_matches_reference_golden(name):
    """Unaligned input takes the one-wave-per-row kernel (the fused append's
    code); the aligned wide kernel is covered by test_gpu_quant's golden test."""
    from tritonkv_amd.quantize import dequantize_groupwise, quantize_groupwise

    z = np.load(GOLDEN)
    x = torch.from_numpy(z[f"{name}__x"])
    nbits, gs = (int(v) for v in z[f"{name}__meta"])
    print(f"row kernel golden {name} nbits={nbits} gs={gs} {x.dtype}", flush=True)
    buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=DEV)
    xu = buf[1:].view(x.shape)
    xu.copy_(x.to(DEV))
    assert xu.data_ptr() % 16
    qt = quantize_groupwise(xu, nbits, gs)
    assert np.array_equal(qt.packed.cpu().numpy(), z[f"{name}__packed"])
    assert np.array_equal(_bits16(qt.scale), z[f"{name}__scale"].view(np.uint16))
    assert np.array_equal(_bits16(qt.zero), z[f"{name}__zero"].view(np.uint16))
    assert same_float_bits(dequantize_groupwise(qt).cpu().numpy(), z[f"{name}__deq"])


@pytest.mark.parametrize("rows", [300, 65600])
@pytest.mark.parametrize("nbits,gs", [(4, 32), (2, 32), (4, 128), (2, 128), (2, 16)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_bulk_quantize_nonfinite_matches_oracle(rows, nbits, gs, dtype):
    """Both wide-kernel launches (a few rows; several rows per wave)."""
    from tritonkv_amd.quantize import quantize_groupwise

    print(f"bulk nonfinite rows={rows} nbits={nbits} gs={gs} {dtype}", flush=True)
    g = torch.Generator().manual_seed(rows + nbits + gs)
    x = torch.randn(1, 2, rows // 2, 128, generator=g)
    if dtype == torch.float32:
        x[0, 0, :50] *= 4.0e4  # ranges and minima past fp16's
    x = _sprinkle(x, seed=rows + gs).to(dtype)
    qt = quantize_groupwise(x.to(DEV), nbits, gs)
    _assert_quant_equal(qt, oq.quantize_groupwise(x.numpy(), nbits, gs), "bulk")


@pytest.mark.parametrize("nbits,gs", [(4, 32), (2, 128)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_append_nonfinite_rows_matches_oracle(nbits, gs, dtype):
    from tritonkv_amd.quantize import append_kv, empty_cache

    B, HKV, S, N, D = 3, 2, 24, 3, 128
    print(f"append nonfinite nbits={nbits} gs={gs} {dtype}", flush=True)
    g = torch.Generator().manual_seed(nbits * gs)
    x = _sprinkle(torch.randn(B, HKV, N, D, generator=g) * 3, seed=11, frac=0.02).to(dtype)
    cache = empty_cache(B, HKV, S, D, nbits, gs, DEV)
    cache.packed.zero_(), cache.scale.zero_(), cache.zero.zero_()
    pos = torch.tensor([0, 7, 20], dtype=torch.int32)
    append_kv(cache, x.to(DEV), pos.to(DEV))
    ref = oq.quantize_groupwise(x.numpy(), nbits, gs)
    for b in range(B):
        p = int(pos[b])
        got = oq.QuantNP(cache.packed[b, :, p:p + N].cpu().numpy(),
                         cache.scale[b, :, p:p + N].cpu().numpy(),
                         cache.zero[b, :, p:p + N].cpu().numpy(), nbits, gs, D)
        assert np.array_equal(got.packed, ref.packed[b])
        assert np.array_equal(got.scale.view(np.uint16), ref.scale[b].view(np.uint16))
        assert np.array_equal(got.zero.view(np.uint16), ref.zero[b].view(np.uint16))


@pytest.mark.parametrize("nbits,gs", [(4, 32), (2, 32)])
def test_paged_append_nonfinite_rows_matches_oracle(nbits, gs):
    from tritonkv_amd.paged import empty_paged_pool, gather_pages, paged_append

    B, HKV, D, page, max_pages = 2, 2, 128, 32, 3
    print(f"paged append nonfinite nbits={nbits} gs={gs}", flush=True)
    g = torch.Generator().manual_seed(5 + nbits)
    N = max_pages * page
    x = _sprinkle(torch.randn(B, HKV, N, D, generator=g), seed=17, frac=0.01).half()
    pool = empty_paged_pool(B * max_pages + 2, HKV, page, D, nbits, gs, DEV)
    table = torch.randperm(B * max_pages + 2, generator=g)[:B * max_pages] \
        .reshape(B, max_pages).to(torch.int32).to(DEV)
    paged_append(pool, x.to(DEV), table, torch.zeros(B, dtype=torch.int32, device=DEV))
    got = gather_pages(pool, table)
    _assert_quant_equal(got, oq.quantize_groupwise(x.numpy(), nbits, gs), "paged")


@pytest.mark.parametrize("nbits", [2, 4])
def test_channel_keys_nonfinite_match_oracle(nbits):
    from tritonkv_amd.channel import quantize_keys_per_channel

    print(f"channel keys nonfinite nbits={nbits}", flush=True)
    g = torch.Generator().manual_seed(nbits)
    k = _sprinkle(torch.randn(2, 2, 96, 128, generator=g), seed=23, frac=0.003).half()
    ck = quantize_keys_per_channel(k.to(DEV), nbits)
    ref = och.quantize_keys_per_channel(k.numpy(), nbits)
    assert np.array_equal(ck.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_bits16(ck.scale), ref.scale.view(np.uint16))
    assert np.array_equal(_bits16(ck.zero), ref.zero.view(np.uint16))


def _assert_nan_parity(got, ref, what: str, expect_nan=None):
    """NaN exactly where the oracle is NaN; the rest finite and within tolerance."""
    g = got.detach().float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(g), nan_ref), \
        f"{what}: NaN at {np.argwhere(np.isnan(g) != nan_ref)[:8].tolist()} differs from the oracle"
    if expect_nan is not None:
        assert np.array_equal(nan_ref, expect_nan), f"{what}: the case does not poison what it meant to"
    fin = ~nan_ref
    assert np.isfinite(g[fin]).all(), f"{what}: inf where the oracle is finite"
    if fin.any():
        assert_close_to_reference(g[fin], ref[fin], what)


def _poisoned_caches(B, HQ, HKV, S, D, kbits, vbits, gs, seed):
    """Seeded caches with non-finite input in chosen units, and the NaN mask the
    oracle must show.  Unit (b, kv):
      (0, 0): one key with a NaN                  -> every head of the unit NaN
      (0, 1): one value group NaN                 -> that group's dims NaN
      (1, 0): one key with +inf (infinite scale)  -> every head NaN
      (1, 1): keys [S/4, S/2) all NaN (a whole split at 4 splits)  -> every head NaN
      (2, *): finite
    """
    from tritonkv_amd.quantize import quantize_groupwise

    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=seed)
    vd = (gs + 3) % D          # a dim of value group 1 (group 0 at gs = D)
    g0 = vd // gs * gs
    k[0, 0, S // 3, 17] = float("nan")
    v[0, 1, S // 5, vd] = float("nan")
    k[1, 0, S - 2, 5] = float("inf")
    k[1, 1, S // 4:S // 2, 64] = float("nan")
    G = HQ // HKV
    expect = np.zeros((B, HQ, D), dtype=bool)
    expect[0, 0:G] = True
    expect[0, G:2 * G, g0:g0 + gs] = True
    expect[1, :2 * G] = True
    kq = quantize_groupwise(k.to(DEV), kbits, gs)
    vq = quantize_groupwise(v.to(DEV), vbits, gs)
    return q.to(DEV), kq, vq, expect


@pytest.mark.parametrize("kbits,vbits,gs", [(4, 4, 32), (2, 2, 32), (4, 2, 32), (2, 2, 128)])
@pytest.mark.parametrize("num_splits", [1, 4, None])
@pytest.mark.parametrize("fused_combine", [False, True])
def test_decode_is_nan_where_the_oracle_is(kbits, vbits, gs, num_splits, fused_combine):
    from tritonkv_amd.kernels import fused_decode_attention

    B, HQ, HKV, S, D = 3, 8, 2, 1024, 128
    print(f"decode NaN parity K{kbits}/V{vbits} gs={gs} splits={num_splits} "
          f"fused_combine={fused_combine}", flush=True)
    q, kq, vq, expect = _poisoned_caches(B, HQ, HKV, S, D, kbits, vbits, gs, seed=kbits + gs)
    out = fused_decode_attention(q, kq, vq, num_splits=num_splits, allow_mixed_bits=True,
                                 fused_combine=fused_combine)
    torch.cuda.synchronize()
    ref = oracle_attention_on_quant(q, kq, vq)
    _assert_nan_parity(out, ref, "decode", expect)


@pytest.mark.parametrize("kbits,vbits", [(4, 4), (2, 2), (4, 2)])
def test_decode_nan_parity_long_rows(kbits, vbits):
    """16384 tokens per workgroup: the paired-tile loop (GQA 4) with rows past
    the hi/lo length, and the 12-wave kernels where the format has them."""
    from tritonkv_amd.kernels import fused_decode_attention

    B, HQ, HKV, S, D, gs = 3, 8, 2, 16384, 128, 32
    print(f"decode NaN parity long rows K{kbits}/V{vbits}", flush=True)
    q, kq, vq, expect = _poisoned_caches(B, HQ, HKV, S, D, kbits, vbits, gs, seed=7)
    out = fused_decode_attention(q, kq, vq, num_splits=1, allow_mixed_bits=True)
    torch.cuda.synchronize()
    ref = oracle_attention_on_quant(q, kq, vq)
    _assert_nan_parity(out, ref, "long rows", expect)


@pytest.mark.parametrize("kbits,vbits", [(2, 2), (4, 4)])
@pytest.mark.parametrize("equal", [True, False])
def test_channel_decode_is_nan_where_the_oracle_is(kbits, vbits, equal):
    """Per-channel keys: a NaN key poisons its channel's 32-token block (zero
    NaN), an infinite one makes the block's scale infinite (0 * inf = NaN), so
    every head of the unit is NaN; a NaN value group its dims.  Rows of 8704
    tokens at GQA 4 run the 12-wave head-column kernel (unsplit plan) or split
    rows and the window combine (ragged plan)."""
    from tritonkv_amd.channel import channel_decode_attention, quantize_keys_per_channel
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, S, D, gs, W = 3, 8, 2, 8704, 128, 32, 16
    G = HQ // HKV
    print(f"channel decode NaN parity K{kbits}/V{vbits} equal_lengths={equal}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=kbits + 31)
    vd = gs + 3
    k[0, 0, S // 3, 17] = float("nan")
    v[0, 1, S // 5, vd] = float("nan")
    k[1, 0, S - 2, 5] = float("inf")
    k[1, 1, S // 4:S // 2, 64] = float("nan")
    expect = np.zeros((B, HQ, D), dtype=bool)
    expect[0, 0:G] = True
    expect[0, G:2 * G, gs:2 * gs] = True
    expect[1, :2 * G] = True
    g = torch.Generator().manual_seed(kbits)
    kres = torch.randn(B, HKV, 32, D, generator=g).half()
    vres = torch.randn(B, HKV, 32, D, generator=g).half()
    ck = quantize_keys_per_channel(k.to(DEV), kbits)
    vq = quantize_groupwise(v.to(DEV), vbits, gs)
    ql = torch.full((B,), S, dtype=torch.int32)
    rl = torch.full((B,), W, dtype=torch.int32)
    out = channel_decode_attention(q.to(DEV), ck, vq, kres.to(DEV), vres.to(DEV), q_lens=ql.to(DEV),
                                   res_lens=rl.to(DEV), equal_lengths=equal)
    torch.cuda.synchronize()
    ckn = och.ChannelKeysNP(ck.packed.cpu().numpy(), ck.scale.cpu().numpy(), ck.zero.cpu().numpy(),
                            kbits, 32, D)
    kh, vh, lens = och.history(ckn, qt_to_np(vq), kres.numpy(), vres.numpy(), ql.tolist(),
                               rl.tolist())
    ref = oatt.reference_grouped(q.float().numpy(), lambda s_, e_: kh[:, :, s_:e_],
                                 lambda s_, e_: vh[:, :, s_:e_], kh.shape[2], HKV, seq_lens=lens)
    _assert_nan_parity(out, ref, "channel decode", expect)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_fused_append_of_a_nonfinite_token(dtype):
    """The decode step's own append quantizes a new token holding NaN / +inf:
    the cache row it writes equals the oracle's, and the output is NaN where
    attention over the oracle's cache is."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, S, D, nbits, gs = 3, 8, 2, 200, 128, 4, 32
    print(f"fused append nonfinite token {dtype}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=3)
    kq = quantize_groupwise(k.to(DEV), nbits, gs)
    vq = quantize_groupwise(v.to(DEV), nbits, gs)
    g = torch.Generator().manual_seed(8)
    k_new = torch.randn(B, HKV, D, generator=g)
    v_new = torch.randn(B, HKV, D, generator=g)
    k_new[0, 1, 40] = float("nan")      # row 0, kv 1: every head NaN
    v_new[1, 0, 100] = float("inf")     # row 1, kv 0: group 3 of the value NaN
    if dtype == torch.float32:
        k_new[2, 0, :32] = -7.0e4       # zero past fp16's range (-inf), finite scale
        k_new[2, 0, 3] = -6.99e4
    k_new, v_new = k_new.to(dtype), v_new.to(dtype)
    lens = torch.tensor([120, 77, 200], dtype=torch.int32)
    out = fused_decode_attention(q.to(DEV), kq, vq, seq_lens=lens.to(DEV),
                                 k_new=k_new.to(DEV), v_new=v_new.to(DEV))
    torch.cuda.synchronize()
    for b in range(B):
        t = int(lens[b]) - 1
        for cache, x in ((kq, k_new), (vq, v_new)):
            ref = oq.quantize_groupwise(x[b].numpy(), nbits, gs)
            assert np.array_equal(cache.packed[b, :, t].cpu().numpy(), ref.packed)
            assert np.array_equal(_bits16(cache.scale[b, :, t]), ref.scale.view(np.uint16))
            assert np.array_equal(_bits16(cache.zero[b, :, t]), ref.zero.view(np.uint16))
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
    if dtype == torch.float32:
        # A zero point of -inf makes the dequantised key -inf in every dim of
        # the group, and q . k is then +-inf or NaN depending on the signs of
        # q's dims; the kernel's folded score (zero * sum(q)) is +-inf or NaN
        # depending on the sign of their sum.  The two agree only on the other
        # rows; unit (2, 0) is compared for its cache row alone (above).
        ref, outn = ref[:2], out[:2].cpu().numpy()
    else:
        outn = out.cpu().numpy()
    G = HQ // HKV
    expect = np.zeros(ref.shape, dtype=bool)
    expect[0, G:2 * G] = True
    expect[1, 0:G, 96:128] = True
    _assert_nan_parity(outn, ref, "fused append", expect)
