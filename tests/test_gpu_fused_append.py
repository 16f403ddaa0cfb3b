"""GPU parity of the decode step with the append fused into the split kernel.

``fused_decode_attention(..., seq_lens=L, k_new=k, v_new=v)`` must leave the
caches and the output *bit-identical* to ``append_kv`` at ``L - 1`` followed by
the plain decode: the fused path quantizes with the append kernel's own code
and feeds the row to the same arithmetic.  Caches are prefilled with 0xFF
(fp16 NaN) past each row's history so a row that is read but not patched, or
a store to the wrong place, breaks equality; the whole caches are compared,
so a store anywhere else shows too.
"""

from __future__ import annotations

import pytest
import torch

from oracle import inputs as oinp
from tests.helpers import assert_close_to_reference, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _caches(k, v, kbits, vbits, gs, hist):
    """Contiguous caches holding k/v's first hist[b] tokens per row, NaN after."""
    from tritonkv_amd.quantize import QuantizedTensor, append_kv, empty_cache

    B, HKV, S, D = k.shape
    out = []
    for x, nb in ((k, kbits), (v, vbits)):
        c = empty_cache(B, HKV, S, D, nb, gs, DEV)
        for t in (c.packed, c.scale, c.zero):
            t.view(torch.uint8).fill_(0xFF)
        for b in range(B):
            if hist[b] > 0:
                view = QuantizedTensor(c.packed[b:b + 1], c.scale[b:b + 1], c.zero[b:b + 1],
                                       nb, gs, D)
                append_kv(view, x[b:b + 1, :, :hist[b]].contiguous())
        out.append(c)
    return out


def _clone(c):
    from tritonkv_amd.quantize import QuantizedTensor

    return QuantizedTensor(c.packed.clone(), c.scale.clone(), c.zero.clone(), c.nbits,
                           c.group_size, c.head_dim)


def _same(a, b):
    return all(torch.equal(x.view(torch.uint8), y.view(torch.uint8))
               for x, y in ((a.packed, b.packed), (a.scale, b.scale), (a.zero, b.zero)))


CASES = [
    # (kbits, vbits, gs, D, HQ, HKV)
    (4, 4, 32, 128, 16, 4),
    (2, 2, 32, 128, 16, 4),
    (4, 2, 32, 128, 32, 4),
    (4, 4, 128, 128, 12, 2),
    (2, 2, 16, 128, 12, 2),
    (4, 4, 64, 64, 8, 8),
    (2, 4, 32, 64, 64, 2),   # G = 32: two blocks of query heads share the new token
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "K{}V{}-gs{}-D{}-G{}".format(
    c[0], c[1], c[2], c[3], c[4] // c[5]))
def test_fused_append_is_bit_identical_to_append_then_decode(case):
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import append_kv

    kbits, vbits, gs, D, HQ, HKV = case
    S = 1100
    lens = torch.tensor([1, 32, 33, 641, S, 1024], dtype=torch.int32)
    B = len(lens)
    print(f"case {case} lens={lens.tolist()}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=kbits * 10 + gs + D)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    g = torch.Generator().manual_seed(7)
    k_new = torch.randn(B, HKV, D, generator=g).half().to(DEV)
    v_new = torch.randn(B, HKV, D, generator=g).half().to(DEV)
    kc0, vc0 = _caches(k, v, kbits, vbits, gs, (lens - 1).tolist())
    lens_d = lens.to(DEV)
    for ns in (None, 1, 5):
        ka, va = _clone(kc0), _clone(vc0)
        append_kv(ka, k_new[:, :, None], lens_d - 1)
        append_kv(va, v_new[:, :, None], lens_d - 1)
        want = fused_decode_attention(q, ka, va, num_splits=ns, seq_lens=lens_d,
                                      allow_mixed_bits=True)
        kb, vb = _clone(kc0), _clone(vc0)
        got = fused_decode_attention(q, kb, vb, num_splits=ns, seq_lens=lens_d,
                                     allow_mixed_bits=True, k_new=k_new, v_new=v_new)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all(), ns
        assert torch.equal(got, want), (ns, (got - want).abs().max().item())
        assert _same(ka, kb) and _same(va, vb), ns
    # and the result is the oracle's attention over the appended caches
    clean = []
    for c in (ka, va):
        c = _clone(c)
        for b in range(B):
            L = int(lens[b])
            c.packed[b, :, L:] = 0
            c.scale[b, :, L:] = 0
            c.zero[b, :, L:] = 0
        clean.append(c)
    ref = oracle_attention_on_quant(q, clean[0], clean[1], seq_lens=lens.numpy())
    assert_close_to_reference(got, ref, f"fused append {case}")


@pytest.mark.parametrize("kbits,gs", [(2, 32), (2, 128), (4, 128)])
def test_fused_append_in_twelve_wave_workgroups(kbits, gs):
    """The fused append in the 12-wave kernels (one split of 9000 tokens at a
    GQA group of 4): bit-identical to append-then-decode, and the oracle's
    attention over the appended caches."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import choose_waves
    from tritonkv_amd.quantize import append_kv

    B, HQ, HKV, D, S = 3, 8, 2, 128, 9000
    assert choose_waves(B, HKV, HQ // HKV, S, 1, D=D, k_nbits=kbits, v_nbits=kbits,
                        group_size=gs) == 12
    lens = torch.tensor([9000, 8193, 100], dtype=torch.int32)
    print(f"fused append, 12 waves: K{kbits}V{kbits} gs{gs}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=41 + gs)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    g = torch.Generator().manual_seed(9)
    k_new = torch.randn(B, HKV, D, generator=g).half().to(DEV)
    v_new = torch.randn(B, HKV, D, generator=g).half().to(DEV)
    kc0, vc0 = _caches(k, v, kbits, kbits, gs, (lens - 1).tolist())
    lens_d = lens.to(DEV)
    ka, va = _clone(kc0), _clone(vc0)
    append_kv(ka, k_new[:, :, None], lens_d - 1)
    append_kv(va, v_new[:, :, None], lens_d - 1)
    want = fused_decode_attention(q, ka, va, num_splits=1, seq_lens=lens_d)
    kb, vb = _clone(kc0), _clone(vc0)
    got = fused_decode_attention(q, kb, vb, num_splits=1, seq_lens=lens_d, k_new=k_new,
                                 v_new=v_new)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got - want).abs().max().item()
    assert _same(ka, kb) and _same(va, vb)
    clean = []
    for c in (ka, va):
        c = _clone(c)
        for b in range(B):
            L = int(lens[b])
            c.packed[b, :, L:] = 0
            c.scale[b, :, L:] = 0
            c.zero[b, :, L:] = 0
        clean.append(c)
    ref = oracle_attention_on_quant(q, clean[0], clean[1], seq_lens=lens.numpy())
    assert_close_to_reference(got, ref, f"fused append, 12 waves, K{kbits} gs{gs}")


def test_fused_append_fp32_tokens_and_no_seq_lens():
    """fp32 new tokens; without seq_lens the token goes to the last slot S - 1."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import append_kv

    B, HQ, HKV, S, D = 2, 8, 2, 256, 128
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=3)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    k_new = torch.randn(B, HKV, 1, D, device=DEV)
    v_new = torch.randn(B, HKV, 1, D, device=DEV)
    kc0, vc0 = _caches(k, v, 4, 4, 32, [S - 1] * B)
    ka, va = _clone(kc0), _clone(vc0)
    pos = torch.full((B,), S - 1, dtype=torch.int32, device=DEV)
    append_kv(ka, k_new, pos)
    append_kv(va, v_new, pos)
    want = fused_decode_attention(q, ka, va)
    kb, vb = _clone(kc0), _clone(vc0)
    got = fused_decode_attention(q, kb, vb, k_new=k_new, v_new=v_new)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert _same(ka, kb) and _same(va, vb)


@pytest.mark.parametrize("page_size", [32, 256])
def test_fused_append_paged(page_size):
    from tritonkv_amd.paged import empty_paged_pool, paged_append, paged_decode_attention

    B, HQ, HKV, D, gs = 4, 32, 4, 128, 32
    lens = torch.tensor([1, 600, page_size, 2 * page_size + 1], dtype=torch.int32)
    mp = (int(lens.max()) + page_size - 1) // page_size + 1
    num_pages = B * mp + 2
    print(f"case page={page_size} lens={lens.tolist()}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, mp * page_size, D, seed=19)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    gen = torch.Generator().manual_seed(page_size)
    table = torch.randperm(num_pages, generator=gen)[:B * mp].reshape(B, mp).to(torch.int32).to(DEV)
    pools = []
    for x, nb in ((k, 4), (v, 2)):
        p = empty_paged_pool(num_pages, HKV, page_size, D, nb, gs, DEV)
        for t in (p.packed, p.scale, p.zero):
            t.view(torch.uint8).fill_(0xFF)
        z = torch.zeros(1, dtype=torch.int32, device=DEV)
        for b in range(B):
            if lens[b] > 1:
                paged_append(p, x[b:b + 1, :, :int(lens[b]) - 1].contiguous(), table[b:b + 1], z)
        pools.append(p)
    k_new = k[:, :, -1:].contiguous()
    v_new = v[:, :, -1:].contiguous()
    lens_d = lens.to(DEV)
    for ns in (None, 1, 3):
        ka, va = _clone(pools[0]), _clone(pools[1])
        paged_append(ka, k_new, table, lens_d - 1)
        paged_append(va, v_new, table, lens_d - 1)
        want = paged_decode_attention(q, ka, va, table, lens_d, num_splits=ns,
                                      allow_mixed_bits=True)
        kb, vb = _clone(pools[0]), _clone(pools[1])
        got = paged_decode_attention(q, kb, vb, table, lens_d, num_splits=ns,
                                     allow_mixed_bits=True, k_new=k_new, v_new=v_new)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all(), ns
        assert torch.equal(got, want), (ns, (got - want).abs().max().item())
        assert _same(ka, kb) and _same(va, vb), ns


def test_fused_append_step_replays_in_a_graph():
    """The serving loop: one captured launch per step (append + decode), with
    the lengths advanced between replays, against eager fused steps."""
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import empty_cache

    B, HQ, HKV, S, D = 2, 16, 2, 512, 128
    kc = empty_cache(B, HKV, S, D, 4, 32, DEV)
    vc = empty_cache(B, HKV, S, D, 4, 32, DEV)
    for t in (kc.packed, kc.scale, kc.zero, vc.packed, vc.scale, vc.zero):
        t.zero_()
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(B, HQ, D, generator=gen).half().to(DEV)
    xs = [torch.randn(B, HKV, D, generator=gen).half().to(DEV) for _ in range(10)]
    lens = torch.tensor([5, 90], dtype=torch.int32, device=DEV)
    xk = torch.empty(B, HKV, D, dtype=torch.float16, device=DEV)
    xv = torch.empty_like(xk)
    out = torch.empty(B, HQ, D, device=DEV)
    ws = {}

    def step():
        fused_decode_attention(q, kc, vc, num_splits=3, out=out, _workspace=ws, seq_lens=lens,
                               k_new=xk, v_new=xv)

    xk.copy_(xs[0])
    xv.copy_(xs[1])
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    ke, ve = _clone(kc), _clone(vc)
    for i in range(4):
        lens.add_(1)
        xk.copy_(xs[2 + 2 * i])
        xv.copy_(xs[3 + 2 * i])
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = fused_decode_attention(q, ke, ve, num_splits=3, seq_lens=lens, k_new=xk, v_new=xv)
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
        assert _same(kc, ke) and _same(vc, ve), i
