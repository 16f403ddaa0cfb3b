"""GPU parity of per-channel (KIVI-style) keys with an fp16 residual window.

* The key quantizer (``tkv_quantize_keys_channel``) is bit-exact with the
  oracle (``oracle/channel.py``), itself pinned through the golden-pinned
  per-token quantizer on transposed blocks.
* The decode step (per-channel key path of the split kernel, the fp16 control
  over the window as one more split, the combine) is within the north-star
  tolerance of the oracle's fp32 attention over the dequantized history
  followed by the window, with ragged history and window lengths (including
  empty ones) and NaN garbage past every length.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import channel as och
from oracle import quant as oq
from tests.helpers import assert_close_to_reference, qt_to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits16(t):
    return t.detach().cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_channel_key_quantizer_matches_oracle_bitwise(D, nbits, dtype):
    from tritonkv_amd.channel import quantize_keys_per_channel

    print(f"channel quantize D={D} nbits={nbits} {dtype}", flush=True)
    g = torch.Generator().manual_seed(D + nbits)
    k = (torch.randn(2, 3, 96, D, generator=g) * 2).to(dtype)
    k[0, 1, 32:64, 5] = 0.75       # a constant group
    k[1, 0, :, 9] *= 40            # an outlier channel
    # non-finite input: NaN propagates through the block's min / max (the
    # canonical NaN zero, scale 1, codes 0), +-Inf as the arithmetic gives
    k[0, 2, 3, 9] = float("nan")
    k[1, 1, 70, 11] = float("inf")
    k[0, 0, 33, 2] = float("-inf")
    if dtype == torch.float16:
        k.view(torch.int16)[1, 2, 90, 4] = -512            # 0xFE00: a NaN with the sign bit
    else:
        k.view(torch.int32)[1, 2, 90, 4] = -4194304        # 0xFFC00000
        k[1, 2, 40, 7], k[1, 2, 41, 7] = 1.0e6, -7.0e4     # beyond the fp16 range
    ck = quantize_keys_per_channel(k.to(DEV), nbits)
    ref = och.quantize_keys_per_channel(k.numpy(), nbits)
    assert np.array_equal(ck.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_bits16(ck.scale), ref.scale.view(np.uint16))
    assert np.array_equal(_bits16(ck.zero), ref.zero.view(np.uint16))


def test_channel_key_append_positions():
    """Blocks land at per-row positions; unaligned or out-of-range blocks are not written."""
    from tritonkv_amd.channel import append_keys_per_channel, empty_channel_keys

    B, H, D, S = 4, 2, 128, 128
    g = torch.Generator().manual_seed(4)
    k = torch.randn(B, H, 64, D, generator=g).half()
    ck = empty_channel_keys(B, H, S, D, 4, DEV)
    for t in (ck.packed, ck.scale, ck.zero):
        t.view(torch.uint8).fill_(0xAB)
    pos = torch.tensor([0, 32, 96, 16], dtype=torch.int32, device=DEV)
    append_keys_per_channel(ck, k.to(DEV), pos)
    ref = och.quantize_keys_per_channel(k.numpy(), 4)
    packed, scale = ck.packed.cpu().numpy(), _bits16(ck.scale)
    assert np.array_equal(packed[0, :, 0:64], ref.packed[0])
    assert np.array_equal(scale[0, :, 0:2], ref.scale[0].view(np.uint16))
    assert np.array_equal(packed[1, :, 32:96], ref.packed[1])
    assert np.array_equal(packed[2, :, 96:128], ref.packed[2, :, :32])   # second block past S
    assert (packed[2, :, :96] == 0xAB).all()
    assert (packed[3] == 0xAB).all()                                     # position 16: unaligned


def _window_case(B, HQ, HKV, D, S, kbits, vbits, gs, q_lens, r_lens, seed, R=32):
    from tritonkv_amd.channel import quantize_keys_per_channel
    from tritonkv_amd.quantize import quantize_groupwise

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, HQ, D, generator=g).half()
    k = torch.randn(B, HKV, S, D, generator=g)
    k[:, :, :, 3] *= 12                     # fixed outlier channels
    k[:, :, :, 70 % D] *= 8
    k = k.half()
    v = torch.randn(B, HKV, S, D, generator=g).half()
    kres = torch.randn(B, HKV, R, D, generator=g).half()
    vres = torch.randn(B, HKV, R, D, generator=g).half()
    ck = quantize_keys_per_channel(k.to(DEV), kbits)
    vq = quantize_groupwise(v.to(DEV), vbits, gs)
    ql = torch.tensor(q_lens, dtype=torch.int32)
    rl = torch.tensor(r_lens, dtype=torch.int32)
    return q, ck, vq, kres, vres, ql, rl


def _oracle(q, ck, vq, kres, vres, ql, rl):
    ckn = och.ChannelKeysNP(ck.packed.cpu().numpy(), ck.scale.cpu().numpy(), ck.zero.cpu().numpy(),
                            ck.nbits, 32, ck.head_dim)
    kh, vh, lens = och.history(ckn, qt_to_np(vq), kres.numpy(), vres.numpy(), ql.tolist(),
                               rl.tolist())
    HKV = kh.shape[1]
    return oatt.reference_grouped(q.float().numpy(), lambda s, e: kh[:, :, s:e],
                                  lambda s, e: vh[:, :, s:e], kh.shape[2], HKV, seq_lens=lens)


CASES = [
    # (kbits, vbits, gs, D, HQ, HKV)
    (2, 2, 32, 128, 16, 4),
    (4, 4, 32, 128, 12, 2),
    (2, 4, 16, 128, 8, 2),
    (4, 2, 32, 64, 32, 4),
    (2, 2, 16, 64, 4, 1),
    (2, 4, 32, 128, 24, 2),   # GQA 12: 16 head columns, hi and lo MFMAs per step
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "K{}V{}-gs{}-D{}-G{}".format(
    c[0], c[1], c[2], c[3], c[4] // c[5]))
@pytest.mark.parametrize("ns", [None, 1, 3])
@pytest.mark.parametrize("lens", ["blocks", "ragged"])
def test_channel_decode_matches_oracle(case, ns, lens):
    """History lengths on block boundaries (what the cache manager makes) and
    anywhere inside a block (the tail chunk's masking)."""
    from tritonkv_amd.channel import channel_decode_attention

    kbits, vbits, gs, D, HQ, HKV = case
    S = 640
    if lens == "blocks":
        q_lens, r_lens = [640, 0, 96, 320, 32], [31, 7, 0, 32, 1]
    else:
        q_lens, r_lens = [77, 639, 33, 5, 1], [0, 3, 31, 1, 32]
    B = len(q_lens)
    print(f"channel decode {case} ns={ns}", flush=True)
    q, ck, vq, kres, vres, ql, rl = _window_case(B, HQ, HKV, D, S, kbits, vbits, gs, q_lens,
                                                 r_lens, seed=kbits + 10 * vbits + gs + D)
    got = channel_decode_attention(q.to(DEV), ck, vq, kres.to(DEV), vres.to(DEV),
                                   q_lens=ql.to(DEV), res_lens=rl.to(DEV), num_splits=ns)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    ref = _oracle(q, ck, vq, kres, vres, ql, rl)
    assert_close_to_reference(got, ref, f"channel decode {case} ns={ns}")


def test_channel_decode_twelve_waves():
    """Per-channel 2-bit keys, 2-bit V gs32, GQA group of 4, one split of 8704
    tokens: the path's default is a 12-wave workgroup."""
    from tritonkv_amd.channel import channel_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import choose_waves

    B, HQ, HKV, D, S = 2, 8, 2, 128, 8704
    assert choose_waves(B, HKV, 4, S, 1, D=D, k_nbits=2, v_nbits=2, group_size=32) == 12
    q, ck, vq, kres, vres, ql, rl = _window_case(B, HQ, HKV, D, S, 2, 2, 32, [8704, 8200],
                                                 [5, 32], seed=77)
    got = channel_decode_attention(q.to(DEV), ck, vq, kres.to(DEV), vres.to(DEV),
                                   q_lens=ql.to(DEV), res_lens=rl.to(DEV), num_splits=1)
    torch.cuda.synchronize()
    ref = _oracle(q, ck, vq, kres, vres, ql, rl)
    assert_close_to_reference(got, ref, "channel decode, 12 waves")


@pytest.mark.parametrize("R", [16, 48])
@pytest.mark.parametrize("q_dtype", [torch.float16, torch.float32])
def test_channel_decode_window_sizes(R, q_dtype):
    """Windows of up to 32 tokens are attended inside the combine, longer ones
    by the fp16 kernel as one more split; fp32 q is rounded to fp16 in both."""
    from tritonkv_amd.channel import channel_decode_attention

    q_lens, r_lens = [64, 0, 33, 128], [R, 5, 0, R - 1]
    print(f"channel decode window R={R} q={q_dtype}", flush=True)
    q, ck, vq, kres, vres, ql, rl = _window_case(4, 12, 2, 128, 128, 4, 2, 32, q_lens, r_lens,
                                                 seed=R, R=R)
    q = q.to(q_dtype)
    got = channel_decode_attention(q.to(DEV), ck, vq, kres.to(DEV), vres.to(DEV),
                                   q_lens=ql.to(DEV), res_lens=rl.to(DEV))
    torch.cuda.synchronize()
    ref = _oracle(q, ck, vq, kres, vres, ql, rl)
    assert_close_to_reference(got, ref, f"channel decode window R={R}")
    # no lengths: every window full
    got = channel_decode_attention(q.to(DEV), ck, vq, kres.to(DEV), vres.to(DEV), q_lens=ql.to(DEV))
    torch.cuda.synchronize()
    ref = _oracle(q, ck, vq, kres, vres, ql, torch.full((4,), R, dtype=torch.int32))
    assert_close_to_reference(got, ref, f"channel decode full window R={R}")


def test_channel_decode_ignores_garbage_past_the_lengths():
    """NaN bit patterns past every row's history and window change nothing."""
    from tritonkv_amd.channel import ChannelQuantizedKeys, channel_decode_attention
    from tritonkv_amd.quantize import QuantizedTensor

    B, HQ, HKV, D, S = 3, 8, 2, 128, 256
    q_lens, r_lens = [96, 256, 0], [5, 0, 20]
    q, ck, vq, kres, vres, ql, rl = _window_case(B, HQ, HKV, D, S, 4, 2, 32, q_lens, r_lens, 9)
    args = dict(q_lens=ql.to(DEV), res_lens=rl.to(DEV), num_splits=2)
    clean = channel_decode_attention(q.to(DEV), ck, vq, kres.to(DEV), vres.to(DEV), **args)
    ck2 = ChannelQuantizedKeys(ck.packed.clone(), ck.scale.clone(), ck.zero.clone(), ck.nbits, D)
    vq2 = QuantizedTensor(vq.packed.clone(), vq.scale.clone(), vq.zero.clone(), vq.nbits,
                          vq.group_size, D)
    kr2, vr2 = kres.clone().to(DEV), vres.clone().to(DEV)
    for b in range(B):
        a, r = q_lens[b], r_lens[b]
        for t in (ck2.packed, vq2.packed, vq2.scale, vq2.zero):
            t[b, :, a:].view(torch.uint8).fill_(0xFF)
        for t in (ck2.scale, ck2.zero):
            t[b, :, a // 32:].view(torch.uint8).fill_(0xFF)
        for t in (kr2, vr2):
            t[b, :, r:].view(torch.uint8).fill_(0xFF)
    dirty = channel_decode_attention(q.to(DEV), ck2, vq2, kr2, vr2, **args)
    torch.cuda.synchronize()
    assert torch.equal(dirty, clean)


def test_channel_kv_cache_prefill_and_decode_steps():
    """The cache manager: prefill, then single-token steps across window flushes."""
    from tritonkv_amd.channel import ChannelKVCache

    B, HQ, HKV, D = 2, 8, 2, 128
    g = torch.Generator().manual_seed(11)
    n0, steps = 70, 40
    k = torch.randn(B, HKV, n0 + steps, D, generator=g).half()
    v = torch.randn(B, HKV, n0 + steps, D, generator=g).half()
    q = torch.randn(B, HQ, D, generator=g).half()
    cache = ChannelKVCache(B, HKV, 256, D, k_nbits=2, v_nbits=4, group_size=32, device=DEV)
    cache.extend(k[:, :, :n0].to(DEV), v[:, :, :n0].to(DEV))
    assert (cache.quantized, cache.window) == (64, 6)
    checked = 0
    for s in range(steps):
        cache.extend(k[:, :, n0 + s:n0 + s + 1].to(DEV), v[:, :, n0 + s:n0 + s + 1].to(DEV))
        n = n0 + s + 1
        if s not in (0, 25, 26, 39):   # before, at and after the flush at 96 tokens
            continue
        got = cache.attend(q.to(DEV))
        torch.cuda.synchronize()
        nq = (n // 32) * 32
        ckn = och.quantize_keys_per_channel(k[:, :, :nq].numpy(), 2) if nq else None
        vqn = oq.quantize_groupwise(v[:, :, :nq].numpy(), 4, 32)
        kd = och.dequantize_keys_per_channel(ckn) if nq else np.zeros((B, HKV, 0, D), np.float32)
        vd = oq.dequantize_groupwise(vqn) if nq else np.zeros((B, HKV, 0, D), np.float32)
        kh = np.concatenate([kd, k[:, :, nq:n].float().numpy()], axis=2)
        vh = np.concatenate([vd, v[:, :, nq:n].float().numpy()], axis=2)
        ref = oatt.reference_decode_attention(q.float().numpy(), kh, vh)
        assert_close_to_reference(got, ref, f"cache step {s} (n={n})")
        checked += 1
    assert checked == 4 and len(cache) == n0 + steps


def test_channel_kv_cache_step_replays_in_a_graph():
    """``step`` (append to the window, attend, flush a full window) captured
    once and replayed across two window flushes: every replay equals an eager
    twin's step bit for bit, and matches the oracle on the step's partition of
    the history (quantized blocks, then the window including the new token)."""
    from tritonkv_amd.channel import ChannelKVCache

    B, HQ, HKV, D = 2, 8, 2, 128
    g = torch.Generator().manual_seed(12)
    n0, steps = 70, 60
    k = torch.randn(B, HKV, n0 + steps, D, generator=g).half()
    v = torch.randn(B, HKV, n0 + steps, D, generator=g).half()
    q = torch.randn(B, HQ, D, generator=g).half().to(DEV)
    caches = [ChannelKVCache(B, HKV, 256, D, k_nbits=4, v_nbits=2, group_size=32, device=DEV)
              for _ in range(2)]
    for c in caches:
        c.extend(k[:, :, :n0].to(DEV), v[:, :, :n0].to(DEV))
    eager, graphed = caches
    kb = torch.empty(B, HKV, 1, D, dtype=torch.float16, device=DEV)
    vb = torch.empty_like(kb)
    out = torch.empty(B, HQ, D, device=DEV)
    for c in caches:  # the first step eagerly on both (allocates the workspace)
        c.step(k[:, :, n0:n0 + 1].to(DEV), v[:, :, n0:n0 + 1].to(DEV), q, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed.step(kb, vb, q, out=out)
    checked = 0
    for s in range(1, steps):
        t = n0 + s
        kb.copy_(k[:, :, t:t + 1].to(DEV))
        vb.copy_(v[:, :, t:t + 1].to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = eager.step(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), q)
        torch.cuda.synchronize()
        assert torch.equal(got, want), s
        n = t + 1
        if s in (1, 25, 26, 58):   # around the flushes at 96 and 128 tokens
            nq = ((n - 1) // 32) * 32
            ckn = och.quantize_keys_per_channel(k[:, :, :nq].numpy(), 4)
            vqn = oq.quantize_groupwise(v[:, :, :nq].numpy(), 2, 32)
            kh = np.concatenate([och.dequantize_keys_per_channel(ckn),
                                 k[:, :, nq:n].float().numpy()], axis=2)
            vh = np.concatenate([oq.dequantize_groupwise(vqn), v[:, :, nq:n].float().numpy()],
                                axis=2)
            ref = oatt.reference_decode_attention(q.float().cpu().numpy(), kh, vh)
            assert_close_to_reference(got, ref, f"graph step {s} (n={n})")
            checked += 1
    assert checked == 4
    for a, b in ((graphed.keys, eager.keys), (graphed.values, eager.values)):
        assert torch.equal(a.packed, b.packed) and torch.equal(a.scale, b.scale)
    # the flushes quantized exactly what the host path quantizes
    nq = int(graphed._qlens[0])
    assert nq == ((n0 + steps) // 32) * 32
    ref = ChannelKVCache(B, HKV, 256, D, k_nbits=4, v_nbits=2, group_size=32, device=DEV)
    ref.extend(k[:, :, :nq].to(DEV), v[:, :, :nq].to(DEV))
    assert torch.equal(graphed.keys.packed[:, :, :nq], ref.keys.packed[:, :, :nq])
    assert torch.equal(graphed.keys.scale[:, :, :nq // 32], ref.keys.scale[:, :, :nq // 32])
    assert torch.equal(graphed.keys.zero[:, :, :nq // 32], ref.keys.zero[:, :, :nq // 32])
    assert torch.equal(graphed.values.packed[:, :, :nq], ref.values.packed[:, :, :nq])
    assert torch.equal(graphed.values.zero[:, :, :nq], ref.values.zero[:, :, :nq])


def test_channel_kv_cache_replay_past_capacity_marks_the_row():
    """Replayed steps are not counted on the host, so only the device guards the
    capacity: the flush that would overrun the history writes nothing, moves no
    length and marks the row (window length 33); further appends are refused
    and the decode attends to the tokens held.  ``overflowed`` reports it."""
    from tritonkv_amd.channel import ChannelKVCache

    B, HQ, HKV, D = 2, 4, 1, 128
    g = torch.Generator().manual_seed(31)
    cache = ChannelKVCache(B, HKV, 64, D, k_nbits=4, v_nbits=4, group_size=32, device=DEV)
    k = torch.randn(B, HKV, 33, D, generator=g).half().to(DEV)
    cache.extend(k, k)  # one block + one window token
    q = torch.randn(B, HQ, D, generator=g).half().to(DEV)
    kb = torch.randn(B, HKV, 1, D, generator=g).half().to(DEV)
    out = torch.empty(B, HQ, D, device=DEV)
    cache.step(kb, kb, q, out=out)  # eager: window 2
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cache.step(kb, kb, q, out=out)
    for _ in range(30):  # window 32 -> flushed into [32, 64): the history is full
        graph.replay()
    torch.cuda.synchronize()
    assert not cache.overflowed()
    assert cache._qlens.tolist() == [64, 64] and cache._rlens.tolist() == [0, 0]
    history = [t.clone() for t in (cache.keys.packed, cache.values.packed)]
    for _ in range(32):  # window fills again; its flush cannot fit
        graph.replay()
    torch.cuda.synchronize()
    assert cache.overflowed()
    assert cache._qlens.tolist() == [64, 64] and cache._rlens.tolist() == [33, 33]
    assert torch.equal(cache.keys.packed, history[0]) and torch.equal(cache.values.packed, history[1])
    graph.replay()  # a marked row stays as it is
    torch.cuda.synchronize()
    assert cache._rlens.tolist() == [33, 33]
    assert torch.isfinite(out).all()
    cache.reset()
    assert not cache.overflowed()
