"""GPU parity at the full sizes of the two large benchmark configurations.

* Llama-3-8B attention (B=32, HQ=32, HKV=8, D=128, ctx 32768) on its own
  inputs -- N(0,1) K/V with 4 x8 outlier channels per KV head -- for all four
  (nbits, group_size) pairs the benchmark times, and for its per-channel key
  steps (2- and 4-bit, 16-token fp16 window).
* The 70B-style ragged batch (B=64, HQ=64, HKV=8, D=128, lengths U[1024,
  131072], K 4-bit / V 2-bit, group 32) with the decode step's one-token
  append fused into the split kernel.

The inputs are ``tritonkv_amd.synthetic``'s, at the benchmark's seeds, so these
tests check the very workloads ``bench.py`` times.  The checks are:

* Llama: every (batch row, kv head) unit of the batch, for both split plans,
  against the C oracle (``oracle/tkv_oracle.c``: dequantise to fp32, attend
  with binary64 sums) on the GPU cache's own codes, within 2e-3 max-abs /
  1e-3 mean-abs;
* size-independent properties over the whole batch: the split count does not
  change the answer (Llama); the fused append is bitwise equal to
  append-then-decode, in the output and in every cache byte (70B-style);
* sampled (batch row, kv head) units -- for the ragged batch the longest and
  the shortest row among them -- against the oracle on the same fp16 values
  copied to the host: codes, scales and zero points bitwise equal to the oracle
  quantizer's, and attention within 2e-3 max-abs / 1e-3 mean-abs (plus the
  reference's cosine and rel-L2 bars) of the fp32 dequantise-then-attend
  reference.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import channel as och
from oracle import quant as oq
from tests.helpers import MAX_ABS_TOL, assert_close_to_reference

pytestmark = pytest.mark.gpu
DEV = "cuda"

LLAMA = dict(B=32, HQ=32, HKV=8, S=32768, D=128)
LLAMA_SEED = 10  # bench.py's first Llama-shape cache copy
LLAMA_UNITS = ((0, 0), (17, 5), (31, 7), (9, 2), (4, 3), (22, 1), (13, 6), (28, 4))
X70B = dict(B=64, HQ=64, HKV=8, D=128, lo=1024, hi=131072, gs=32)
X70B_SEED = 2024  # bench.py's 70B-style batch
X70B_CAPACITY = 131072 + 64


def _say(msg):
    print(msg, flush=True)


def _whole_batch_vs_c_oracle(q, kq, vq, outs, what):
    """Every (b, kv head) unit of each output in ``outs`` against the C oracle on
    the cache's codes (one unit per task; ctypes releases the GIL)."""
    import concurrent.futures as cf
    import os

    from oracle import c_oracle

    B, HQ, D = q.shape
    HKV = kq.packed.shape[1]
    G = HQ // HKV
    host = [t.cpu().numpy() for t in (kq.packed, kq.scale, kq.zero, vq.packed, vq.scale, vq.zero)]
    qf = q.float().cpu().numpy()
    units = [(b, h) for b in range(B) for h in range(HKV)]

    def run(u):
        b, h = u
        sub = [a[b:b + 1, h:h + 1] for a in host]
        return c_oracle.quantized_decode_attention(
            qf[b:b + 1, h * G:(h + 1) * G], (sub[0], sub[1], sub[2], kq.nbits, kq.group_size),
            (sub[3], sub[4], sub[5], vq.nbits, vq.group_size), D ** -0.5)[0]

    with cf.ThreadPoolExecutor(max_workers=min(16, len(os.sched_getaffinity(0)))) as ex:
        refs = list(ex.map(run, units))
    for plan, out in outs:
        o = out.cpu().numpy().astype(np.float64)
        err = np.stack([np.abs(o[b, h * G:(h + 1) * G] - r) for (b, h), r in zip(units, refs)])
        worst = units[int(err.reshape(len(units), -1).max(axis=1).argmax())]
        _say(f"  whole batch {plan}: max-abs {err.max():.3e} mean-abs {err.mean():.3e} "
             f"(worst unit b={worst[0]} h={worst[1]})")
        assert err.max() <= MAX_ABS_TOL, f"{what} {plan}: max-abs {err.max()} at unit {worst}"
        assert err.mean() <= 1e-3, f"{what} {plan}: mean-abs {err.mean()}"


def _assert_unit_codes(kq_gpu, x_unit, b, h, L, what):
    """GPU cache rows [0, L) of unit (b, h) == the oracle quantizer on x_unit (L, D) fp16."""
    want = oq.quantize_groupwise(x_unit, kq_gpu.nbits, kq_gpu.group_size)
    assert np.array_equal(kq_gpu.packed[b, h, :L].cpu().numpy(), want.packed), f"{what} codes"
    for name in ("scale", "zero"):
        got = getattr(kq_gpu, name)[b, h, :L].cpu().numpy().view(np.uint16)
        assert np.array_equal(got, getattr(want, name).view(np.uint16)), f"{what} {name}"
    return want


# ---------------------------------------------------------------------------
# Llama-3-8B shape, outlier-channel inputs, all four formats
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def llama_kv():
    from tritonkv_amd import synthetic

    _say(f"llama inputs {LLAMA} seed={LLAMA_SEED}")
    q, k, v, chans = synthetic.outlier_channel_kv(LLAMA["B"], LLAMA["HQ"], LLAMA["HKV"],
                                                  LLAMA["S"], LLAMA["D"], seed=LLAMA_SEED)
    yield q, k, v, chans
    del q, k, v
    torch.cuda.empty_cache()


def test_llama_inputs_have_four_scaled_channels_per_kv_head(llama_kv):
    q, k, v, chans = llama_kv
    assert chans.shape == (LLAMA["HKV"], 4)
    # per KV head: the four chosen channels carry 8x the spread of the others
    sd = k[:4].float().std(dim=(0, 2))  # (HKV, D)
    for h in range(LLAMA["HKV"]):
        mask = torch.zeros(LLAMA["D"], dtype=torch.bool, device=DEV)
        mask[chans[h]] = True
        assert torch.allclose(sd[h][mask], torch.full_like(sd[h][mask], 8.0), rtol=0.02)
        assert torch.allclose(sd[h][~mask], torch.ones_like(sd[h][~mask]), rtol=0.02)


@pytest.mark.parametrize("nbits,gs", [(4, 32), (4, 128), (2, 32), (2, 128)])
def test_llama3_8b_outlier_channels_full_shape(llama_kv, nbits, gs):
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import quantize_kv

    q, k, v, _ = llama_kv
    B, HQ, HKV, S, D = (LLAMA[x] for x in ("B", "HQ", "HKV", "S", "D"))
    G = HQ // HKV
    _say(f"llama full shape nbits={nbits} gs={gs}: quantize + decode")
    kq, vq = quantize_kv(k, v, nbits, gs)
    got = fused_decode_attention(q, kq, vq)      # one workgroup per unit (paired tiles)
    split = fused_decode_attention(q, kq, vq, num_splits=8)  # 4096-token splits + combine
    torch.cuda.synchronize()
    assert torch.isfinite(got).all() and torch.isfinite(split).all()
    # size-independent: both split plans approximate one answer within the
    # tolerance each is held to below, over the whole batch
    assert (got - split).abs().max().item() <= 2 * MAX_ABS_TOL
    _whole_batch_vs_c_oracle(q, kq, vq, (("default", got), ("8 splits", split)),
                             f"llama nbits={nbits} gs={gs}")
    got_np, split_np = got.cpu().numpy(), split.cpu().numpy()
    for b, h in LLAMA_UNITS:
        _say(f"  unit b={b} h={h}")
        kw = _assert_unit_codes(kq, k[b, h].cpu().numpy(), b, h, S, f"K b={b} h={h}")
        vw = _assert_unit_codes(vq, v[b, h].cpu().numpy(), b, h, S, f"V b={b} h={h}")
        qn = q[b:b + 1, G * h:G * (h + 1)].float().cpu().numpy()
        kd = oq.dequantize_groupwise(oq.QuantNP(kw.packed[None, None], kw.scale[None, None],
                                                kw.zero[None, None], nbits, gs, D))
        vd = oq.dequantize_groupwise(oq.QuantNP(vw.packed[None, None], vw.scale[None, None],
                                                vw.zero[None, None], nbits, gs, D))
        ref = oatt.reference_decode_attention(qn, kd, vd)
        for out, plan in ((got_np, "default"), (split_np, "8 splits")):
            assert_close_to_reference(out[b:b + 1, G * h:G * (h + 1)], ref,
                                      f"llama nbits={nbits} gs={gs} b={b} h={h} {plan}")
    del kq, vq
    torch.cuda.empty_cache()


@pytest.mark.parametrize("nbits", [2, 4])
def test_llama3_8b_per_channel_keys_full_shape(llama_kv, nbits):
    """The per-channel key step the benchmark times (keys per 32-token block and
    channel, values per token, a 16-token fp16 window) on the same inputs, with
    the unsplit plan (``equal_lengths``: one workgroup per unit, 12 waves at
    2-bit) and the ragged plan (split rows + combine): sampled units' key and
    value codes bitwise equal to the oracle quantizers', and attention within
    the oracle tolerance of fp32 attention over the oracle's dequantised
    history and window."""
    from tritonkv_amd.channel import channel_decode_attention, quantize_keys_per_channel
    from tritonkv_amd.quantize import quantize_groupwise

    q, k, v, _ = llama_kv
    B, HQ, HKV, S, D = (LLAMA[x] for x in ("B", "HQ", "HKV", "S", "D"))
    G, W = HQ // HKV, 16
    _say(f"llama per-channel keys nbits={nbits}: quantize + decode")
    g = torch.Generator(device=DEV).manual_seed(77 + nbits)
    kr = torch.randn(B, HKV, 32, D, device=DEV, generator=g, dtype=torch.float16)
    vr = torch.randn(B, HKV, 32, D, device=DEV, generator=g, dtype=torch.float16)
    ck = quantize_keys_per_channel(k, nbits)
    vq = quantize_groupwise(v, nbits, 32)
    ql = torch.full((B,), S, dtype=torch.int32, device=DEV)
    rl = torch.full((B,), W, dtype=torch.int32, device=DEV)
    got = channel_decode_attention(q, ck, vq, kr, vr, q_lens=ql, res_lens=rl, equal_lengths=True)
    ragged = channel_decode_attention(q, ck, vq, kr, vr, q_lens=ql, res_lens=rl)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all() and torch.isfinite(ragged).all()
    assert (got - ragged).abs().max().item() <= 2 * MAX_ABS_TOL
    got_np, rag_np = got.cpu().numpy(), ragged.cpu().numpy()
    for b, h in LLAMA_UNITS:
        _say(f"  unit b={b} h={h}")
        want = och.quantize_keys_per_channel(k[b, h].cpu().numpy(), nbits)
        packed = ck.packed[b, h].cpu().numpy()
        scale, zero = ck.scale[b, h].cpu().numpy(), ck.zero[b, h].cpu().numpy()
        assert np.array_equal(packed, want.packed), f"K codes b={b} h={h}"
        assert np.array_equal(scale.view(np.uint16), want.scale.view(np.uint16)), f"K scale b={b} h={h}"
        assert np.array_equal(zero.view(np.uint16), want.zero.view(np.uint16)), f"K zero b={b} h={h}"
        vw = _assert_unit_codes(vq, v[b, h].cpu().numpy(), b, h, S, f"V b={b} h={h}")
        ckn = och.ChannelKeysNP(packed[None, None], scale[None, None], zero[None, None], nbits,
                                32, D)
        vqn = oq.QuantNP(vw.packed[None, None], vw.scale[None, None], vw.zero[None, None], nbits,
                         32, D)
        kk, vv, _ = och.history(ckn, vqn, kr[b, h].cpu().numpy()[None, None],
                                vr[b, h].cpu().numpy()[None, None], [S], [W])
        qn = q[b:b + 1, G * h:G * (h + 1)].float().cpu().numpy()
        ref = oatt.reference_decode_attention(qn, kk, vv)
        for out, plan in ((got_np, "equal lengths"), (rag_np, "ragged plan")):
            assert_close_to_reference(out[b:b + 1, G * h:G * (h + 1)], ref,
                                      f"llama per-channel nbits={nbits} b={b} h={h} {plan}")
    del ck, vq
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# 70B-style ragged batch with the fused append, full size
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def ragged_step():
    from tritonkv_amd import synthetic
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import QuantizedTensor, append_kv

    B, HQ, HKV, D, gs = (X70B[x] for x in ("B", "HQ", "HKV", "D", "gs"))
    lens = synthetic.ragged_lengths(B, X70B["lo"], X70B["hi"], seed=X70B_SEED)
    _say(f"70B-style batch: B={B} lengths {int(lens.min())}..{int(lens.max())} "
         f"sum {int(lens.sum())}, capacity {X70B_CAPACITY}")
    q, kc, vc, k_new, v_new = synthetic.ragged_batch(B, HQ, HKV, D, lens, X70B_CAPACITY, 4, 2, gs,
                                                     seed=X70B_SEED)
    torch.cuda.synchronize()

    def clone(c):
        return QuantizedTensor(c.packed.clone(), c.scale.clone(), c.zero.clone(), c.nbits,
                               c.group_size, c.head_dim)
    kc2, vc2 = clone(kc), clone(vc)
    pos = lens.to(DEV)
    lens1 = (lens + 1).to(DEV)
    _say("70B-style: fused append + decode")
    out_fused = fused_decode_attention(q, kc, vc, seq_lens=lens1, allow_mixed_bits=True,
                                       k_new=k_new, v_new=v_new)
    _say("70B-style: append_kv x2, then decode")
    append_kv(kc2, k_new, pos)
    append_kv(vc2, v_new, pos)
    out_sep = fused_decode_attention(q, kc2, vc2, seq_lens=lens1, allow_mixed_bits=True)
    torch.cuda.synchronize()
    yield dict(lens=lens, q=q, kc=kc, vc=vc, kc2=kc2, vc2=vc2, k_new=k_new, v_new=v_new,
               out_fused=out_fused, out_sep=out_sep)
    del kc, vc, kc2, vc2
    torch.cuda.empty_cache()


def test_70b_fused_append_is_bitwise_append_then_decode(ragged_step):
    r = ragged_step
    assert torch.isfinite(r["out_fused"]).all()
    assert torch.equal(r["out_fused"], r["out_sep"])
    # byte views: never-written slots may hold NaN bit patterns, which == would reject
    for name in ("packed", "scale", "zero"):
        for c1, c2, what in ((r["kc"], r["kc2"], "K"), (r["vc"], r["vc2"], "V")):
            assert torch.equal(getattr(c1, name).view(torch.uint8),
                               getattr(c2, name).view(torch.uint8)), f"{what} {name}"


def _ragged_units(lens):
    b_long, b_short = int(torch.argmax(lens)), int(torch.argmin(lens))
    others = [b for b in (5, 23, 40, 63, 11, 50) if b not in (b_long, b_short)]
    return [("longest", b_long, 7), ("shortest", b_short, 0)] + \
        [(f"row{b}", b, (3 * b) % 8) for b in others[:4]]


@pytest.mark.parametrize("which", range(6))
def test_70b_sampled_unit_matches_oracle(ragged_step, which):
    from tritonkv_amd import synthetic

    r = ragged_step
    HQ, HKV, D, gs = (X70B[x] for x in ("HQ", "HKV", "D", "gs"))
    G = HQ // HKV
    role, b, h = _ragged_units(r["lens"])[which]
    L = int(r["lens"][b])
    _say(f"70B-style unit {role}: b={b} h={h} L={L}")
    k, v = synthetic.ragged_row_kv(X70B_SEED, b, HKV, L, D)
    # history rows: bitwise the oracle quantizer's; appended row L: the oracle's on the new token
    kw = _assert_unit_codes(r["kc"], k[h].cpu().numpy(), b, h, L, f"K {role}")
    vw = _assert_unit_codes(r["vc"], v[h].cpu().numpy(), b, h, L, f"V {role}")
    del k, v
    kn = oq.quantize_groupwise(r["k_new"][b, h].cpu().numpy(), 4, gs)
    vn = oq.quantize_groupwise(r["v_new"][b, h].cpu().numpy(), 2, gs)
    for cache, want, what in ((r["kc"], kn, "K"), (r["vc"], vn, "V")):
        assert np.array_equal(cache.packed[b, h, L:L + 1].cpu().numpy(), want.packed), what
        assert np.array_equal(cache.scale[b, h, L:L + 1].cpu().numpy().view(np.uint16),
                              want.scale.view(np.uint16)), what
        assert np.array_equal(cache.zero[b, h, L:L + 1].cpu().numpy().view(np.uint16),
                              want.zero.view(np.uint16)), what

    def dq(w, n, nbits):
        return oq.dequantize_groupwise(oq.QuantNP(
            np.concatenate([w.packed, n.packed])[None, None],
            np.concatenate([w.scale, n.scale])[None, None],
            np.concatenate([w.zero, n.zero])[None, None], nbits, gs, D))

    qn = r["q"][b:b + 1, G * h:G * (h + 1)].float().cpu().numpy()
    ref = oatt.reference_decode_attention(qn, dq(kw, kn, 4), dq(vw, vn, 2))
    got = r["out_fused"][b:b + 1, G * h:G * (h + 1)].cpu().numpy()
    assert_close_to_reference(got, ref, f"70B-style {role} b={b} h={h} L+1={L + 1}")
