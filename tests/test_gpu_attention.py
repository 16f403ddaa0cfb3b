"""GPU parity of the fused decode-attention and fp16 control kernels.

Ports every kernel assertion of the reference's ``test_correctness.py:163-343``
to the HIP kernels, with the oracle's fp32 dequantise-then-attend as the
reference, and adds the north-star tolerance (2e-3 max-abs, 1e-3 mean-abs)
to every comparison.  Beyond the reference: the fp16 control kernel, mixed
K/V bit widths, per-row context lengths, q in fp32, head_dim 64, GQA groups
larger than 16 and HIP-graph replay.  The two large benchmark configurations
are checked at full size in ``test_gpu_large_configs.py``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import inputs as oinp
from oracle import quant as oq
from tests.helpers import (
    KERNEL_COSINE_MIN,
    KERNEL_REL_L2_MAX,
    KERNEL_VS_BASELINE_ERR_RATIO_MAX,
    assert_close_to_reference,
    fp16_baseline_rows,
    make_case,
    metrics,
    oracle_attention_on_quant,
    qt_to_np,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [
    # (B, HQ, HKV, D) -- Qwen2.5-1.5B attention shape, plus GQA edge cases
    (1, 12, 2, 128),
    (1, 8, 8, 64),  # no GQA sharing (MHA)
    (2, 32, 8, 64),  # Llama-3.2-1B shape, batch 2
]
SEQ_LENS = [1, 17, 128, 512, 2048, 8192, 16384]


def _fused(q, kq, vq, **kw):
    from tritonkv_amd.kernels import fused_decode_attention

    return fused_decode_attention(q, kq, vq, **kw)


def _case_and_check(B, HQ, HKV, D, S, nbits, gs, seed, **kw):
    print(f"case B={B} HQ={HQ} HKV={HKV} D={D} S={S} nbits={nbits} gs={gs} seed={seed} {kw}",
          flush=True)
    q, k, v, kq, vq = make_case(B, HQ, HKV, D, S, nbits, gs, seed)
    got = _fused(q, kq, vq, **kw)
    torch.cuda.synchronize()
    ref = oracle_attention_on_quant(q, kq, vq)
    return assert_close_to_reference(got, ref, f"S={S} nbits={nbits} gs={gs} seed={seed} {kw}")


@pytest.mark.parametrize("S", SEQ_LENS)
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_kernel_matches_dequant_reference_4bit(S, seed):
    _case_and_check(1, 12, 2, 128, S, 4, 32, seed)


@pytest.mark.parametrize("S", [512, 2048, 8192, 16384])
@pytest.mark.parametrize("seed", [0, 1])
def test_kernel_matches_dequant_reference_2bit(S, seed):
    _case_and_check(1, 12, 2, 128, S, 2, 32, seed)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("nbits", [2, 4])
def test_kernel_shapes_and_gqa(shape, nbits):
    B, HQ, HKV, D = shape
    _case_and_check(B, HQ, HKV, D, 1024, nbits, 32, 3)


@pytest.mark.parametrize("group_size", [16, 32, 64, 128])
@pytest.mark.parametrize("nbits", [2, 4])
def test_kernel_group_sizes(group_size, nbits):
    _case_and_check(1, 12, 2, 128, 2048, nbits, group_size, 4)


@pytest.mark.parametrize("S", [1, 33, 777, 1025])
@pytest.mark.parametrize("nbits", [2, 4])
def test_one_group_per_row_with_odd_lengths(S, nbits):
    # group_size == head_dim: one 2-byte scale/zero per token, so the metadata
    # block of an odd-length cache ends in the middle of a dword.
    _case_and_check(2, 8, 2, 128, S, nbits, 128, 21)
    _case_and_check(2, 8, 2, 64, S, nbits, 64, 22)


@pytest.mark.parametrize("S", [2, 3, 5, 31, 32, 33])
@pytest.mark.parametrize("D,gs", [(128, 32), (64, 64)])
@pytest.mark.parametrize("nbits", [2, 4])
def test_tiny_contexts_meet_the_north_star_tolerance(S, D, gs, nbits):
    # With a handful of tokens each probability carries a large share of the
    # output, so an fp16 P (as the reference's tl.dot takes it) would put up to
    # 2^-10 * max|v| of rounding into it -- above 2e-3 with the x8 outliers.
    # The step holding a split's last token takes P and P * s_g as hi/lo fp16
    # pairs, so these meet the fixed tolerance like long contexts do.
    _case_and_check(2, 8, 2, D, S, nbits, gs, 5)


@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("num_splits", [None, 1, 5])
def test_short_and_long_rows_in_one_batch(nbits, num_splits):
    # Rows of at most 256 tokens take hi/lo probabilities in every chunk, longer
    # ones fp16 probabilities; one launch serves both, around the boundary.
    lens = [33, 256, 257, 3000]
    q, k, v, kq, vq = make_case(4, 8, 2, 128, 3000, nbits, 32, 31)
    got = _fused(q, kq, vq, seq_lens=torch.tensor(lens, dtype=torch.int32, device=DEV),
                 num_splits=num_splits)
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens)
    assert_close_to_reference(got, ref, f"short and long rows nbits={nbits} ns={num_splits}")


@pytest.mark.parametrize("D", [64])
@pytest.mark.parametrize("group_size", [16, 32, 64])
@pytest.mark.parametrize("nbits", [2, 4])
def test_kernel_head_dim_64_group_sizes(D, group_size, nbits):
    _case_and_check(2, 8, 2, D, 777, nbits, group_size, 12)


def test_kernel_is_not_the_source_of_error():
    """Kernel error vs the fp16 truth must stay within 1.5x the fp16 dequant baseline's."""
    for S in (512, 2048, 8192, 16384):
        q, k, v, kq, vq = make_case(1, 12, 2, 128, S, 4, 32, 5)
        got = _fused(q, kq, vq)
        qn, kn, vn = q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy()
        truth = oatt.reference_decode_attention(qn, kn, vn)
        # reference.py:288-304: fp16 dequant (c*s, +z each rounded to fp16), then attention.
        kb = fp16_baseline_rows(qt_to_np(kq)).astype(np.float32)
        vb = fp16_baseline_rows(qt_to_np(vq)).astype(np.float32)
        base = oatt.reference_decode_attention(qn.astype(np.float16).astype(np.float32), kb, vb)
        e_kernel = metrics(got, truth)["rel_l2"]
        e_base = metrics(base, truth)["rel_l2"]
        assert e_kernel <= KERNEL_VS_BASELINE_ERR_RATIO_MAX * e_base, (S, e_kernel, e_base)


@pytest.mark.parametrize("num_splits", [1, 2, 5, 17, 64])
def test_split_count_does_not_change_the_answer(num_splits):
    _case_and_check(1, 12, 2, 128, 4096, 4, 32, 6, num_splits=num_splits)


@pytest.mark.parametrize("block_n", [16, 32, 64, 128])
def test_block_sizes(block_n):
    _case_and_check(1, 12, 2, 128, 3000, 4, 32, 7, block_n=block_n)


def test_output_is_finite_with_extreme_scores():
    q, k, v, kq, vq = make_case(1, 12, 2, 128, 2048, 4, 32, 8)
    q = q * 50.0
    got = _fused(q, kq, vq)
    assert torch.isfinite(got).all()
    ref = oracle_attention_on_quant(q, kq, vq)
    assert metrics(got, ref)["cosine"] >= KERNEL_COSINE_MIN


def test_single_token_cache():
    """S=1: attention output must be exactly the single dequantized V row."""
    q, k, v, kq, vq = make_case(1, 12, 2, 128, 1, 4, 32, 9)
    got = _fused(q, kq, vq).cpu().numpy()
    v_deq = oq.dequantize_groupwise(qt_to_np(vq))  # (1, HKV, 1, D)
    expect = np.repeat(v_deq[:, :, 0, :], 6, axis=1)
    assert metrics(got, expect)["rel_l2"] < 1e-3
    assert np.abs(got - expect).max() <= 2e-3


def test_per_element_worst_case_not_hidden_by_aggregate():
    q, k, v, kq, vq = make_case(1, 12, 2, 128, 8192, 4, 32, 10)
    got = _fused(q, kq, vq).cpu().numpy()
    ref = oracle_attention_on_quant(q, kq, vq)
    worst = np.abs(got - ref).max() / max(np.abs(ref).mean(), 1e-6)
    assert worst < 0.05


@pytest.mark.parametrize("S", [1, 17, 512, 2048, 8192])
@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("group_size", [16, 32, 64, 128])
def test_metadata_broadcast_and_fp16_dequant_flags_are_bitwise_identical(S, nbits, group_size):
    """meta_bcast / dequant_fp16 / fold_zp select Triton variants; here they must not change a bit."""
    q, k, v, kq, vq = make_case(1, 12, 2, 128, S, nbits, group_size, 11)
    base = _fused(q, kq, vq)
    for kw in (dict(meta_bcast=False), dict(dequant_fp16=True), dict(fold_zp=True),
               dict(num_warps=8, num_stages=3)):
        assert torch.equal(base, _fused(q, kq, vq, **kw)), kw


def test_deterministic_across_calls_and_workspace_reuse():
    q, k, v, kq, vq = make_case(1, 12, 2, 128, 5000, 4, 32, 13)
    ws = {}
    out = torch.empty(1, 12, 128, device=DEV)
    a = _fused(q, kq, vq, out=out, _workspace=ws).clone()
    acc_ptr = ws["acc"].data_ptr()
    b = _fused(q, kq, vq, out=out, _workspace=ws)
    assert torch.equal(a, b) and ws["acc"].data_ptr() == acc_ptr and b.data_ptr() == out.data_ptr()


def test_q_in_fp32_is_rounded_like_fp16():
    q, k, v, kq, vq = make_case(1, 12, 2, 128, 2048, 4, 32, 14)
    assert torch.equal(_fused(q.float(), kq, vq), _fused(q, kq, vq))


def test_gqa_group_larger_than_16():
    # 32 query heads per kv head: two 16-head blocks per workgroup column.
    _case_and_check(1, 64, 2, 128, 1500, 4, 32, 15)


@pytest.mark.parametrize("kbits,vbits", [(4, 2), (2, 4)])
def test_mixed_bit_widths(kbits, vbits):
    from tritonkv_amd.quantize import quantize_groupwise

    q, k, v = oinp.make_random_kv(2, 16, 2, 3000, 128, seed=16)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, kbits, 32), quantize_groupwise(v, vbits, 32)
    with pytest.raises(ValueError):
        _fused(q, kq, vq)
    got = _fused(q, kq, vq, allow_mixed_bits=True)
    assert_close_to_reference(got, oracle_attention_on_quant(q, kq, vq), f"K{kbits}/V{vbits}")


def test_ragged_sequence_lengths():
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, S, D = 4, 16, 2, 5000, 128
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=17)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, 4, 32), quantize_groupwise(v, 2, 32)
    lens = torch.tensor([5000, 1, 777, 4097], dtype=torch.int32)
    for ns in (None, 1, 13):
        got = _fused(q, kq, vq, seq_lens=lens.to(DEV), allow_mixed_bits=True, num_splits=ns)
        ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
        assert_close_to_reference(got, ref, f"ragged ns={ns}")


def _launch(q, kq, vq, out, num_splits, waves, seq_lens):
    """One fused call through the C ABI with an explicit wave count (one split:
    no partials)."""
    from tritonkv_amd import _lib

    assert num_splits == 1
    B, HQ, D = q.shape
    _, HKV, S, _ = kq.packed.shape
    a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                        v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                        seq_lens=seq_lens.data_ptr(), out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV,
                        S=S, D=D, k_nbits=kq.nbits, v_nbits=vq.nbits, group_size=kq.group_size,
                        sm_scale=D ** -0.5, split_size=S, num_splits=1, waves=waves)
    _lib.check(_lib.load().tkv_fused_decode_attention(a, _lib.stream_handle(q.device)), "fused")
    torch.cuda.synchronize()


TWELVE_WAVE_CASES = [
    # (K bits, V bits, group size, HQ, HKV): formats with a 12-wave kernel, and
    # one without (4-bit gs32), whose 12-wave request runs 8 waves
    (2, 2, 32, 8, 2),
    (2, 2, 128, 12, 2),
    (4, 4, 128, 12, 2),
    (4, 4, 32, 8, 2),
]


@pytest.mark.parametrize("case", TWELVE_WAVE_CASES, ids=lambda c: "K{}V{}-gs{}-G{}".format(
    c[0], c[1], c[2], c[3] // c[4]))
def test_twelve_wave_workgroups(case):
    """12-wave workgroups (one split of 9000 tokens, rows of 9000, 100 and 5000
    tokens: a short row leaves most waves without a chunk) against the oracle
    and against 8 waves; the default wave count of a long split is 12 exactly
    for the listed formats."""
    from tritonkv_amd.kernels.fused_decode_attn import choose_waves, twelve_wave_format
    from tritonkv_amd.quantize import quantize_groupwise

    kb, vb, gs, HQ, HKV = case
    B, S, D = 3, 9000, 128
    print(f"twelve waves {case}", flush=True)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=29 + kb + gs)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kq, vq = quantize_groupwise(k, kb, gs), quantize_groupwise(v, vb, gs)
    lens = torch.tensor([9000, 100, 5000], dtype=torch.int32)
    listed = twelve_wave_format(D, HQ // HKV, kb, vb, gs)
    assert listed == (case != (4, 4, 32, 8, 2))
    assert choose_waves(B, HKV, HQ // HKV, S, 1, D=D, k_nbits=kb, v_nbits=vb,
                        group_size=gs) == (12 if listed else 8)
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens.numpy())
    outs = {}
    for waves in (12, 8):
        got = torch.empty(B, HQ, D, device=DEV)
        _launch(q, kq, vq, got, num_splits=1, waves=waves, seq_lens=lens.to(DEV))
        assert_close_to_reference(got, ref, f"{case} waves={waves}")
        outs[waves] = got
    if not listed:  # the request ran the 8-wave kernel
        assert torch.equal(outs[12], outs[8])
    got = _fused(q, kq, vq, seq_lens=lens.to(DEV), num_splits=1)  # the Python API's default
    assert_close_to_reference(got, ref, f"{case} default waves")


def test_append_then_decode_ragged_batch():
    """The 70B-style decode step at reduced size: per-row lengths, K 4-bit /
    V 2-bit, one new token appended by the GPU quantizer at position S_b, then
    attention over S_b + 1 tokens -- against the oracle on the caches the step
    produced, and with the appended rows checked against the oracle quantizer."""
    from tritonkv_amd.quantize import QuantizedTensor, append_kv, empty_cache

    B, HQ, HKV, D, gs, cap = 4, 32, 4, 128, 32, 3072
    lens = torch.tensor([3000, 1, 1234, 2047], dtype=torch.int32)
    q, k, v = oinp.make_random_kv(B, HQ, HKV, cap, D, seed=23)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kc = empty_cache(B, HKV, cap, D, 4, gs, DEV)
    vc = empty_cache(B, HKV, cap, D, 2, gs, DEV)
    for t in (kc.packed, vc.packed, kc.scale, kc.zero, vc.scale, vc.zero):
        t.view(torch.uint8).fill_(0xFF)  # never-written slots: fp16 NaN scale/zero
    for b in range(B):
        L = int(lens[b])
        for cache, x in ((kc, k), (vc, v)):
            view = QuantizedTensor(cache.packed[b:b + 1], cache.scale[b:b + 1], cache.zero[b:b + 1],
                                   cache.nbits, gs, D)
            append_kv(view, x[b:b + 1, :, :L].contiguous())
    k_new = k[:, :, -1:].contiguous()
    v_new = v[:, :, -1:].contiguous()
    append_kv(kc, k_new, lens.to(DEV))
    append_kv(vc, v_new, lens.to(DEV))
    lens1 = lens + 1
    for ns in (None, 1, 7):
        got = _fused(q, kc, vc, seq_lens=lens1.to(DEV), allow_mixed_bits=True, num_splits=ns)
        assert torch.isfinite(got).all(), ns
        clean = []
        for cache in (kc, vc):  # the oracle sees zeros where the kernel saw NaN garbage
            c = QuantizedTensor(cache.packed.clone(), cache.scale.clone(), cache.zero.clone(),
                                cache.nbits, gs, D)
            for b in range(B):
                L = int(lens1[b])
                c.packed[b, :, L:] = 0
                c.scale[b, :, L:] = 0
                c.zero[b, :, L:] = 0
            clean.append(c)
        ref = oracle_attention_on_quant(q, clean[0], clean[1], seq_lens=lens1.numpy())
        assert_close_to_reference(got, ref, f"append + ragged decode ns={ns}")
    # the appended token of every row is what the oracle quantizer makes of it
    for cache, x in ((kc, k_new), (vc, v_new)):
        want = oq.quantize_groupwise(x.cpu().numpy(), cache.nbits, gs)
        for b in range(B):
            L = int(lens[b])
            assert np.array_equal(cache.packed[b, :, L].cpu().numpy(), want.packed[b, :, 0])
            assert np.array_equal(cache.scale[b, :, L].cpu().numpy().view(np.uint16),
                                  want.scale[b, :, 0].view(np.uint16))
            assert np.array_equal(cache.zero[b, :, L].cpu().numpy().view(np.uint16),
                                  want.zero[b, :, 0].view(np.uint16))


def test_fp16_control_ignores_nan_rows_past_each_length():
    from tritonkv_amd.kernels import fp16_decode_attention

    B, HQ, HKV, S, D = 3, 16, 2, 700, 128
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=29)
    lens = torch.tensor([700, 45, 333], dtype=torch.int32)
    kg, vg = k.clone(), v.clone()
    for b in range(B):
        kg[b, :, int(lens[b]):] = float("nan")
        vg[b, :, int(lens[b]):] = float("inf")
    for ns in (None, 1, 5):
        got = fp16_decode_attention(q.to(DEV), kg.to(DEV), vg.to(DEV), seq_lens=lens.to(DEV),
                                    num_splits=ns).cpu().numpy()
        assert np.isfinite(got).all(), ns
        ref = oatt.reference_decode_attention_f64(q.float().numpy(), k.float().numpy(),
                                                  v.float().numpy(), seq_lens=lens.numpy())
        assert np.abs(got - ref).max() <= 2e-3, ns


@pytest.mark.parametrize("S", [1, 17, 1000, 8192, 16384])
@pytest.mark.parametrize("shape", [(1, 12, 2, 128), (2, 32, 8, 64)])
def test_fp16_control_matches_fp32_reference(S, shape):
    from tritonkv_amd.kernels import fp16_decode_attention

    B, HQ, HKV, D = shape
    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=18)
    got = fp16_decode_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    ref = oatt.reference_decode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    assert_close_to_reference(got, ref, f"fp16 control S={S} {shape}")


@pytest.mark.parametrize("num_splits", [1, 3, 64])
def test_fp16_control_split_invariance(num_splits):
    from tritonkv_amd.kernels import fp16_decode_attention

    q, k, v = oinp.make_random_kv(1, 12, 2, 4096, 128, seed=19)
    got = fp16_decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), num_splits=num_splits)
    ref = oatt.reference_decode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    assert_close_to_reference(got, ref, f"fp16 control ns={num_splits}")


def test_graph_replay_matches_eager():
    """Captured decode steps (fused + control) replayed with eager work in between."""
    from tritonkv_amd.kernels import fp16_decode_attention

    q, k, v, kq, vq = make_case(1, 12, 2, 128, 8192, 4, 32, 20)
    out_f = torch.empty(1, 12, 128, device=DEV)
    out_c = torch.empty(1, 12, 128, device=DEV)
    ws_f, ws_c = {}, {}
    want_f = _fused(q, kq, vq, out=out_f, _workspace=ws_f).clone()
    want_c = fp16_decode_attention(q, k, v, out=out_c, _workspace=ws_c).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _fused(q, kq, vq, out=out_f, _workspace=ws_f)
        fp16_decode_attention(q, k, v, out=out_c, _workspace=ws_c)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        _fused(q, kq, vq, out=out_f, _workspace=ws_f)
        fp16_decode_attention(q, k, v, out=out_c, _workspace=ws_c)
    for i in range(4):
        out_f.zero_(), out_c.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_f, want_f), i
        assert torch.equal(out_c, want_c), i
        _ = (q.float() * 2).sum().item()  # eager work between replays


def test_split_partials_combine_through_the_c_abi():
    """tkv_fused_decode_split + tkv_combine_splits == tkv_fused_decode_attention."""
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits

    q, k, v, kq, vq = make_case(2, 12, 2, 128, 3333, 4, 32, 22)
    _, ns, size = plan_splits(3333, 64, 9, 2, 2, 6)
    acc = torch.empty(2, 12, ns, 128, device=DEV)
    mx = torch.empty(2, 12, ns, device=DEV)
    sm = torch.empty(2, 12, ns, device=DEV)
    out = torch.empty(2, 12, 128, device=DEV)
    a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                        v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                        acc=acc.data_ptr(), maxs=mx.data_ptr(), sums=sm.data_ptr(),
                        out=out.data_ptr(), B=2, HQ=12, HKV=2, S=3333, D=128, k_nbits=4,
                        v_nbits=4, group_size=32, sm_scale=128 ** -0.5, split_size=size,
                        num_splits=ns)
    L = _lib.load()
    st = _lib.stream_handle(q.device)
    _lib.check(L.tkv_fused_decode_split(a, st), "split")
    _lib.check(L.tkv_combine_splits(acc.data_ptr(), mx.data_ptr(), sm.data_ptr(), out.data_ptr(),
                                    2, 12, ns, 128, st), "combine")
    # The wrapper may pick another workgroup size (a different per-wave token
    # partition, hence different fp16 rounding of P) and merges the partials
    # inside the split kernel: equal within the kernel's own rounding.
    want = _fused(q, kq, vq, num_splits=9)
    ref = oracle_attention_on_quant(q, kq, vq)
    assert_close_to_reference(out, ref, "split + combine kernels")
    assert_close_to_reference(want, ref, "wrapper")
    assert (out - want).abs().max().item() < 1e-3
    # The partials themselves: each split's acc/sum is the split-local softmax numerator/denominator.
    m = mx.cpu().numpy()
    assert np.isfinite(m).all() and (sm.cpu().numpy() > 0).all()


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("fused_combine", [False, True])
@pytest.mark.parametrize("num_splits", [1, 3, 40])
def test_workgroup_size_and_combine_mode(waves, fused_combine, num_splits):
    """Both workgroup sizes and both combine modes (separate kernel / last workgroup)."""
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits

    B, HQ, HKV, D, S = 2, 12, 2, 128, 5000
    q, k, v, kq, vq = make_case(B, HQ, HKV, D, S, 4, 32, 23)
    _, ns, size = plan_splits(S, 64, num_splits, B, HKV, HQ // HKV)
    acc = torch.empty(B, HQ, ns, D, device=DEV)
    mx = torch.empty(B, HQ, ns, device=DEV)
    sm = torch.empty(B, HQ, ns, device=DEV)
    cnt = torch.zeros(B * HKV, dtype=torch.int32, device=DEV)
    out = torch.empty(B, HQ, D, device=DEV)
    a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                        v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                        acc=acc.data_ptr(), maxs=mx.data_ptr(), sums=sm.data_ptr(),
                        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=4,
                        v_nbits=4, group_size=32, sm_scale=D ** -0.5, split_size=size,
                        num_splits=ns, counters=cnt.data_ptr() if fused_combine else None,
                        waves=waves)
    ref = oracle_attention_on_quant(q, kq, vq)
    for rep in range(3):  # the tickets must reset after every call
        out.fill_(float("nan"))
        _lib.check(_lib.load().tkv_fused_decode_attention(a, _lib.stream_handle(q.device)), "fused")
        torch.cuda.synchronize()
        assert_close_to_reference(out, ref, f"waves={waves} fused={fused_combine} ns={ns} rep={rep}")
        assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("fused_combine", [False, True])
def test_twelve_wave_splits_and_combine_modes(fused_combine):
    """12-wave workgroups writing split partials (3 splits), merged by the
    combine kernel or by the last workgroup; the tickets reset every call."""
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits

    B, HQ, HKV, D, S = 2, 8, 2, 128, 5000
    q, k, v, kq, vq = make_case(B, HQ, HKV, D, S, 2, 32, 31)
    _, ns, size = plan_splits(S, 64, 3, B, HKV, HQ // HKV)
    acc = torch.empty(B, HQ, ns, D, device=DEV)
    mx = torch.empty(B, HQ, ns, device=DEV)
    sm = torch.empty(B, HQ, ns, device=DEV)
    cnt = torch.zeros(B * HKV, dtype=torch.int32, device=DEV)
    out = torch.empty(B, HQ, D, device=DEV)
    a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                        v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                        acc=acc.data_ptr(), maxs=mx.data_ptr(), sums=sm.data_ptr(),
                        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=2,
                        v_nbits=2, group_size=32, sm_scale=D ** -0.5, split_size=size,
                        num_splits=ns, counters=cnt.data_ptr() if fused_combine else None,
                        waves=12)
    ref = oracle_attention_on_quant(q, kq, vq)
    for rep in range(3):
        out.fill_(float("nan"))
        _lib.check(_lib.load().tkv_fused_decode_attention(a, _lib.stream_handle(q.device)), "fused")
        torch.cuda.synchronize()
        assert_close_to_reference(out, ref, f"12 waves fused={fused_combine} ns={ns} rep={rep}")
        assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("num_splits", [8, 32])
def test_fused_combine_reads_this_calls_partials(num_splits):
    """The in-kernel combine hands partials between workgroups (possibly on
    other XCDs) through coherent stores and loads.  Back-to-back calls on one
    workspace with a different q each: a partial read stale from the previous
    call would hold that call's values.  Each output must equal, bit for bit,
    the same fused call on a fresh workspace whose partials start as NaN, and
    the oracle within tolerance."""
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits

    B, HQ, HKV, D, S = 2, 12, 2, 128, 6000
    print(f"fused combine, new q per call, ns={num_splits}", flush=True)
    _, _, _, kq, vq = make_case(B, HQ, HKV, D, S, 4, 32, 41)
    _, ns, size = plan_splits(S, 64, num_splits, B, HKV, HQ // HKV)
    lib, st = _lib.load(), _lib.stream_handle(torch.device(DEV))

    def workspace(fill):
        return (torch.full((B, HQ, ns, D), fill, device=DEV),
                torch.full((B, HQ, ns), fill, device=DEV),
                torch.full((B, HQ, ns), fill, device=DEV),
                torch.zeros(B * HKV, dtype=torch.int32, device=DEV))

    def call(q, ws, out):
        acc, mx, sm, cnt = ws
        a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                            k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                            v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                            acc=acc.data_ptr(), maxs=mx.data_ptr(), sums=sm.data_ptr(),
                            out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=4,
                            v_nbits=4, group_size=32, sm_scale=D ** -0.5, split_size=size,
                            num_splits=ns, counters=cnt.data_ptr(), waves=8)
        _lib.check(lib.tkv_fused_decode_attention(a, st), "fused combine")

    shared = workspace(0.0)
    g = torch.Generator().manual_seed(5)
    qs = [(torch.randn(B, HQ, D, generator=g) * (1 + 2 * i)).half().to(DEV) for i in range(6)]
    outs = [torch.full((B, HQ, D), float("nan"), device=DEV) for _ in qs]
    for q, out in zip(qs, outs):  # back to back, no host sync between the calls
        call(q, shared, out)
    torch.cuda.synchronize()
    assert int(shared[3].abs().sum()) == 0
    for i, (q, out) in enumerate(zip(qs, outs)):
        fresh_out = torch.full((B, HQ, D), float("nan"), device=DEV)
        call(q, workspace(float("nan")), fresh_out)
        torch.cuda.synchronize()
        assert torch.equal(out, fresh_out), f"call {i}: differs from the fresh-workspace call"
        assert_close_to_reference(out, oracle_attention_on_quant(q, kq, vq), f"call {i}")


@pytest.mark.parametrize("kbits,vbits,gs,waves", [(4, 4, 32, 8), (2, 2, 128, 4), (4, 2, 32, 8)])
def test_read_probe_runs_over_the_split_kernels_reads(kbits, vbits, gs, waves):
    """tkv_read_probe (the bandwidth-ceiling probe of the split kernel's access
    pattern) launches over a cache like the split kernel and leaves the
    caller's out untouched."""
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, S = 2, 8, 2, 128, 5000
    print(f"read probe K{kbits}V{vbits} gs={gs} waves={waves}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(2, B, HKV, S, D, device=DEV, generator=g, dtype=torch.float16)
    kq, vq = quantize_groupwise(x[0], kbits, gs), quantize_groupwise(x[1], vbits, gs)
    q = torch.randn(B, HQ, D, device=DEV, generator=g, dtype=torch.float16)
    _, ns, size = plan_splits(S, 64, 3, B, HKV, HQ // HKV)
    out = torch.full((B, HQ, D), 7.0, device=DEV)
    a = _lib.DecodeArgs(q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
                        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(),
                        v_scale=vq.scale.data_ptr(), v_zero=vq.zero.data_ptr(),
                        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=kbits,
                        v_nbits=vbits, group_size=gs, sm_scale=D ** -0.5, split_size=size,
                        num_splits=ns, waves=waves)
    acc = torch.empty(B, HQ, ns, D, device=DEV)
    a.acc = a.maxs = a.sums = acc.data_ptr()
    for _ in range(3):
        _lib.check(_lib.load().tkv_read_probe(a, _lib.stream_handle(q.device)), "read probe")
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_workspace_reuses_the_checked_argument_block():
    """A ``_workspace`` keeps the checked argument block of its last call
    (``_PreparedCall``); a later call with the same caches, buffers and flags
    reuses it with its own q (and new token).  Every output must equal, bit for
    bit, the same call without a workspace: a new q per call, ``out=None``,
    another cache on the same workspace, a misaligned q, the fused append with
    a new token per step, and the fp16 control."""
    from tritonkv_amd.kernels import fp16_decode_attention, fused_decode_attention
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, S = 2, 12, 2, 128, 3000
    print("prepared-call reuse", flush=True)
    _, k, v, kq, vq = make_case(B, HQ, HKV, D, S, 4, 32, 51)
    g = torch.Generator().manual_seed(52)
    ws, out = {}, torch.empty(B, HQ, D, device=DEV)
    for i in range(4):
        qi = (torch.randn(B, HQ, D, generator=g) * (1 + i)).half().to(DEV)
        got = fused_decode_attention(qi, kq, vq, out=out, _workspace=ws)
        assert got is out and "call" in ws
        assert torch.equal(got, fused_decode_attention(qi, kq, vq)), i
    prep = ws["call"]
    got = fused_decode_attention(qi, kq, vq, _workspace=ws)  # out=None: a new tensor
    assert got is not out and torch.equal(got, out)
    _, _, _, kq2, vq2 = make_case(B, HQ, HKV, D, S, 4, 32, 53)  # another cache
    got = fused_decode_attention(qi, kq2, vq2, out=out, _workspace=ws)
    assert ws["call"] is not prep and torch.equal(got, fused_decode_attention(qi, kq2, vq2))
    buf = torch.empty(B * HQ * D + 1, dtype=torch.float16, device=DEV)
    qm = buf[1:].view(B, HQ, D)  # 2 bytes past a 16-byte boundary: the full path
    qm.copy_(qi)
    got = fused_decode_attention(qm, kq2, vq2, out=out, _workspace=ws)
    assert torch.equal(got, fused_decode_attention(qi, kq2, vq2))
    # fused append: a new token per step, on two copies of the cache
    ka = quantize_groupwise(k.to(DEV), 4, 32)
    va = quantize_groupwise(v.to(DEV), 4, 32)
    kb = type(ka)(ka.packed.clone(), ka.scale.clone(), ka.zero.clone(), 4, 32, D)
    vb = type(va)(va.packed.clone(), va.scale.clone(), va.zero.clone(), 4, 32, D)
    ws2 = {}
    for i in range(3):
        lens = torch.full((B,), S - 3 + i + 1, dtype=torch.int32, device=DEV)
        kn = torch.randn(B, HKV, D, generator=g).half().to(DEV)
        vn = torch.randn(B, HKV, D, generator=g).half().to(DEV)
        qi = torch.randn(B, HQ, D, generator=g).half().to(DEV)
        got = fused_decode_attention(qi, ka, va, seq_lens=lens, k_new=kn, v_new=vn,
                                     out=out, _workspace=ws2)
        want = fused_decode_attention(qi, kb, vb, seq_lens=lens, k_new=kn, v_new=vn)
        assert torch.equal(got, want), i
    assert torch.equal(ka.packed, kb.packed) and torch.equal(va.zero, vb.zero)
    # the fp16 control
    kf, vf = k.to(DEV), v.to(DEV)
    ws3 = {}
    for i in range(3):
        qi = torch.randn(B, HQ, D, generator=g).half().to(DEV)
        got = fp16_decode_attention(qi, kf, vf, out=out, _workspace=ws3)
        assert torch.equal(got, fp16_decode_attention(qi, kf, vf)), i
    assert "call" in ws3
