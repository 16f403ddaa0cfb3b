"""GPU test of ``tkv_fused_decode_attention_noalloc`` through the C ABI.

The entry point keeps the split partials in a static device array instead of
a caller's workspace.  It runs the same kernels as
``tkv_fused_decode_attention``, so its output must be bitwise equal to that
entry point's on the same arguments.  Two calls run back to back, the second
on a smaller input, so the second one reads the array after the first has
left its partials there; a third call uses one split (no partials at all).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests.helpers import assert_close_to_reference, make_case, oracle_attention_on_quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(q, kq, vq, ns, size, out, seq_lens=None, ws=None, waves=0):
    from tritonkv_amd import _lib

    B, HQ, D = q.shape
    HKV, S = kq.packed.shape[1], kq.packed.shape[2]
    acc, mx, sm = ws if ws is not None else (None, None, None)
    return _lib.DecodeArgs(
        q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(), v_scale=vq.scale.data_ptr(),
        v_zero=vq.zero.data_ptr(), seq_lens=_lib.ptr(seq_lens), acc=_lib.ptr(acc),
        maxs=_lib.ptr(mx), sums=_lib.ptr(sm), out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S,
        D=D, k_nbits=kq.nbits, v_nbits=vq.nbits, group_size=kq.group_size,
        sm_scale=D ** -0.5, split_size=size, num_splits=ns, waves=waves)


def _one_call(B, HQ, HKV, D, S, nbits, gs, seed, num_splits, lens=None, waves=0):
    from tritonkv_amd import _lib
    from tritonkv_amd.kernels import plan_splits

    print(f"noalloc case B={B} HQ={HQ} HKV={HKV} D={D} S={S} nbits={nbits} gs={gs} "
          f"ns={num_splits} lens={lens} waves={waves}", flush=True)
    q, k, v, kq, vq = make_case(B, HQ, HKV, D, S, nbits, gs, seed)
    _, ns, size = plan_splits(S, 64, num_splits, B, HKV, HQ // HKV)
    seq_lens = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    ws = None
    if ns > 1:
        ws = (torch.empty(B, HQ, ns, D, device=DEV), torch.empty(B, HQ, ns, device=DEV),
              torch.empty(B, HQ, ns, device=DEV))
    want = torch.full((B, HQ, D), float("nan"), device=DEV)
    got = torch.full((B, HQ, D), float("nan"), device=DEV)
    L = _lib.load()
    st = _lib.stream_handle(q.device)
    _lib.check(L.tkv_fused_decode_attention(_args(q, kq, vq, ns, size, want, seq_lens, ws, waves),
                                            st), "tkv_fused_decode_attention")
    _lib.check(L.tkv_fused_decode_attention_noalloc(_args(q, kq, vq, ns, size, got, seq_lens,
                                                          None, waves), st),
               "tkv_fused_decode_attention_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got - want).abs().max().item()
    ref = oracle_attention_on_quant(q, kq, vq, seq_lens=lens)
    assert_close_to_reference(got, ref, f"noalloc S={S} nbits={nbits} gs={gs} ns={ns}")
    return ns


def test_noalloc_matches_the_workspace_entry_point_on_consecutive_calls():
    # 1: ragged rows, so some splits of row 1 are empty (they still write their partials)
    ns = _one_call(2, 12, 2, 128, 6000, 4, 32, 41, 23, lens=[6000, 2500])
    assert ns > 1
    # 2: a smaller input right after, reusing the array's stale partials region
    ns = _one_call(1, 12, 2, 128, 1500, 2, 64, 42, 5, waves=4)
    assert ns > 1
    # 3: one split -- no partials, the array is not used
    assert _one_call(1, 8, 8, 64, 700, 4, 16, 43, 1) == 1


def test_noalloc_rejects_a_workspace_and_oversized_partials():
    from tritonkv_amd import _lib

    q, k, v, kq, vq = make_case(1, 12, 2, 128, 4096, 4, 32, 44)
    out = torch.empty(1, 12, 128, device=DEV)
    L = _lib.load()
    st = _lib.stream_handle(q.device)
    acc = torch.empty(1, 12, 8, 128, device=DEV)
    a = _args(q, kq, vq, 8, 512, out, ws=(acc, acc, acc))
    assert L.tkv_fused_decode_attention_noalloc(ctypes.byref(a), st) == _lib.TKV_EINVAL
    # 12 rows x 4096 splits x 130 floats > 16 MiB: rejected, nothing launched
    big = _args(q, kq, vq, 4096, 1, out)
    big.S = 4096
    assert L.tkv_fused_decode_attention_noalloc(ctypes.byref(big), st) == _lib.TKV_ESCRATCH
    torch.cuda.synchronize()
