"""fp16 flash-decoding attention on MI355X -- the *control* for the fused kernel.

Drop-in for the reference's ``kernels/fp16_decode_attn.py``
(``fp16_decode_attention`` :142-241).  It shares the fused path's split
arithmetic, workspace, C-ABI skeleton (``tkv_fp16_decode_attention``), online
softmax, GQA grouping, workgroup merge and combine kernel.  Two differences
besides the unpack remain, both deliberate:

* the default split targets 256 tokens per workgroup instead of 512 (an fp16
  token is 3-6x the bytes of a packed one); ``num_splits=`` set to the fused
  call's count gives the reference's identical split (``:161-163``), and the
  benchmark reports the quantization effect both ways;
* K/V rows are prefetched into registers (16-byte non-temporal loads, one
  chunk ahead) rather than staged through LDS: two LDS stages of fp16 chunks
  per wave would not fit 8 waves in a CU's LDS.

So fused vs control isolates the quantization effect, and SDPA vs control the
flash-decoding effect (reference :1-25).
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from .fused_decode_attn import (
    TOKENS_PER_WORKGROUP_FP16,
    _aligned16,
    _cache_arg,
    _check_out,
    _PreparedCall,
    _prepared,
    _seq_lens_arg,
    _tensor_key,
    _workspace_for,
    choose_waves,
    plan_splits,
    triton_available,
)


def fp16_decode_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    sm_scale: float | None = None,
    block_n: int = 64,
    num_warps: int = 4,
    num_stages: int = 2,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    _workspace: dict | None = None,
    *,
    seq_lens: torch.Tensor | None = None,
    equal_lengths: bool = False,
) -> torch.Tensor:
    """Decode attention on an unquantized fp16 cache, same shape as the fused kernel.

    q: (B, HQ, D); k, v: (B, HKV, S, D) fp16. Returns (B, HQ, D) float32.
    ``seq_lens`` / ``equal_lengths`` and the reuse of a workspace's checked
    argument block as for ``fused_decode_attention``.
    """
    key = None
    if _workspace is not None:
        key = ("fp16", q.shape, q.dtype, q.device, q.is_contiguous(), _tensor_key(k),
               _tensor_key(v), sm_scale, block_n, num_splits, _tensor_key(out),
               _tensor_key(seq_lens), equal_lengths)
        prep = _prepared(_workspace, key)
        if prep is not None:
            res = prep.run(q, out)
            if res is not None:
                return res
    B, HQ, D = q.shape
    _, HKV, S, _ = k.shape
    if HQ % HKV != 0:
        raise ValueError(f"HQ={HQ} must be a multiple of HKV={HKV}")
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} incompatible with q {tuple(q.shape)}")
    if k.device != q.device or v.device != q.device:
        raise ValueError("q, k and v must be on the same device")

    ok, why = triton_available()
    if not ok:
        raise RuntimeError(f"tritonkv_amd HIP backend unavailable: {why}")

    group = HQ // HKV
    sm_scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    _, num_splits, split_size = plan_splits(S, block_n, num_splits, B, HKV, group,
                                            TOKENS_PER_WORKGROUP_FP16,
                                            ragged=seq_lens is not None and not equal_lengths)

    q_in = q
    if q.dtype not in (torch.float16, torch.float32):
        q = q.float()
    q = _aligned16(q)
    k_in, v_in = k, v
    k = _cache_arg(k if k.dtype == torch.float16 else k.half(), 16, "k")
    v = _cache_arg(v if v.dtype == torch.float16 else v.half(), 16, "v")
    out = _check_out(out, B, HQ, D, q.device)
    acc, maxs, sums, counters = _workspace_for(_workspace, B, HQ, num_splits, D, q.device, HKV)
    lens = _seq_lens_arg(seq_lens, B, S, q.device)

    args = _lib.DecodeArgs(
        q=q.data_ptr(), q_is_fp32=int(q.dtype == torch.float32),
        k=k.data_ptr(), v=v.data_ptr(), seq_lens=_lib.ptr(lens),
        acc=_lib.ptr(acc), maxs=_lib.ptr(maxs), sums=_lib.ptr(sums), out=out.data_ptr(),
        B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=16, v_nbits=16, group_size=D,
        sm_scale=float(sm_scale), split_size=split_size, num_splits=num_splits,
        counters=None, waves=choose_waves(B, HKV, group, split_size, num_splits))
    with torch.cuda.device(q.device):
        rc = _lib.load().tkv_fp16_decode_attention(args, _lib.stream_handle(q.device))
    _lib.check(rc, "fp16_decode_attention")
    # k / v are read in place; a converted copy (not fp16, not contiguous) is not kept
    if key is not None and q is q_in and k is k_in and v is v_in:
        _workspace["call"] = _PreparedCall(key, args, _lib.load().tkv_fp16_decode_attention,
                                           "fp16_decode_attention", (B, HQ, D), q.device, False)
    return out
