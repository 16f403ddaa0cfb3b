"""Paged quantized KV cache: page pools addressed through a block table.

The reference keeps one contiguous ``(B, HKV, S, ...)`` cache per sequence
(``quantize.py:218-225``), so growing a sequence means reallocating it.  A
serving engine instead carves HBM into fixed-size pages and gives every
sequence a block table of page indices.  Here a *pool* is an ordinary
:class:`~tritonkv_amd.quantize.QuantizedTensor` whose leading axis counts pages
instead of sequences:

    packed  (num_pages, HKV, page_size, D/P)  uint8   split-P codes
    scale   (num_pages, HKV, page_size, D/gs) fp16
    zero    (num_pages, HKV, page_size, D/gs) fp16

Logical token t of batch row b lives in page ``block_table[b, t // page_size]``
at slot ``t % page_size``.  Each (page, kv head) slab is ``page_size``
consecutive rows of the same per-row format as the contiguous cache, so the
decode kernel streams a page exactly as it streams a contiguous block; only
the buffer base changes at page boundaries.  ``page_size`` must be a multiple
of 32 (the kernel's token chunk), so a chunk never straddles two pages.

Codes, metadata and results are bit-identical to the contiguous cache holding
the same logical tokens.  The fp16 control has no paged form.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .kernels.fused_decode_attn import (_aligned16, _check_out, _order_for, _workspace_for,
                                        choose_waves, new_token_args, plan_splits,
                                        triton_available)
from .quantize import QuantizedTensor, _check_bits, _require_gpu, empty_cache

PAGE_MULTIPLE = 32


def empty_paged_pool(num_pages: int, HKV: int, page_size: int, D: int, nbits: int,
                     group_size: int, device="cuda") -> QuantizedTensor:
    """An uninitialised page pool of ``num_pages`` pages of ``page_size`` tokens."""
    if page_size <= 0 or page_size % PAGE_MULTIPLE:
        raise ValueError(f"page_size must be a positive multiple of {PAGE_MULTIPLE}, got {page_size}")
    if num_pages <= 0:
        raise ValueError(f"num_pages must be positive, got {num_pages}")
    return empty_cache(num_pages, HKV, page_size, D, nbits, group_size, device=device)


def _check_pool(pool: QuantizedTensor, what: str) -> None:
    _check_bits(pool.nbits)
    if pool.packed.dim() != 4:
        raise ValueError(f"{what} must have packed shape (num_pages, HKV, page_size, D/P)")
    page_size = pool.packed.shape[2]
    if page_size % PAGE_MULTIPLE:
        raise ValueError(f"{what} page_size must be a multiple of {PAGE_MULTIPLE}, got {page_size}")
    for t in (pool.packed, pool.scale, pool.zero):
        if not t.is_contiguous():
            raise ValueError(f"{what} tensors must be contiguous")


def _check_table(block_table: torch.Tensor, B: int, device) -> torch.Tensor:
    if not isinstance(block_table, torch.Tensor) or block_table.dtype != torch.int32 \
            or block_table.dim() != 2 or block_table.shape[0] != B \
            or block_table.device != torch.device(device):
        raise ValueError("block_table must be an int32 (B, max_pages) tensor on the pool's device")
    if block_table.shape[1] == 0:
        raise ValueError("block_table must have at least one column")
    return block_table.contiguous()


def paged_append(pool: QuantizedTensor, x_new: torch.Tensor, block_table: torch.Tensor,
                 positions: torch.Tensor) -> QuantizedTensor:
    """Quantize ``x_new`` ``(B, HKV, N, D)`` into a page pool.

    Row b's N tokens take logical positions ``[positions[b], positions[b]+N)``
    and land in the pages the block table names.  Tokens past
    ``block_table.shape[1] * page_size``, or mapped to a table entry outside
    ``[0, num_pages)``, are not written.  Bit-exact with
    :func:`~tritonkv_amd.quantize.append_kv` on a contiguous cache; allocates
    nothing and does not synchronise.
    """
    _require_gpu(x_new, "paged_append")
    _check_pool(pool, "pool")
    B, HKV, N, D = x_new.shape
    num_pages, HKVp, page_size, _ = pool.packed.shape
    if (HKV, D) != (HKVp, pool.head_dim):
        raise ValueError(f"x_new shape {tuple(x_new.shape)} incompatible with pool "
                         f"{tuple(pool.packed.shape)} (head_dim {pool.head_dim})")
    if x_new.dtype not in (torch.float16, torch.float32):
        raise TypeError(f"x_new must be float16 or float32, got {x_new.dtype}")
    if pool.packed.device != x_new.device:
        raise ValueError(f"x_new is on {x_new.device}, the pool on {pool.packed.device}")
    if positions is None or positions.dtype != torch.int32 or positions.numel() != B \
            or positions.device != x_new.device:
        raise ValueError("positions must be an int32 tensor of B entries on the pool's device")
    table = _check_table(block_table, B, x_new.device)
    xc = x_new.contiguous()
    with torch.cuda.device(x_new.device):
        rc = _lib.load().tkv_paged_quantize_pack(
            xc.data_ptr(), int(xc.dtype == torch.float32), B, HKV, N, D, pool.nbits,
            pool.group_size, positions.contiguous().data_ptr(), table.data_ptr(),
            table.shape[1], page_size, num_pages, pool.packed.data_ptr(), pool.scale.data_ptr(),
            pool.zero.data_ptr(), _lib.stream_handle(x_new.device))
        _lib.check(rc, "paged_append")
    return pool


def paged_decode_attention(
    q: torch.Tensor,
    k_pool: QuantizedTensor,
    v_pool: QuantizedTensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor | None = None,
    sm_scale: float | None = None,
    block_n: int = 64,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    _workspace: dict | None = None,
    *,
    allow_mixed_bits: bool = False,
    k_new: torch.Tensor | None = None,
    v_new: torch.Tensor | None = None,
    dispatch_order: bool | None = None,
    equal_lengths: bool = False,
) -> torch.Tensor:
    """One decode step of attention over paged 2/4-bit K/V pools.

    q: ``(B, HQ, D)``; pools as :func:`empty_paged_pool`; block_table:
    ``(B, max_pages)`` int32; seq_lens: ``(B,)`` int32 (None = every row holds
    ``max_pages * page_size`` tokens).  Same split planning, workspace reuse
    and ``out`` contract as
    :func:`~tritonkv_amd.kernels.fused_decode_attention`; returns
    ``(B, HQ, D)`` float32, bit-identical to that function on a contiguous
    cache holding the same tokens with the same ``num_splits``.  ``k_new`` /
    ``v_new`` fuse the step's append into the same launch (the token lands at
    ``seq_lens[b] - 1``), bit-identical to :func:`paged_append` followed by
    this call.  ``dispatch_order`` and ``equal_lengths`` as for
    ``fused_decode_attention``.
    """
    if k_pool.group_size != v_pool.group_size or (k_pool.nbits != v_pool.nbits
                                                  and not allow_mixed_bits):
        raise ValueError("K and V must use the same nbits/group_size")
    _check_pool(k_pool, "k_pool")
    _check_pool(v_pool, "v_pool")
    B, HQ, D = q.shape
    num_pages, HKV, page_size, _ = k_pool.packed.shape
    if v_pool.packed.shape[:3] != k_pool.packed.shape[:3] or v_pool.head_dim != k_pool.head_dim:
        raise ValueError("K and V pools must have the same shape")
    if D != k_pool.head_dim:
        raise ValueError(f"q head_dim {D} != pool head_dim {k_pool.head_dim}")
    if HQ % HKV:
        raise ValueError(f"HQ={HQ} must be a multiple of HKV={HKV}")
    if D & (D - 1):
        raise ValueError(f"head_dim must be a power of two, got {D}")
    table = _check_table(block_table, B, k_pool.device)
    S = table.shape[1] * page_size
    if seq_lens is not None and (not isinstance(seq_lens, torch.Tensor)
                                 or seq_lens.dtype != torch.int32 or seq_lens.numel() != B
                                 or seq_lens.device != q.device):
        raise ValueError("seq_lens must be an int32 tensor of B lengths on the pool's device")
    if q.device != k_pool.device or v_pool.device != k_pool.device:
        raise ValueError("q and the pools must be on the same device")
    kn, vn, new_f32 = new_token_args(k_new, v_new, B, HKV, D, q.device)
    ok, why = triton_available()
    if not ok:
        raise RuntimeError(f"paged_decode_attention requires the tritonkv_amd HIP backend: {why}")

    group = HQ // HKV
    sm_scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    ragged = seq_lens is not None and not equal_lengths
    _, num_splits, split_size = plan_splits(S, block_n, num_splits, B, HKV, group, ragged=ragged)
    if q.dtype not in (torch.float16, torch.float32):
        q = q.float()
    q = _aligned16(q)
    out = _check_out(out, B, HQ, D, q.device)
    acc, maxs, sums, _ = _workspace_for(_workspace, B, HQ, num_splits, D, q.device, HKV)
    lens = seq_lens.contiguous() if seq_lens is not None else None
    order = _order_for(_workspace, B, HKV, num_splits, q.device, seq_lens if ragged else None,
                       dispatch_order, group, D)
    args = _lib.DecodeArgs(
        q=q.data_ptr(), q_is_fp32=int(q.dtype == torch.float32),
        k=k_pool.packed.data_ptr(), k_scale=k_pool.scale.data_ptr(),
        k_zero=k_pool.zero.data_ptr(), v=v_pool.packed.data_ptr(),
        v_scale=v_pool.scale.data_ptr(), v_zero=v_pool.zero.data_ptr(),
        seq_lens=_lib.ptr(lens), acc=_lib.ptr(acc), maxs=_lib.ptr(maxs), sums=_lib.ptr(sums),
        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D,
        k_nbits=k_pool.nbits, v_nbits=v_pool.nbits, group_size=k_pool.group_size,
        sm_scale=float(sm_scale), split_size=split_size, num_splits=num_splits, counters=None,
        waves=choose_waves(B, HKV, group, split_size, num_splits, D=D, k_nbits=k_pool.nbits,
                           v_nbits=v_pool.nbits, group_size=k_pool.group_size, paged=True),
        block_table=table.data_ptr(), block_table_stride=table.shape[1], page_size=page_size,
        num_pages=num_pages, k_new=_lib.ptr(kn), v_new=_lib.ptr(vn), new_is_fp32=new_f32,
        work_order=_lib.ptr(order))
    with torch.cuda.device(q.device):
        rc = _lib.load().tkv_fused_decode_attention(args, _lib.stream_handle(q.device))
    _lib.check(rc, "paged_decode_attention")
    return out


def gather_pages(pool: QuantizedTensor, block_table: torch.Tensor) -> QuantizedTensor:
    """Contiguous ``(B, HKV, max_pages*page_size, ...)`` copy of the pages a
    block table names (a torch gather, for tests and debugging)."""
    idx = block_table.long().clamp(0, pool.packed.shape[0] - 1)

    def g(t):
        x = t[idx]  # (B, max_pages, HKV, page, F)
        B, MP, H, PG, F = x.shape
        return x.permute(0, 2, 1, 3, 4).reshape(B, H, MP * PG, F).contiguous()

    return QuantizedTensor(g(pool.packed), g(pool.scale), g(pool.zero), pool.nbits,
                           pool.group_size, pool.head_dim)


__all__ = ["PAGE_MULTIPLE", "empty_paged_pool", "paged_append", "paged_decode_attention",
           "gather_pages"]
