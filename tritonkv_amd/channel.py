"""Per-channel (KIVI-style) quantized keys with an fp16 residual window.

The reference plans this as its next key format (``docs/future_work.md:229-293``)
and has no implementation of it.  Keys whose large values sit in fixed channels
quantize badly in per-token groups (one outlier channel sets every group's
scale); grouping *along tokens, within one channel* gives each channel its own
scale.  Here:

* keys are quantized in blocks of 32 tokens (the decode kernel's chunk): within
  a block every channel is one group -- fp32 min/max, fp16 scale and zero,
  codes -- the reference's group-wise arithmetic (``quantize.py:209-226``)
  along the token axis.  Codes keep the split-P row layout of
  ``quantize.py:40-54``; scale and zero are ``(B, HKV, S / 32, D)`` fp16;
* values keep the reference's per-token groups (``QuantizedTensor``);
* tokens that do not fill a block yet stay in fp16: the residual window.  The
  decode step runs the split kernel over the quantized blocks (per-channel key
  path: the chunk's ``q * scale`` as the score operand, one dot product with
  the zero row per head), the fp16 control kernel over the window as one more
  split, and the log-sum-exp combine over both -- the plan of
  ``docs/future_work.md:259-262``.

:class:`ChannelKVCache` keeps one such cache and its window per layer, with
one length for every batch row.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .kernels.fused_decode_attn import (_aligned16, _cache_arg, _check_out, _seq_lens_arg, _workspace_for,
                                        choose_waves, plan_splits, triton_available)
from .quantize import QuantizedTensor, _check_bits, _require_gpu, append_kv, empty_cache

BLOCK = 32  # tokens per key block


@dataclass
class ChannelQuantizedKeys:
    """Keys quantized per (32-token block, channel); codes per token row."""

    packed: torch.Tensor  # uint8 (B, HKV, S, D // P), split-P
    scale: torch.Tensor   # fp16 (B, HKV, S // 32, D)
    zero: torch.Tensor    # fp16 (B, HKV, S // 32, D)
    nbits: int
    head_dim: int

    block = BLOCK

    @property
    def shape(self) -> tuple:
        B, H, S, _ = self.packed.shape
        return (B, H, S, self.head_dim)

    @property
    def device(self):
        return self.packed.device

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.packed, self.scale, self.zero))

    def effective_bits_per_element(self) -> float:
        return self.nbits + 2 * 16 / BLOCK


def empty_channel_keys(B: int, HKV: int, S: int, D: int, nbits: int,
                       device="cuda") -> ChannelQuantizedKeys:
    """An uninitialised key cache of capacity S (a multiple of 32)."""
    _check_bits(nbits)
    if S <= 0 or S % BLOCK:
        raise ValueError(f"capacity must be a positive multiple of {BLOCK}, got {S}")
    P = 8 // nbits
    return ChannelQuantizedKeys(
        packed=torch.empty((B, HKV, S, D // P), dtype=torch.uint8, device=device),
        scale=torch.empty((B, HKV, S // BLOCK, D), dtype=torch.float16, device=device),
        zero=torch.empty((B, HKV, S // BLOCK, D), dtype=torch.float16, device=device),
        nbits=nbits, head_dim=D)


def append_keys_per_channel(ck: ChannelQuantizedKeys, k_new: torch.Tensor,
                            positions: torch.Tensor | None = None) -> ChannelQuantizedKeys:
    """Quantize ``k_new`` ``(B, HKV, N, D)``, N a multiple of 32, into ``ck``.

    Row b's blocks land at tokens ``positions[b] + 32 i`` (int32 on the cache's
    device; None = 0).  A block that does not start on a 32-token boundary or
    does not fit the capacity is not written.  Allocates nothing.
    """
    _require_gpu(k_new, "append_keys_per_channel")
    B, HKV, N, D = k_new.shape
    Bc, Hc, S, _ = ck.packed.shape
    if (B, HKV, D) != (Bc, Hc, ck.head_dim):
        raise ValueError(f"k_new shape {tuple(k_new.shape)} incompatible with keys {ck.shape}")
    if N % BLOCK:
        raise ValueError(f"token count {N} must be a multiple of {BLOCK}")
    if k_new.dtype not in (torch.float16, torch.float32):
        raise TypeError(f"k_new must be float16 or float32, got {k_new.dtype}")
    if k_new.device != ck.device:
        raise ValueError(f"k_new is on {k_new.device}, the keys on {ck.device}")
    if positions is not None and (positions.dtype != torch.int32 or positions.numel() != B
                                  or positions.device != k_new.device):
        raise ValueError("positions must be an int32 tensor of B entries on the cache's device")
    kc = k_new.contiguous()
    with torch.cuda.device(k_new.device):
        rc = _lib.load().tkv_quantize_keys_channel(
            kc.data_ptr(), int(kc.dtype == torch.float32), B, HKV, N, D, ck.nbits,
            _lib.ptr(positions), S, ck.packed.data_ptr(), ck.scale.data_ptr(),
            ck.zero.data_ptr(), _lib.stream_handle(k_new.device))
        _lib.check(rc, "append_keys_per_channel")
    return ck


def quantize_keys_per_channel(k: torch.Tensor, nbits: int) -> ChannelQuantizedKeys:
    """Per-channel quantization of ``k`` ``(B, HKV, S, D)``, S a multiple of 32."""
    _require_gpu(k, "quantize_keys_per_channel")
    _check_bits(nbits)
    B, HKV, S, D = k.shape
    ck = empty_channel_keys(B, HKV, S, D, nbits, k.device)
    return append_keys_per_channel(ck, k)


def channel_decode_attention(
    q: torch.Tensor,
    ck: ChannelQuantizedKeys,
    vq: QuantizedTensor,
    k_res: torch.Tensor,
    v_res: torch.Tensor,
    q_lens: torch.Tensor | None = None,
    res_lens: torch.Tensor | None = None,
    sm_scale: float | None = None,
    block_n: int = 64,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    _workspace: dict | None = None,
    *,
    equal_lengths: bool = False,
) -> torch.Tensor:
    """One decode step over per-channel keys, per-token values and an fp16 window.

    q ``(B, HQ, D)``; ``ck``/``vq`` the quantized history of capacity S (a
    multiple of 32), row b holding ``q_lens[b]`` tokens (None = S); ``k_res``,
    ``v_res`` fp16 ``(B, HKV, R, D)``, row b's next ``res_lens[b]`` tokens
    (None = R).  Returns ``(B, HQ, D)`` float32 -- attention over each row's
    quantized tokens followed by its window tokens.  ``vq.group_size`` must be
    16 or 32.  ``num_splits`` / ``out`` / ``_workspace`` as for
    :func:`~tritonkv_amd.kernels.fused_decode_attention` (the workspace holds
    one more split, the window's); ``equal_lengths``: every entry of
    ``q_lens`` is the same, so the split plan of a batch without lengths
    applies.
    """
    for t, what in ((q, "q"), (k_res, "k_res"), (v_res, "v_res")):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{what} must be a tensor")
    B, HQ, D = q.shape
    Bk, HKV, S, Dk = ck.shape
    if (Bk, Dk) != (B, D) or vq.packed.shape[:3] != ck.packed.shape[:3] or vq.head_dim != D:
        raise ValueError(f"q {tuple(q.shape)}, keys {ck.shape} and values "
                         f"{tuple(vq.packed.shape)} are inconsistent")
    if HQ % HKV:
        raise ValueError(f"HQ={HQ} must be a multiple of HKV={HKV}")
    if vq.group_size not in (16, 32):
        raise ValueError(f"values need group_size 16 or 32 with per-channel keys, got {vq.group_size}")
    if k_res.dtype != torch.float16 or v_res.dtype != torch.float16 or k_res.dim() != 4 \
            or k_res.shape != v_res.shape or k_res.shape[:2] != (B, HKV) or k_res.shape[3] != D:
        raise ValueError("k_res / v_res must be fp16 (B, HKV, R, D) tensors of the same shape")
    if q.device != ck.device or k_res.device != q.device:
        raise ValueError("q, the caches and the window must be on the same device")
    R = k_res.shape[2]
    qlens = _seq_lens_arg(q_lens, B, S, q.device)
    rlens = _seq_lens_arg(res_lens, B, R, q.device)
    ok, why = triton_available()
    if not ok:
        raise RuntimeError(f"channel_decode_attention requires the tritonkv_amd HIP backend: {why}")

    group = HQ // HKV
    sm_scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    _, num_splits, split_size = plan_splits(S, block_n, num_splits, B, HKV, group,
                                            ragged=q_lens is not None and not equal_lengths)
    if q.dtype not in (torch.float16, torch.float32):
        q = q.float()
    q = _aligned16(q)
    kr, vr = _cache_arg(k_res, 16, "k_res"), _cache_arg(v_res, 16, "v_res")
    kp, vp = _cache_arg(ck.packed, 16, "ck.packed"), _cache_arg(vq.packed, 16, "vq.packed")
    ks, kz, vs, vz = (_cache_arg(t, 4, n) for t, n in ((ck.scale, "ck.scale"), (ck.zero, "ck.zero"),
                                                       (vq.scale, "vq.scale"), (vq.zero, "vq.zero")))
    out = _check_out(out, B, HQ, D, q.device)
    acc, maxs, sums, _ = _workspace_for(_workspace, B, HQ, num_splits + 1, D, q.device, HKV)
    args = _lib.DecodeArgs(
        q=q.data_ptr(), q_is_fp32=int(q.dtype == torch.float32),
        k=kp.data_ptr(), k_scale=ks.data_ptr(), k_zero=kz.data_ptr(),
        v=vp.data_ptr(), v_scale=vs.data_ptr(), v_zero=vz.data_ptr(),
        seq_lens=_lib.ptr(qlens), acc=_lib.ptr(acc), maxs=_lib.ptr(maxs), sums=_lib.ptr(sums),
        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=ck.nbits,
        v_nbits=vq.nbits, group_size=vq.group_size, sm_scale=float(sm_scale),
        split_size=split_size, num_splits=num_splits, counters=None,
        waves=choose_waves(B, HKV, group, split_size, num_splits, D=D, k_nbits=ck.nbits,
                           v_nbits=vq.nbits, group_size=vq.group_size), key_block=BLOCK)
    with torch.cuda.device(q.device):
        rc = _lib.load().tkv_channel_decode_attention(
            args, kr.data_ptr(), vr.data_ptr(), _lib.ptr(rlens), R, _lib.stream_handle(q.device))
    _lib.check(rc, "channel_decode_attention")
    return out


class ChannelKVCache:
    """One layer's cache: per-channel keys, per-token values, fp16 window.

    All batch rows hold the same number of tokens.  ``extend`` appends any
    number of tokens from the host (prefill): whole blocks go straight into the
    history, the rest into the window, which is quantized into the history
    whenever it holds 32 tokens.  ``step`` is one decode step -- append one
    token to the window, attend, quantize the window if it is now full -- with
    the lengths and the flush decision kept on the device, so it allocates no
    host-dependent state and a captured step stays right when its graph is
    replayed for any window fill.  The host-side counters (``quantized``,
    ``window``) follow eager calls only, so under replay only the device
    guards the capacity: a full window that no longer fits the history is not
    flushed and the row is marked (its device-side window length becomes 33);
    from then on that row stores no new token.  :meth:`overflowed` reads the
    marks (a host sync).
    """

    def __init__(self, B: int, HKV: int, capacity: int, D: int, k_nbits: int = 2,
                 v_nbits: int = 2, group_size: int = 32, device="cuda"):
        cap = -(-capacity // BLOCK) * BLOCK
        self.keys = empty_channel_keys(B, HKV, cap, D, k_nbits, device)
        self.values = empty_cache(B, HKV, cap, D, v_nbits, group_size, device)
        for t in (self.keys.packed, self.keys.scale, self.keys.zero, self.values.packed,
                  self.values.scale, self.values.zero):
            t.zero_()
        self.k_res = torch.zeros(B, HKV, BLOCK, D, dtype=torch.float16, device=device)
        self.v_res = torch.zeros_like(self.k_res)
        self.capacity = cap
        self.quantized = 0   # tokens in the quantized history (a multiple of 32)
        self.window = 0      # tokens in the fp16 window (< 32)
        self._pos = torch.zeros(B, dtype=torch.int32, device=device)
        self._qlens = torch.zeros(B, dtype=torch.int32, device=device)
        self._rlens = torch.zeros(B, dtype=torch.int32, device=device)
        self.workspace: dict = {}

    def __len__(self) -> int:
        return self.quantized + self.window

    def reset(self) -> None:
        """Forget every token (host counters and device-side lengths)."""
        self.quantized = self.window = 0
        self._qlens.zero_()
        self._rlens.zero_()

    def nbytes(self) -> int:
        return self.keys.nbytes() + self.values.nbytes() + 2 * self.k_res.numel() * 2

    def overflowed(self) -> bool:
        """Whether any row's window filled up with no room left in the history
        (possible only through replayed steps, which the host does not count);
        such a row has stopped storing tokens.  Synchronises with the device."""
        return bool((self._rlens > BLOCK).any())

    def _check_tokens(self, k: torch.Tensor, v: torch.Tensor, n: int | None = None) -> None:
        B, HKV, _, D = self.k_res.shape
        if not isinstance(k, torch.Tensor) or not isinstance(v, torch.Tensor):
            raise TypeError("k and v must be tensors")
        if k.dim() != 4 or k.shape != v.shape or (k.shape[0], k.shape[1], k.shape[3]) != (B, HKV, D) \
                or (n is not None and k.shape[2] != n):
            want = f"({B}, {HKV}, {'N' if n is None else n}, {D})"
            raise ValueError(f"k / v must be {want} tensors of one shape, got {tuple(k.shape)} "
                             f"and {tuple(v.shape)}")
        if k.device != self.k_res.device or v.device != self.k_res.device:
            raise ValueError(f"k / v must be on the cache's device {self.k_res.device}")

    def _flush(self) -> None:
        self._pos.fill_(self.quantized)
        append_keys_per_channel(self.keys, self.k_res, self._pos)
        append_kv(self.values, self.v_res, self._pos)
        self.quantized += BLOCK
        self.window = 0

    def extend(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append ``(B, HKV, N, D)`` keys and values from the host (prefill)."""
        self._check_tokens(k, v)
        if k.dtype != torch.float16:
            k = k.to(torch.float16)
        if v.dtype != torch.float16:
            v = v.to(torch.float16)
        N = k.shape[2]
        if len(self) + N > self.capacity:
            raise ValueError(f"cache capacity {self.capacity} exceeded ({len(self)} + {N})")
        i = 0
        if self.window == 0 and N >= BLOCK:  # whole blocks straight into the history
            n = (N // BLOCK) * BLOCK
            self._pos.fill_(self.quantized)
            append_keys_per_channel(self.keys, k[:, :, :n], self._pos)
            append_kv(self.values, v[:, :, :n].contiguous(), self._pos)
            self.quantized += n
            i = n
        while i < N:
            take = min(BLOCK - self.window, N - i)
            self.k_res[:, :, self.window:self.window + take] = k[:, :, i:i + take]
            self.v_res[:, :, self.window:self.window + take] = v[:, :, i:i + take]
            self.window += take
            i += take
            if self.window == BLOCK:
                self._flush()
        self._qlens.fill_(self.quantized)
        self._rlens.fill_(self.window)

    def attend(self, q: torch.Tensor, sm_scale: float | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
        """Attention of ``q`` ``(B, HQ, D)`` over everything appended so far.
        Every row holds the same number of tokens, so the split plan is the
        one for equal lengths."""
        return channel_decode_attention(q, self.keys, self.values, self.k_res, self.v_res,
                                        q_lens=self._qlens, res_lens=self._rlens,
                                        sm_scale=sm_scale, out=out, _workspace=self.workspace,
                                        equal_lengths=True)

    def step(self, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
             sm_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """One decode step: append ``k``/``v`` ``(B, HKV, 1, D)`` to the window,
        attend with ``q`` ``(B, HQ, D)``, then quantize the window into the
        history if it is full.  Three kinds of launches (window append,
        attention, window flush), device-side lengths only: graph-capturable."""
        if len(self) + 1 > self.capacity:
            raise ValueError(f"cache capacity {self.capacity} exceeded")
        self._check_tokens(k, v, 1)
        B, HKV, _, D = self.k_res.shape
        kk = k.to(torch.float16).contiguous()
        vv = v.to(torch.float16).contiguous()
        lib, st = _lib.load(), _lib.stream_handle(self.k_res.device)
        with torch.cuda.device(self.k_res.device):
            rc = lib.tkv_channel_window_append(kk.data_ptr(), vv.data_ptr(), B, HKV, D,
                                               self.k_res.data_ptr(), self.v_res.data_ptr(), BLOCK,
                                               self._rlens.data_ptr(), st)
            _lib.check(rc, "ChannelKVCache.step (window append)")
        out = self.attend(q, sm_scale=sm_scale, out=out)
        ks, vs = self.keys, self.values
        with torch.cuda.device(self.k_res.device):
            rc = lib.tkv_channel_window_flush(
                self.k_res.data_ptr(), self.v_res.data_ptr(), B, HKV, D, ks.nbits, vs.nbits,
                vs.group_size, BLOCK, self._qlens.data_ptr(), self._rlens.data_ptr(),
                self.capacity, ks.packed.data_ptr(), ks.scale.data_ptr(), ks.zero.data_ptr(),
                vs.packed.data_ptr(), vs.scale.data_ptr(), vs.zero.data_ptr(), st)
            _lib.check(rc, "ChannelKVCache.step (window flush)")
        self.window += 1
        if self.window == BLOCK:
            self.quantized += BLOCK
            self.window = 0
        return out


__all__ = ["BLOCK", "ChannelQuantizedKeys", "empty_channel_keys", "append_keys_per_channel",
           "quantize_keys_per_channel", "channel_decode_attention", "ChannelKVCache"]
