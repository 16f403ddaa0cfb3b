"""Fused dequantize + decode attention on MI355X (gfx950 HIP kernels).

Drop-in for the reference's ``kernels/fused_decode_attn.py``: same public names
(``fused_decode_attention`` :419-570, ``pick_num_splits`` :402-416,
``triton_available`` :81-86), same arguments, defaults, validation order of
checks, split arithmetic, workspace keys and return value.  The two Triton
launches (split :525-556, combine :558-568) are replaced by one call into the
C ABI ``tkv_fused_decode_attention`` (``include/tkv.h``), which enqueues the
gfx950 split kernel and, for more than one split, the combine kernel on
torch's current stream.  Nothing is allocated inside the call once ``out`` and
``_workspace`` are supplied, so it can be captured in a HIP graph.

Differences a caller can observe, all deliberate:

* Argument errors are raised *before* the backend check, so they are testable
  on a host without a GPU (the reference checks the backend first, :461-463).
* ``num_warps`` / ``num_stages`` are Triton tuning knobs: accepted and ignored.
  ``meta_bcast`` and ``dequant_fp16`` selected between bitwise-identical
  Triton variants (``test_correctness.py:292-343``); here both values run the
  same kernel, so the outputs are trivially ``torch.equal``.
* ``fold_zp``: the HIP kernel always computes scores in the folded form
  ``sum_g s_g (q_g . c_g) + z_g sum(q_g)`` (the reference's FOLD_ZP algebra,
  :229-272) -- it is the form that lets the matrix cores consume raw codes.
  The ``gs >= 16`` check of ``fold_zp=True`` is kept.
* When ``num_splits`` is None the split count is chosen for 256 compute units
  (see :func:`default_num_splits`); an explicit ``num_splits`` is honoured
  exactly as in the reference (clamp to ``n_blocks``, then tighten).
* ``allow_mixed_bits=True`` (new, keyword-only) lets K and V use different bit
  widths (e.g. 4-bit K, 2-bit V); without it the reference's ValueError is
  raised.  ``seq_lens`` (new) gives one context length per batch row.
  ``fused_combine=True`` (new) merges split partials inside the split kernel
  (last workgroup per unit) instead of a second launch; it is correct but
  measured slower on MI355X (every workgroup's agent-scope release writes back
  its L2), so it is off by default.
* ``k_new`` / ``v_new`` (new, keyword-only): the decode-step append fused into
  the same launch -- see :func:`new_token_args`.
* ``equal_lengths`` (new, keyword-only): the caller promises that every entry
  of ``seq_lens`` is the same.  The split plan is then the one of a call
  without ``seq_lens`` -- no cut of long histories into pieces, no dispatch
  order -- while the kernel still stops each row at its length.  The promise
  only steers the plan: a batch that breaks it still gets the right answer,
  only less evenly spread over the compute units.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from ..quantize import QuantizedTensor

LOG2E = 1.4426950408889634



def triton_available() -> tuple[bool, str]:
    """``(ok, why)`` for the HIP backend (the reference's name is kept for callers)."""
    err = _lib.load_error()
    if err is not None:
        return False, err
    if not torch.cuda.is_available():
        return False, "torch.cuda.is_available() is False"
    return True, f"tritonkv_amd HIP backend (abi {_lib.load().tkv_abi_version()})"


hip_available = triton_available


def _next_pow2(x: int) -> int:
    return 1 << (x - 1).bit_length()


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


_CU_COUNT: dict = {}


def compute_units(device=None) -> int | None:
    try:
        dev = torch.cuda.current_device() if device is None else torch.device(device).index or 0
        if dev not in _CU_COUNT:
            _CU_COUNT[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
        return _CU_COUNT[dev]
    except Exception:
        return None


def pick_num_splits(B: int, HKV: int, n_blocks: int, target_programs: int | None = None) -> int:
    """The reference's heuristic (:402-416): ``target // (B*HKV)`` clamped to ``[1, n_blocks]``.

    ``target_programs`` defaults to 4 programs per compute unit (1024 on a
    256-CU MI355X), or 128 without a device.
    """
    if target_programs is None:
        cu = compute_units()
        target_programs = cu * 4 if cu else 128
    want = max(1, target_programs // max(1, B * HKV))
    return max(1, min(n_blocks, want))


# Tokens one workgroup of a split history should stream (see default_num_splits).
TOKENS_PER_WORKGROUP = 512      # fused 2/4-bit kernel
TOKENS_PER_WORKGROUP_FP16 = 256  # fp16 control: 3-6x the bytes per token


MAX_SPLITS = 65535  # grid y-dimension limit


def default_num_splits(B: int, HKV: int, G: int, S: int, block_n: int,
                       tokens_per_workgroup: int = TOKENS_PER_WORKGROUP, *,
                       ragged: bool = False) -> int:
    """Split count used when the caller passes ``num_splits=None``.

    Chosen from sweeps on MI355X (split count x workgroup size, DRAM-resident
    caches, batch 1..64, 2..8 KV heads, ctx 2048..32768):

    * a batch that already offers one (b, kv head, 16-head block) unit per
      compute unit or more runs unsplit -- no partials, no combine launch --
      and so does a history of at most ``tokens_per_workgroup`` tokens (512
      for the fused kernel, 256 for the fp16 control, whose tokens are 3-6x
      larger);
    * otherwise the history is cut so that each workgroup streams about
      ``tokens_per_workgroup`` tokens, with at least 32 and at most one
      workgroup per compute unit in total, and no split shorter than a
      quarter of that (128 / 64 tokens).  Fewer, longer workgroups win at
      small caches (the Qwen2.5-1.5B shape, fused: 64 workgroups at ctx
      16384); one per CU wins as soon as the cache is tens of MB (e.g. 3x
      over a fixed 64 at B=16, ctx 32768).  Even a short history gains from
      the split: a workgroup's 8 waves take about 1 us of compute per two
      chunks each, more than the combine launch costs (Qwen2.5-1.5B shape,
      ctx 1024: 7.3 us at 8 splits vs 9.6 unsplit; fp16 control at ctx 512:
      6.6 us at 8 splits vs 7.9 unsplit).

    With per-row lengths (``ragged``: the call passes ``seq_lens``, which the
    host cannot read without a sync), a batch of at least one unit per compute
    unit and a history of at least 16384 tokens is cut into pieces of at most
    32768 tokens, and at least two: rows of very different lengths make one
    workgroup per unit finish unevenly, and shorter pieces even that out.
    B=64, HKV=8, lengths U[1k, 128k], K4/V2, in grid order: 823 us unsplit,
    746 us at 2 splits, 733 us at 4 (a split past a row's end leaves at
    once), 743 us at 8; run longest piece first (``_order_for``), 672, 683,
    699 and 715 us.  The cap stays because the host cannot see the lengths:
    a few full-length rows among many short ones would each sit on one CU
    unsplit.  Equal lengths pay for the second split (Llama-3-8B shape:
    206.6 vs 200.7 us).

    Returned in units of ``block_n`` blocks so the reference's tightening
    applies unchanged.
    """
    cu = compute_units() or 256
    units = B * HKV * _cdiv(G, 16)
    if S <= tokens_per_workgroup:
        return 1
    if units >= cu:
        if not ragged or S < 16384:
            return 1
        return min(max(2, S // 32768), _cdiv(S, block_n))
    workgroups = min(cu, max(32, units * S // tokens_per_workgroup))
    want = max(1, workgroups // units)
    max_splits = max(1, S // max(tokens_per_workgroup // 4, block_n))
    return max(1, min(want, max_splits, _cdiv(S, block_n)))


# Workgroups that stream at least this many tokens run 12 waves where the
# library has a 12-wave kernel (twelve_wave_format).
TWELVE_WAVES_MIN_SPLIT = 8192


def twelve_wave_format(D: int, G: int, k_nbits: int, v_nbits: int, group_size: int,
                       paged: bool = False) -> bool:
    """Whether the library has a 12-wave split kernel for this format (the list
    in ``csrc/quant_split.h``, ``kTwelveWaves``): head_dim 128, contiguous
    caches, and 2-bit K/V with groups of 32 at GQA groups of at most 4 query
    heads (per-token or per-channel keys), or groups of 128 with equal K/V bits.
    These kernels are bound by instruction issue, and a third wave per SIMD
    gives it more to interleave (Llama-3-8B shape: 3-7% faster); a request of
    12 waves for any other kernel runs 8."""
    if D != 128 or paged:
        return False
    return (k_nbits == 2 and v_nbits == 2 and group_size == 32 and G <= 4) or \
        (k_nbits == v_nbits and k_nbits in (2, 4) and group_size == 128)


def choose_waves(B: int, HKV: int, G: int, split_size: int, num_splits: int = 0, *,
                 D: int = 128, k_nbits: int = 16, v_nbits: int = 16, group_size: int = 0,
                 paged: bool = False) -> int:
    """Waves per workgroup: 12 for the formats of ``twelve_wave_format`` when a
    workgroup streams at least ``TWELVE_WAVES_MIN_SPLIT`` tokens; else 8 when
    it streams the whole history or at least 512 tokens (two 32-token chunks
    per wave, so each wave overlaps a load with compute); else 4.  The default
    format (16-bit) is the fp16 control's."""
    if split_size >= TWELVE_WAVES_MIN_SPLIT and \
            twelve_wave_format(D, G, k_nbits, v_nbits, group_size, paged):
        return 12
    return 8 if num_splits == 1 or split_size >= 512 else 4


def plan_splits(S: int, block_n: int, num_splits: int | None, B: int, HKV: int, G: int,
                tokens_per_workgroup: int = TOKENS_PER_WORKGROUP, *, ragged: bool = False):
    """Reference split arithmetic (:486-499) -> (block_n, num_splits, split_size).

    One addition: the count is capped at 65535 before tightening (splits are
    the launch grid's y axis), which the reference's shapes never reach."""
    block_n = min(block_n, max(16, _next_pow2(S)))
    n_blocks = _cdiv(S, block_n)
    if num_splits is None:
        num_splits = default_num_splits(B, HKV, G, S, block_n, tokens_per_workgroup,
                                        ragged=ragged)
    num_splits = max(1, min(num_splits, n_blocks, MAX_SPLITS))
    blocks_per_split = _cdiv(n_blocks, num_splits)
    num_splits = _cdiv(n_blocks, blocks_per_split)  # tighten: no empty splits
    return block_n, num_splits, blocks_per_split * block_n


def _workspace_for(ws: dict | None, B: int, HQ: int, num_splits: int, D: int, device,
                   HKV: int = 1):
    """Partials buffers, reused under the reference's keys (:505-521).

    Returns ``(acc, maxs, sums, counters)``.  ``counters`` holds one int32
    ticket per (batch row, kv head, block of 16 query heads); it is zeroed once
    when allocated and the kernels leave it zero, so the split kernel can merge
    its own partials (no combine launch) and the call stays graph-capturable.
    """
    ws = ws if ws is not None else {}
    if num_splits == 1:
        acc = ws.get("dummy_acc")
        if acc is None:
            acc = torch.empty((1, 1, 1, 1), device=device, dtype=torch.float32)
            ws["dummy_acc"] = acc
        return None, None, None, None
    key = (B, HQ, num_splits, D)
    if ws.get("key") != key or ws["acc"].device != torch.device(device):
        acc = torch.empty((B, HQ, num_splits, D), device=device, dtype=torch.float32)
        maxs = torch.empty((B, HQ, num_splits), device=device, dtype=torch.float32)
        sums = torch.empty((B, HQ, num_splits), device=device, dtype=torch.float32)
        ws.update(key=key, acc=acc, maxs=maxs, sums=sums)
    n_counters = B * HKV * _cdiv(HQ // HKV, 16)
    cnt = ws.get("counters")
    if cnt is None or cnt.numel() < n_counters or cnt.device != torch.device(device):
        cnt = torch.zeros(n_counters, device=device, dtype=torch.int32)
        ws["counters"] = cnt
    return ws["acc"], ws["maxs"], ws["sums"], cnt


# The order kernel ranks each piece against every row (O(B) per piece, so
# O(B^2 * num_splits) in all); the automatic order stops at this many rows.
ORDER_MAX_ROWS = 2048


def _order_for(ws: dict | None, B: int, HKV: int, num_splits: int, device, seq_lens,
               dispatch_order: bool | None, G: int = 1, D: int = 128):
    """The ``work_order`` buffer of a split call, or None.

    ``dispatch_order=None`` takes it when ``seq_lens`` is given, the batch
    has at most ``ORDER_MAX_ROWS`` rows and the grid holds more workgroups
    than the GPU has compute units: the call then runs the split workgroups
    longest piece first (``ragged_order_kernel``), which evens out the end of
    the launch when rows differ in length (B=64, HKV=8, lengths U[1k, 128k],
    K4/V2: decode 711-720 -> 669-671 us).  A grid that fits the CUs at once
    has no tail to even out, and the order would only add its launch
    boundary (4.7-7.7 us measured ahead of the split kernel).  The output is
    bit-identical either way; ``True`` forces the order, ``False`` keeps the
    grid order.  Ordered kernels exist for head dim 128 only: elsewhere the
    automatic order is off, and a forced one is refused (ValueError).
    """
    if dispatch_order is False:
        return None
    if dispatch_order is None:
        workgroups = B * HKV * _cdiv(G, 16) * num_splits
        if seq_lens is None or workgroups <= (compute_units(device) or 256) \
                or B > ORDER_MAX_ROWS or D != 128:
            return None
    ws = ws if ws is not None else {}
    n = 2 * B * HKV * num_splits  # (s * B * HKV + unit, row length) pairs
    buf = ws.get("work_order")
    if buf is None or buf.numel() < n or buf.device != torch.device(device):
        buf = torch.empty(n, device=device, dtype=torch.int32)
        ws["work_order"] = buf
    return buf


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """q (a few KB) as the kernels load it: contiguous and 16-byte aligned,
    copied if it is not."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _cache_arg(t: torch.Tensor, align: int, name: str, written: bool = False) -> torch.Tensor:
    """A cache tensor as the kernels take it.  A non-contiguous cache that is
    only read is made contiguous, as the reference does (``:489-491``; that is
    a copy of the cache); one the step writes into (the fused append) must be
    contiguous already, or the token would land in a temporary copy.  Caches
    are never realigned: codes and fp16 rows need 16-byte, scale/zero 4-byte
    aligned storage, which every contiguous allocation has."""
    if not t.is_contiguous():
        if written:
            raise ValueError(f"{name} must be contiguous: the step writes the new token into it")
        t = t.contiguous()
    if t.data_ptr() % align:
        raise ValueError(f"{name} must start on a {align}-byte boundary "
                         f"(data_ptr % {align} = {t.data_ptr() % align})")
    return t


def _check_out(out, B, HQ, D, device):
    if out is None:
        return torch.empty((B, HQ, D), device=device, dtype=torch.float32)
    if out.shape != (B, HQ, D) or out.dtype != torch.float32 or not out.is_contiguous() \
            or out.device != torch.device(device):
        raise ValueError(f"out must be a contiguous float32 ({B}, {HQ}, {D}) tensor on {device}")
    return out


def _seq_lens_arg(seq_lens, B, S, device):
    if seq_lens is None:
        return None
    if not isinstance(seq_lens, torch.Tensor) or seq_lens.dtype != torch.int32 \
            or seq_lens.numel() != B or seq_lens.device != device:
        raise ValueError("seq_lens must be an int32 tensor of B lengths on the cache's device")
    return seq_lens.contiguous()


def new_token_args(k_new, v_new, B: int, HKV: int, D: int, device):
    """Validated ``(k_new, v_new, is_fp32)`` for the fused append, or Nones.

    ``k_new`` / ``v_new``: ``(B, HKV, D)`` or ``(B, HKV, 1, D)``, both fp16 or
    both fp32.  The token goes to position ``L_b - 1`` of row b, where ``L_b``
    is ``seq_lens[b]`` (or the cache capacity), and is quantized into the
    caches in place exactly as :func:`~tritonkv_amd.quantize.append_kv` at
    ``positions = L - 1`` would; attention then covers ``[0, L_b)``.
    """
    if k_new is None and v_new is None:
        return None, None, 0
    if k_new is None or v_new is None:
        raise ValueError("k_new and v_new must be given together")
    out = []
    for name, x in (("k_new", k_new), ("v_new", v_new)):
        if x.dim() == 4 and x.shape[2] == 1:
            x = x[:, :, 0]
        if tuple(x.shape) != (B, HKV, D):
            raise ValueError(f"{name} must have shape ({B}, {HKV}, {D}) or ({B}, {HKV}, 1, {D}), "
                             f"got {tuple(x.shape)}")
        if x.dtype not in (torch.float16, torch.float32):
            raise TypeError(f"{name} must be float16 or float32, got {x.dtype}")
        if x.device != torch.device(device):
            raise ValueError(f"{name} must be on the cache's device")
        out.append(x.contiguous())
    if out[0].dtype != out[1].dtype:
        raise TypeError("k_new and v_new must have the same dtype")
    return out[0], out[1], int(out[0].dtype == torch.float32)


def _tensor_key(t):
    """What the argument checks and the argument block depend on for a tensor
    the call reads in place: its storage, shape, dtype and layout."""
    return None if t is None else (t.data_ptr(), t.shape, t.dtype, t.is_contiguous())


def _new_key(t):
    """The same for the new token's rows, whose storage may change every step."""
    return None if t is None else (t.shape, t.dtype, t.is_contiguous())


class _PreparedCall:
    """The validated argument block of a decode call, kept in the caller's
    ``_workspace`` under ``"call"``.  A later call whose key matches (same
    caches, buffers, shapes and flags; q and the new token's rows may be new
    tensors of the same shape) reuses it: only those pointers are refreshed.
    This takes validation, the split plan and the construction of the ctypes
    argument block (most of the ~16-20 us an eager call spent on the host)
    off every step of a decode loop."""

    __slots__ = ("key", "args", "entry", "what", "out_shape", "device", "new")

    def __init__(self, key, args, entry, what, out_shape, device, new):
        self.key, self.args, self.entry, self.what = key, args, entry, what
        self.out_shape, self.device, self.new = out_shape, device, new

    def run(self, q, out, k_new=None, v_new=None):
        """Launch with this q (and new token); None when q does not qualify
        (misaligned), so that the caller takes the full path."""
        qp = q.data_ptr()
        if qp % 16:
            return None
        a = self.args
        a.q = qp
        if self.new:
            a.k_new, a.v_new = k_new.data_ptr(), v_new.data_ptr()
        if out is None:
            out = torch.empty(self.out_shape, device=self.device, dtype=torch.float32)
            a.out = out.data_ptr()
        if self.device.index == torch.cuda.current_device():
            rc = self.entry(a, torch.cuda.current_stream().cuda_stream)
        else:
            with torch.cuda.device(self.device):
                rc = self.entry(a, torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, self.what)
        return out


def _prepared(ws, key):
    """The workspace's prepared call if its key matches, else None."""
    if ws is None:
        return None
    prep = ws.get("call")
    return prep if prep is not None and prep.key == key else None


def fused_decode_attention(
    q: torch.Tensor,
    kq: QuantizedTensor,
    vq: QuantizedTensor,
    sm_scale: float | None = None,
    block_n: int = 64,
    num_warps: int = 4,
    num_stages: int = 2,
    num_splits: int | None = None,
    meta_bcast: bool = True,
    fold_zp: bool = False,
    dequant_fp16: bool = False,
    out: torch.Tensor | None = None,
    _workspace: dict | None = None,
    *,
    seq_lens: torch.Tensor | None = None,
    allow_mixed_bits: bool = False,
    fused_combine: bool = False,
    k_new: torch.Tensor | None = None,
    v_new: torch.Tensor | None = None,
    dispatch_order: bool | None = None,
    equal_lengths: bool = False,
) -> torch.Tensor:
    """Single decode step of attention, computed directly on packed low-bit K/V.

    q: ``(B, HQ, D)`` fp16 or fp32 (rounded to fp16 in the kernel, as the
    reference does); kq, vq: quantized caches with ``packed`` of shape
    ``(B, HKV, S, D//P)``.  Returns ``(B, HQ, D)`` float32.
    ``dispatch_order`` (new): longest-piece-first order of the split
    workgroups (``_order_for``); the result does not depend on it.
    ``equal_lengths`` (new): every row of ``seq_lens`` holds the same length,
    so the split plan of a batch without ``seq_lens`` applies.
    With ``_workspace``, a call like the previous one on the same workspace
    reuses its checked argument block (``_PreparedCall``).
    """
    key = None
    if _workspace is not None:
        key = ("fused", q.shape, q.dtype, q.device, q.is_contiguous(),
               _tensor_key(kq.packed), _tensor_key(kq.scale), _tensor_key(kq.zero),
               _tensor_key(vq.packed), _tensor_key(vq.scale), _tensor_key(vq.zero),
               kq.nbits, vq.nbits, kq.group_size, vq.group_size, kq.head_dim, vq.head_dim,
               sm_scale, block_n, num_splits, fold_zp, _tensor_key(out), _tensor_key(seq_lens),
               allow_mixed_bits, fused_combine, _new_key(k_new), _new_key(v_new),
               dispatch_order, equal_lengths)
        prep = _prepared(_workspace, key)
        if prep is not None:
            res = prep.run(q, out, k_new, v_new)
            if res is not None:
                return res
    if kq.group_size != vq.group_size or (kq.nbits != vq.nbits and not allow_mixed_bits):
        raise ValueError("K and V must use the same nbits/group_size")

    B, HQ, D = q.shape
    Bk, HKV, S, DPk = kq.packed.shape
    if (B, D) != (Bk, kq.head_dim):
        raise ValueError(f"q shape {tuple(q.shape)} incompatible with cache {tuple(kq.packed.shape)}")
    if vq.packed.shape[:3] != kq.packed.shape[:3] or vq.head_dim != kq.head_dim \
            or (vq.nbits == kq.nbits and vq.packed.shape != kq.packed.shape):
        raise ValueError("K and V caches must have the same shape")
    if HQ % HKV != 0:
        raise ValueError(f"HQ={HQ} must be a multiple of HKV={HKV}")
    if D & (D - 1):
        raise ValueError(f"head_dim must be a power of two, got {D}")
    if D % kq.group_size:
        raise ValueError(f"head_dim {D} must be a multiple of group_size {kq.group_size}")
    if fold_zp and kq.group_size < 16:
        raise ValueError(f"fold_zp needs group_size >= 16, got {kq.group_size}")
    if kq.packed.device != q.device or vq.packed.device != q.device:
        raise ValueError("q and the K/V caches must be on the same device")
    kn, vn, new_f32 = new_token_args(k_new, v_new, B, HKV, D, q.device)
    w = kn is not None
    kp, vp = (_cache_arg(t.packed, 16, f"{n}.packed", w) for t, n in ((kq, "kq"), (vq, "vq")))
    ks, kz, vs, vz = (_cache_arg(t, 4, n, w) for t, n in ((kq.scale, "kq.scale"),
                                                          (kq.zero, "kq.zero"),
                                                          (vq.scale, "vq.scale"),
                                                          (vq.zero, "vq.zero")))

    ok, why = triton_available()
    if not ok:
        raise RuntimeError(f"fused_decode_attention requires the tritonkv_amd HIP backend: {why}")

    group = HQ // HKV
    sm_scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    ragged = seq_lens is not None and not equal_lengths
    _, num_splits, split_size = plan_splits(S, block_n, num_splits, B, HKV, group, ragged=ragged)

    q_in = q
    if q.dtype not in (torch.float16, torch.float32):
        q = q.float()
    q = _aligned16(q)
    out = _check_out(out, B, HQ, D, q.device)
    acc, maxs, sums, counters = _workspace_for(_workspace, B, HQ, num_splits, D, q.device, HKV)
    lens = _seq_lens_arg(seq_lens, B, S, q.device)
    order = _order_for(_workspace, B, HKV, num_splits, q.device, seq_lens if ragged else None,
                       dispatch_order, group, D)

    args = _lib.DecodeArgs(
        q=q.data_ptr(), q_is_fp32=int(q.dtype == torch.float32),
        k=kp.data_ptr(), k_scale=ks.data_ptr(), k_zero=kz.data_ptr(),
        v=vp.data_ptr(), v_scale=vs.data_ptr(), v_zero=vz.data_ptr(),
        seq_lens=_lib.ptr(lens), acc=_lib.ptr(acc), maxs=_lib.ptr(maxs), sums=_lib.ptr(sums),
        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D,
        k_nbits=kq.nbits, v_nbits=vq.nbits, group_size=kq.group_size,
        sm_scale=float(sm_scale), split_size=split_size, num_splits=num_splits,
        counters=_lib.ptr(counters) if fused_combine else None,
        waves=choose_waves(B, HKV, group, split_size, num_splits, D=D, k_nbits=kq.nbits,
                           v_nbits=vq.nbits, group_size=kq.group_size),
        k_new=_lib.ptr(kn), v_new=_lib.ptr(vn), new_is_fp32=new_f32,
        work_order=_lib.ptr(order))
    with torch.cuda.device(q.device):
        rc = _lib.load().tkv_fused_decode_attention(args, _lib.stream_handle(q.device))
    _lib.check(rc, "fused_decode_attention")
    # q is kept as given unless it had to be converted or realigned (then no reuse)
    if key is not None and q is q_in and kp is kq.packed and vp is vq.packed and \
            ks is kq.scale and kz is kq.zero and vs is vq.scale and vz is vq.zero:
        _workspace["call"] = _PreparedCall(key, args, _lib.load().tkv_fused_decode_attention,
                                           "fused_decode_attention", (B, HQ, D), q.device,
                                           kn is not None)
    return out

