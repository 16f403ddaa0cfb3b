"""Shared helpers of the test suite (thresholds, metrics, case builders).

The thresholds are the reference's (``test_correctness.py:50-56``) plus the
north-star tolerance of this build: attention output within 2e-3 max-abs and
1e-3 mean-abs of the fp32 dequantise-then-attend reference.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention as oatt
from oracle import inputs as oinp
from oracle import quant as oq

# Fused kernel vs float32 dequant-then-attend on identical dequantized values.
KERNEL_COSINE_MIN = 0.99999
KERNEL_REL_L2_MAX = 5e-3
# How much worse than the fp16 dequant baseline the kernel may be vs the fp16 truth.
KERNEL_VS_BASELINE_ERR_RATIO_MAX = 1.5
# max-abs / mean-abs vs the fp32 reference.
MAX_ABS_TOL = 2e-3
MEAN_ABS_TOL = 1e-3


def same_float_bits(a, b) -> bool:
    """Bit-for-bit equal float arrays, where a NaN matches any NaN in the same place.

    A NaN's sign and payload are not a value: the reference's dequant computes
    ``0 * inf`` on the host CPU, which returns x86's default NaN (sign bit set),
    while the GPU returns the positive canonical one.
    """
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    ui = {2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize]
    return bool(np.array_equal(a[~na].view(ui), b[~nb].view(ui)))


def metrics(got, ref) -> dict:
    if isinstance(got, torch.Tensor):
        got = got.detach().float().cpu().numpy()
    if isinstance(ref, torch.Tensor):
        ref = ref.detach().float().cpu().numpy()
    return oatt.metrics(got, ref)


def assert_close_to_reference(got, ref, what: str) -> dict:
    m = metrics(got, ref)
    assert m["cosine"] >= KERNEL_COSINE_MIN, f"{what}: {m}"
    assert m["rel_l2"] <= KERNEL_REL_L2_MAX, f"{what}: {m}"
    assert m["max_abs_err"] <= MAX_ABS_TOL, f"{what}: {m}"
    assert m["mean_abs_err"] <= MEAN_ABS_TOL, f"{what}: {m}"
    return m


def qt_to_np(qt) -> oq.QuantNP:
    """Pull a device QuantizedTensor back as the oracle's numpy container."""
    return oq.QuantNP(qt.packed.cpu().numpy(), qt.scale.cpu().numpy(), qt.zero.cpu().numpy(),
                      qt.nbits, qt.group_size, qt.head_dim)


def oracle_attention_on_quant(q, kq, vq, sm_scale=None, seq_lens=None, chunk=8192):
    """fp32 dequantise-then-attend of device caches, computed by the oracle on the host."""
    kn, vn = qt_to_np(kq), qt_to_np(vq)
    qn = q.detach().float().cpu().numpy()
    B, HKV, S, _ = kn.packed.shape

    def rows(qnp):
        def f(s, e):
            part = oq.QuantNP(qnp.packed[:, :, s:e], qnp.scale[:, :, s:e], qnp.zero[:, :, s:e],
                              qnp.nbits, qnp.group_size, qnp.head_dim)
            return oq.dequantize_groupwise(part)
        return f

    lens = None if seq_lens is None else np.asarray(seq_lens)
    return oatt.reference_grouped(qn, rows(kn), rows(vn), S, HKV, sm_scale=sm_scale,
                                  chunk=chunk, seq_lens=lens)


def make_case(B, HQ, HKV, D, S, nbits, group_size, seed, device="cuda", outlier_frac=0.01):
    """The reference's _run_case inputs (test_correctness.py:150-160), quantized on the GPU."""
    from tritonkv_amd.quantize import quantize_kv

    q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=seed, outlier_frac=outlier_frac)
    q, k, v = q.to(device), k.to(device), v.to(device)
    kq, vq = quantize_kv(k, v, nbits, group_size)
    return q, k, v, kq, vq


def fp16_baseline_rows(qnp):
    """The reference baseline's fp16 dequant (reference.py:96-108): c*s then +z, each rounded to fp16."""
    return oq.dequantize_fp16(qnp)
