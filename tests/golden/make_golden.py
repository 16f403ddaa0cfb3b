"""Write golden vectors for ``quantize_groupwise`` from the reference itself.

Why this script exists: the reference's own tests pin the quantizer only by
round trip and by a half-step error bound (``test_correctness.py:78-134``).
Neither fixes the exact bits at rounding ties after the division, the fp16
rounding of the scale, or the degenerate-range cases.  So the reference's
``quantize.py`` (pure torch, ``quantize.py:186-236``) is imported here, in the
build container only, to write small input/output vectors.  Nothing else of
the reference is imported, and the reference never travels: only the vectors
in ``quantize_golden.npz`` are committed.

Run:  python tests/golden/make_golden.py [/root/reference]
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch


def _cases():
    """(name, x fp32 or fp16 tensor (rows, D), nbits, group_size)."""
    g = torch.Generator().manual_seed(1234)
    out = []
    # 1) random fp16 rows with 1% x8 outliers (the reference's input model)
    for nbits in (2, 4):
        for gs in (16, 32, 64, 128):
            x = torch.randn(8, 128, generator=g)
            m = torch.rand(8, 128, generator=g) < 0.01
            x = torch.where(m, x * 8, x).half()
            out.append((f"rand_f16_b{nbits}_g{gs}", x, nbits, gs))
    # 2) fp32 rows (the reference's CPU tests quantize fp32 tensors)
    for nbits in (2, 4):
        out.append((f"rand_f32_b{nbits}_g32", torch.randn(6, 128, generator=g), nbits, 32))
    # 3) exact .5 ties after the division: min 0, max 2*qmax -> scale 2
    for nbits in (2, 4):
        qmax = (1 << nbits) - 1
        row = torch.arange(0, 2 * qmax + 1, dtype=torch.float32)
        row = torch.cat([row, torch.full((32 - row.numel(),), float(qmax))])
        row[1] = 2 * qmax  # keep max at 2*qmax
        x = row.repeat(4)[None, :128].clone()
        out.append((f"ties_b{nbits}", x.half(), nbits, 32))
    # 4) scale not representable in fp16 (rounded before the codes are made)
    x = torch.linspace(-1.0, 1.3333, 128)[None].half()
    out.append(("scale_round_b4", x, 4, 32))
    out.append(("scale_round_b2", x, 2, 32))
    # 5) constant groups (scale -> 1, codes 0), incl. zeros and -0.0
    x = torch.tensor([[3.5] * 32 + [0.0] * 32 + [-0.0] * 32 + [-7.25] * 32]).half()
    out.append(("constant_b4", x, 4, 32))
    out.append(("constant_b2", x, 2, 32))
    # 6) extreme range: +-65504
    x = torch.randn(2, 128, generator=g).half()
    x[0, 0], x[0, 1], x[1, 64], x[1, 100] = 65504.0, -65504.0, 65504.0, -65504.0
    out.append(("extreme_b4", x, 4, 32))
    out.append(("extreme_b2", x, 2, 64))
    # 7) fp16 subnormal inputs and a range whose fp16 scale underflows to 0
    sub = torch.tensor([2.0 ** -24, 0.0, 2.0 ** -20, 2.0 ** -15, -2.0 ** -24] * 7)[:32]
    tiny = torch.tensor([0.0, 2.0 ** -24] * 16)
    x = torch.cat([sub, tiny, sub * 1024, torch.randn(32, generator=g)])[None].half()
    out.append(("subnormal_b4", x, 4, 32))
    out.append(("subnormal_b2", x, 2, 32))
    return out + _nonfinite_cases()


def _nonfinite_cases():
    """NaN, +-Inf and fp32-beyond-fp16 input, at nbits 2/4 and gs 32/128.

    These pin how the reference's ``amin``/``amax`` propagate a NaN (the group
    gets the canonical fp16 NaN zero, scale 1, codes 0), how an infinite range
    becomes an infinite scale, and how a range or minimum past 65504 rounds to
    an infinite fp16 scale or zero.  A generator of their own keeps the earlier
    cases' vectors unchanged.
    """
    g = torch.Generator().manual_seed(4321)
    nan, inf = float("nan"), float("inf")
    out = []
    for nbits in (2, 4):
        for gs in (32, 128):
            tag = f"b{nbits}_g{gs}"
            # one NaN per row, at different dims; a negative NaN bit pattern;
            # the last row stays finite
            x = torch.randn(4, 128, generator=g).half()
            x[0, 5] = nan
            x[1, 127] = nan
            x.view(torch.int16)[2, 40] = -512  # 0xFE00: NaN with the sign bit
            out.append((f"nan_one_{tag}", x, nbits, gs))
            # a whole group of NaN, and a whole row
            x = torch.randn(3, 128, generator=g).half()
            x[0, :gs] = nan
            x[1, :] = nan
            x[2, 64:64 + gs // 2] = nan
            out.append((f"nan_all_{tag}", x, nbits, gs))
            # +Inf, -Inf, both in one group, Inf beside NaN, a group of +Inf
            x = torch.randn(5, 128, generator=g).half()
            x[0, 3] = inf
            x[1, 70] = -inf
            x[2, 10], x[2, 11] = inf, -inf
            x[3, 0], x[3, 1] = inf, nan
            x[4, 96:] = inf
            out.append((f"inf_{tag}", x, nbits, gs))
            # fp32 input beyond fp16's range: an overflowing scale, an
            # overflowing zero (-inf) with a finite scale, a zero of +inf,
            # the rounding edge at 65520, and an fp32 NaN with a payload
            x = torch.randn(6, 128, generator=g)
            x[0, 7] = 1.0e6
            x[1, :] = -7.0e4 + torch.rand(128, generator=g)
            x[2, :] = 1.0e5 + torch.rand(128, generator=g)
            x[3, :] = 65519.0
            x[3, 1] = 65520.0
            x[4, :] = -65520.0
            x[4, 2] = -65519.0
            x.view(torch.int32)[5, 9] = 0x7FC12345
            out.append((f"f32_range_{tag}", x, nbits, gs))
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import quantize as ref_quantize  # the reference's quantize.py

    arrays = {}
    names = []
    for name, x, nbits, gs in _cases():
        qt = ref_quantize.quantize_groupwise(x, nbits, gs)
        names.append(name)
        arrays[f"{name}__x"] = x.float().numpy() if x.dtype == torch.float32 else x.numpy()
        arrays[f"{name}__meta"] = np.array([nbits, gs], dtype=np.int64)
        arrays[f"{name}__packed"] = qt.packed.numpy()
        arrays[f"{name}__scale"] = qt.scale.numpy()
        arrays[f"{name}__zero"] = qt.zero.numpy()
        deq = ref_quantize.dequantize_groupwise(qt, torch.float32)
        arrays[f"{name}__deq"] = deq.numpy()
    arrays["names"] = np.array(names)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quantize_golden.npz")
    np.savez_compressed(dst, **arrays)
    print(f"wrote {len(names)} cases to {dst} (torch {torch.__version__})")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
