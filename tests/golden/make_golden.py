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
