"""GPU parity of the quantize / pack / unpack / dequant kernels -- bit-exact.

Compared with the oracle (itself pinned by ``tests/test_oracle.py``) and with
the golden vectors written from the reference's ``quantize_groupwise``.  The
unpack/dequant export runs through both register unpack paths of the decode
kernel (K operand, transposed V operand), so these tests also prove that the
decode kernel sees exactly the reference's codes and ``code*scale + zero``.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import inputs as oinp
from oracle import quant as oq
from tests.helpers import same_float_bits

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quantize_golden.npz")
DEV = "cuda"


def _bits16(t):
    return t.detach().cpu().numpy().view(np.uint16)


def _golden_names():
    return [str(n) for n in np.load(GOLDEN)["names"]]


@pytest.mark.parametrize("name", _golden_names())
def test_gpu_quantize_matches_reference_golden(name):
    from tritonkv_amd.quantize import dequantize_groupwise, quantize_groupwise

    z = np.load(GOLDEN)
    x = torch.from_numpy(z[f"{name}__x"]).to(DEV)
    nbits, gs = (int(v) for v in z[f"{name}__meta"])
    print(f"golden case {name} nbits={nbits} gs={gs} dtype={x.dtype}", flush=True)
    qt = quantize_groupwise(x, nbits, gs)
    assert np.array_equal(qt.packed.cpu().numpy(), z[f"{name}__packed"])
    assert np.array_equal(_bits16(qt.scale), z[f"{name}__scale"].view(np.uint16))
    assert np.array_equal(_bits16(qt.zero), z[f"{name}__zero"].view(np.uint16))
    deq = dequantize_groupwise(qt).cpu().numpy()
    assert same_float_bits(deq, z[f"{name}__deq"])


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("gs", [16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gpu_quantize_matches_oracle_bitwise(D, nbits, gs, dtype):
    if gs > D:
        pytest.skip("group larger than head_dim")
    from tritonkv_amd.quantize import quantize_groupwise

    print(f"quantize D={D} nbits={nbits} gs={gs} {dtype}", flush=True)
    _, k, _ = oinp.make_random_kv(2, 4, 2, 257, D, seed=D + nbits + gs, dtype=dtype)
    qt = quantize_groupwise(k.to(DEV), nbits, gs)
    ref = oq.quantize_groupwise(k.numpy(), nbits, gs)
    assert np.array_equal(qt.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_bits16(qt.scale), ref.scale.view(np.uint16))
    assert np.array_equal(_bits16(qt.zero), ref.zero.view(np.uint16))


@pytest.mark.parametrize("nbits,gs,D,dtype", [(4, 32, 128, torch.float16),
                                              (2, 16, 64, torch.float32)])
def test_gpu_bulk_quantize_matches_oracle_bitwise(nbits, gs, D, dtype):
    """>= 65536 rows take the several-rows-per-wave launch; 65604 rows is not a
    multiple of its 32 rows per workgroup, so the last wave has a partial batch."""
    from tritonkv_amd.quantize import quantize_groupwise

    print(f"bulk quantize D={D} nbits={nbits} gs={gs} {dtype}", flush=True)
    g = torch.Generator().manual_seed(nbits + D)
    k = (torch.randn(2, 2, 16401, D, generator=g) * 3).to(dtype)
    k[0, 1, 7, :gs] = 1.5  # a constant group
    qt = quantize_groupwise(k.to(DEV), nbits, gs)
    ref = oq.quantize_groupwise(k.numpy(), nbits, gs)
    assert np.array_equal(qt.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_bits16(qt.scale), ref.scale.view(np.uint16))
    assert np.array_equal(_bits16(qt.zero), ref.zero.view(np.uint16))


@pytest.mark.parametrize("nbits,gs,D", [(4, 32, 128), (2, 16, 128), (4, 64, 64), (2, 128, 128)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gpu_quantize_unaligned_input_takes_the_row_kernel(nbits, gs, D, dtype):
    """Input not 16-byte aligned: quantized one wave per row (lane j owns byte
    j), the same code the fused decode-step append runs; bit-exact too."""
    from tritonkv_amd.quantize import quantize_groupwise

    g = torch.Generator().manual_seed(nbits * gs + D)
    n = 3 * 2 * 77 * D
    buf = torch.empty(n + 1, dtype=dtype, device=DEV)
    x = buf[1:].view(3, 2, 77, D)  # one element past a 256-byte boundary
    x.copy_((torch.randn(3, 2, 77, D, generator=g) * 2).to(dtype))
    assert x.data_ptr() % 16
    qt = quantize_groupwise(x, nbits, gs)
    ref = oq.quantize_groupwise(x.cpu().numpy(), nbits, gs)
    assert np.array_equal(qt.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_bits16(qt.scale), ref.scale.view(np.uint16))
    assert np.array_equal(_bits16(qt.zero), ref.zero.view(np.uint16))
    xb = _boundary_rows(300, 128, nbits, 32, seed=5).to(torch.float32)
    buf = torch.empty(xb.numel() + 1, dtype=torch.float32, device=DEV)
    xu = buf[1:].view(xb.shape)
    xu.copy_(xb)
    qt = quantize_groupwise(xu, nbits, 32)
    ref = oq.quantize_groupwise(xb.numpy(), nbits, 32)
    assert np.array_equal(qt.packed.cpu().numpy(), ref.packed)


def test_gpu_quantize_unaligned_beyond_one_launch():
    """More unaligned rows than one 2^32-work-item grid holds (4 * (2^24 - 1)):
    the row kernel is launched in pieces; the result equals the wide kernel's
    on the same (aligned) data bit for bit."""
    from tritonkv_amd.quantize import quantize_groupwise

    rows, D = 4 * ((1 << 24) - 1) + 100, 64
    print(f"unaligned quantize of {rows} rows", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    xa = torch.randn(1, 1, rows, D, device=DEV, generator=g, dtype=torch.float16)
    buf = torch.empty(xa.numel() + 1, dtype=torch.float16, device=DEV)
    xu = buf[1:].view(xa.shape)
    xu.copy_(xa)
    assert xu.data_ptr() % 16
    want = quantize_groupwise(xa, 4, 32)
    got = quantize_groupwise(xu, 4, 32)
    del buf, xu, xa
    assert torch.equal(got.packed, want.packed)
    assert torch.equal(got.scale.view(torch.int16), want.scale.view(torch.int16))
    assert torch.equal(got.zero.view(torch.int16), want.zero.view(torch.int16))


def _boundary_rows(rows, D, nbits, gs, seed):
    """fp32 rows whose values sit on, and one or two ulps either side of, the
    half-integer code boundaries (x - zero) / scale = k + 1/2 of their group."""
    rng = np.random.default_rng(seed)
    qmax = 2 ** nbits - 1
    x = np.empty((rows, D // gs, gs), np.float32)
    mn = rng.standard_normal((rows, D // gs)).astype(np.float16).astype(np.float32)
    rngw = rng.choice(np.array([1e-3, 0.37, 1.0, 3.0, 250.0], np.float32), size=mn.shape)
    mx = (mn + rngw).astype(np.float32)
    sf = ((mx - mn) / np.float32(qmax)).astype(np.float16).astype(np.float32)
    k = rng.integers(0, qmax, size=x.shape).astype(np.float32)
    v = (mn[..., None] + ((k + np.float32(0.5)) * sf[..., None]).astype(np.float32)).astype(np.float32)
    nudge = rng.integers(-2, 3, size=x.shape)
    for _ in range(2):
        v = np.where(nudge > 0, np.nextafter(v, np.float32(np.inf)), v)
        v = np.where(nudge < 0, np.nextafter(v, np.float32(-np.inf)), v)
        nudge = nudge - np.sign(nudge)
    x[:] = np.clip(v, mn[..., None], mx[..., None])
    x[..., 0], x[..., 1] = mn, mx
    return torch.from_numpy(x.reshape(1, 1, rows, D))


@pytest.mark.parametrize("rows", [300, 65600])
@pytest.mark.parametrize("nbits,gs", [(4, 32), (2, 16), (4, 128)])
def test_gpu_quantize_rounding_boundaries(rows, nbits, gs):
    """Values on and next to the codes' rounding boundaries, where a quotient
    taken as a product with the reciprocal could round the other way; both
    launches (a few rows, and the several-rows-per-wave bulk one)."""
    from tritonkv_amd.quantize import quantize_groupwise

    D = 128
    print(f"boundaries rows={rows} nbits={nbits} gs={gs}", flush=True)
    x = _boundary_rows(rows, D, nbits, gs, seed=rows + nbits + gs)
    qt = quantize_groupwise(x.to(DEV), nbits, gs)
    ref = oq.quantize_groupwise(x.numpy(), nbits, gs)
    assert np.array_equal(qt.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_bits16(qt.scale), ref.scale.view(np.uint16))
    assert np.array_equal(_bits16(qt.zero), ref.zero.view(np.uint16))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("gs", [16, 32, 64, 128])
@pytest.mark.parametrize("path", [0, 1])
def test_decode_unpack_paths_are_bit_exact(D, nbits, gs, path):
    """Codes and fp32 dequant through the decode kernel's own register unpack."""
    if gs > D:
        pytest.skip("group larger than head_dim")
    from tritonkv_amd.quantize import quantize_groupwise, unpack_dequant_path

    print(f"unpack path={path} D={D} nbits={nbits} gs={gs}", flush=True)
    # 77 rows: not a multiple of the 16/32-row unpack tiles, so the tail is exercised.
    _, k, _ = oinp.make_random_kv(1, 1, 1, 77, D, seed=31 * D + nbits + gs)
    qt = quantize_groupwise(k.to(DEV), nbits, gs)
    codes, vals = unpack_dequant_path(qt, path)
    ref = oq.QuantNP(qt.packed.cpu().numpy(), qt.scale.cpu().numpy(), qt.zero.cpu().numpy(),
                     nbits, gs, D)
    assert np.array_equal(codes.cpu().numpy(), oq.unpack_codes(ref.packed, nbits, D))
    assert np.array_equal(vals.cpu().numpy().view(np.uint32),
                          oq.dequantize_groupwise(ref).view(np.uint32))


@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("D", [64, 128])
def test_gpu_pack_unpack_roundtrip(nbits, D):
    from tritonkv_amd.quantize import pack_codes, unpack_codes

    g = torch.Generator().manual_seed(0)
    codes = torch.randint(0, 2 ** nbits, (3, 5, D), generator=g, dtype=torch.uint8)
    packed = pack_codes(codes.to(DEV), nbits)
    assert np.array_equal(packed.cpu().numpy(), oq.pack_codes(codes.numpy(), nbits))
    assert torch.equal(unpack_codes(packed, nbits, D).cpu(), codes)


@pytest.mark.parametrize("nbits", [2, 4])
def test_append_matches_whole_cache_quantization(nbits):
    """Token-by-token append at ragged per-row positions == quantizing the whole cache."""
    from tritonkv_amd.quantize import append_kv, empty_cache, quantize_groupwise

    B, HKV, S, D, gs = 3, 2, 40, 128, 32
    _, k, _ = oinp.make_random_kv(B, 4, HKV, S, D, seed=nbits)
    k = k.to(DEV)
    whole = quantize_groupwise(k, nbits, gs)
    cache = empty_cache(B, HKV, S, D, nbits, gs, DEV)
    cache.packed.zero_(), cache.scale.zero_(), cache.zero.zero_()
    for t in range(S):
        pos = torch.tensor([t] * B, dtype=torch.int32, device=DEV)
        append_kv(cache, k[:, :, t:t + 1].contiguous(), pos)
    assert torch.equal(cache.packed, whole.packed)
    assert torch.equal(cache.scale, whole.scale)
    assert torch.equal(cache.zero, whole.zero)


def test_append_ragged_positions_and_out_of_range_rows_are_not_written():
    from tritonkv_amd.quantize import append_kv, empty_cache, quantize_groupwise

    B, HKV, S, D, nbits, gs = 4, 2, 16, 128, 4, 32
    _, k, _ = oinp.make_random_kv(B, 4, HKV, 2, D, seed=9)
    k = k.to(DEV)
    cache = empty_cache(B, HKV, S, D, nbits, gs, DEV)
    cache.packed.fill_(0xAB), cache.scale.zero_(), cache.zero.zero_()
    pos = torch.tensor([0, 5, 15, 40], dtype=torch.int32, device=DEV)  # row 2: 1 of 2 fits; row 3: none
    append_kv(cache, k, pos)
    ref = quantize_groupwise(k, nbits, gs)
    assert torch.equal(cache.packed[0, :, 0:2], ref.packed[0])
    assert torch.equal(cache.packed[1, :, 5:7], ref.packed[1])
    assert torch.equal(cache.packed[2, :, 15:16], ref.packed[2, :, :1])
    assert bool((cache.packed[3] == 0xAB).all())
    untouched = torch.ones(S, dtype=torch.bool, device=DEV)
    untouched[5:7] = False
    assert bool((cache.packed[1][:, untouched] == 0xAB).all())


def test_roundtrip_error_report():
    from tritonkv_amd.quantize import roundtrip_error

    x = torch.randn(4, 7, 128, generator=torch.Generator().manual_seed(1)).to(DEV)
    r4 = roundtrip_error(x, 4, 32)
    r2 = roundtrip_error(x, 2, 32)
    assert r4["effective_bits"] == 5.0 and r2["effective_bits"] == 3.0
    assert r4["rel_l2"] < r2["rel_l2"] and r4["cosine"] > 0.99
