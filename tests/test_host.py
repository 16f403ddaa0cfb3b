"""CPU tests of the host side and the C ABI (no kernel is launched).

* the library loads and exports every symbol ``include/tkv.h`` declares;
* the ctypes mirror of ``tkv_decode_args`` has the C struct's layout;
* the C entry points reject bad arguments before touching the GPU;
* the Python wrappers validate in the reference's order and raise its errors
  (``kernels/fused_decode_attn.py:465-483``) before the backend check;
* split arithmetic matches the oracle's restatement of the reference;
* nothing on the product path runs on the CPU (no fallback).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

from oracle import splits as osp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tkv.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(tkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi():
    syms = _declared_symbols()
    for name in ("tkv_fused_decode_attention", "tkv_fp16_decode_attention", "tkv_combine_splits",
                 "tkv_quantize_pack", "tkv_unpack_dequant", "tkv_pack_codes"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    from tritonkv_amd import _lib

    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.tkv_abi_version() == 7


def test_library_is_gfx950_only():
    from tritonkv_amd import _lib

    with tempfile.TemporaryDirectory() as d:
        fb = os.path.join(d, "fatbin.bin")
        subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", _lib.LIB_PATH, fb],
                       check=True)
        out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                              f"--input={fb}"], capture_output=True, text=True, check=True)
    targets = [t for t in out.stdout.split() if "amdgcn" in t]
    assert targets == ["hipv4-amdgcn-amd-amdhsa--gfx950"], targets


def test_decode_args_layout_matches_c():
    from tritonkv_amd import _lib

    src = r"""
    #include <stdio.h>
    #include <stddef.h>
    #include "tkv.h"
    int main(void) {
      printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(tkv_decode_args),
             offsetof(tkv_decode_args, q_is_fp32), offsetof(tkv_decode_args, seq_lens),
             offsetof(tkv_decode_args, B), offsetof(tkv_decode_args, sm_scale),
             offsetof(tkv_decode_args, num_splits), offsetof(tkv_decode_args, counters),
             offsetof(tkv_decode_args, waves), offsetof(tkv_decode_args, block_table),
             offsetof(tkv_decode_args, page_size), offsetof(tkv_decode_args, num_pages),
             offsetof(tkv_decode_args, k_new), offsetof(tkv_decode_args, new_is_fp32),
             offsetof(tkv_decode_args, key_block), offsetof(tkv_decode_args, num_splits_total),
             sizeof(tkv_device_info_t));
      return 0;
    }"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        open(c, "w").write(src)
        exe = os.path.join(d, "l")
        subprocess.run(["gcc", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True,
                                               check=True).stdout.split()]
    A = _lib.DecodeArgs
    assert vals == [ctypes.sizeof(A), A.q_is_fp32.offset, A.seq_lens.offset, A.B.offset,
                    A.sm_scale.offset, A.num_splits.offset, A.counters.offset, A.waves.offset,
                    A.block_table.offset, A.page_size.offset, A.num_pages.offset,
                    A.k_new.offset, A.new_is_fp32.offset, A.key_block.offset,
                    A.num_splits_total.offset, ctypes.sizeof(_lib.DeviceInfo)]


def test_work_order_argument_checks_without_a_gpu():
    """work_order: 8-byte aligned, slots that fit int32, quantized path only and
    not with the allocation-free entry (each check returns before any launch)."""
    from tritonkv_amd import _lib

    lib = _lib.load()
    dummy = 0x1000
    a = _lib.DecodeArgs(q=dummy, k=dummy, v=dummy, k_scale=dummy, k_zero=dummy, v_scale=dummy,
                        v_zero=dummy, out=dummy, acc=dummy, maxs=dummy, sums=dummy, B=2, HQ=4,
                        HKV=2, S=256, D=128, k_nbits=4, v_nbits=4, group_size=32, sm_scale=0.1,
                        split_size=64, num_splits=4, waves=8, work_order=dummy + 2)
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.work_order = dummy + 4  # (idx, length) pairs: 8-byte aligned
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.work_order = dummy
    a.group_size = 8  # not instantiated: refused before the order launch as well
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.group_size = 32
    assert lib.tkv_fp16_decode_attention(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    assert lib.tkv_fp16_decode_split(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.acc = a.maxs = a.sums = None
    assert lib.tkv_fused_decode_attention_noalloc(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.acc = a.maxs = a.sums = dummy
    a.D = 64  # ordered kernels exist for head dim 128 only
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.D = 128
    a.B, a.HQ, a.HKV = 1 << 15, 1 << 15, 1 << 15  # B * HKV * num_splits = 2^32 slots
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL


def test_blocks_past_the_32bit_buffer_range_are_refused_without_a_gpu():
    """One (b, kv head) block (or page slab) of any cache tensor must span less
    than 2^32 bytes: the split kernels' buffer resources have 32-bit ranges.
    Larger ones are refused before any launch, where a wrapped range would
    have read zeros past the wrap."""
    from tritonkv_amd import _lib

    lib = _lib.load()
    dummy = 0x1000
    a = _lib.DecodeArgs(q=dummy, k=dummy, v=dummy, k_scale=dummy, k_zero=dummy, v_scale=dummy,
                        v_zero=dummy, out=dummy, acc=dummy, maxs=dummy, sums=dummy, B=1, HQ=8,
                        HKV=2, D=128, k_nbits=4, v_nbits=4, group_size=32, sm_scale=0.1,
                        waves=8)

    def with_s(S, ns=64):
        a.S, a.num_splits, a.split_size = S, ns, -(-S // ns)
        return a

    # 4-bit codes: 64 B per row, so 2^26 rows are exactly 2^32 bytes
    rc = lib.tkv_fused_decode_attention(ctypes.byref(with_s(1 << 26)), None)
    assert rc == _lib.TKV_EUNSUPPORTED
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    assert lib.tkv_read_probe(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.acc = a.maxs = a.sums = None
    assert lib.tkv_fused_decode_attention_noalloc(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.acc = a.maxs = a.sums = dummy
    # 2-bit K with 4-bit V: the V codes are the larger range
    a.k_nbits = 2
    assert lib.tkv_fused_decode_attention(ctypes.byref(with_s(1 << 26)), None) == \
        _lib.TKV_EUNSUPPORTED
    # 2-bit K and V, groups of 16: 32 B of codes and 16 B of scale per row -> 2^27 rows
    a.v_nbits, a.group_size = 2, 16
    assert lib.tkv_fused_decode_attention(ctypes.byref(with_s(1 << 27)), None) == \
        _lib.TKV_EUNSUPPORTED
    # the fp16 control: 256 B per row, 2^24 rows
    assert lib.tkv_fp16_decode_attention(ctypes.byref(with_s(1 << 24)), None) == \
        _lib.TKV_EUNSUPPORTED
    # a paged pool is bounded per page slab, not per sequence: a huge page is refused
    a.k_nbits = a.v_nbits = 4
    a.group_size = 32
    a.block_table, a.block_table_stride, a.num_pages = dummy, 1, 4
    a.page_size = 1 << 26
    assert lib.tkv_fused_decode_attention(ctypes.byref(with_s(1 << 26)), None) == \
        _lib.TKV_EUNSUPPORTED


def test_order_buffer_policy():
    """The Python entries take a work_order buffer for ragged split calls only."""
    from tritonkv_amd.kernels.fused_decode_attn import _order_for

    lens = object()  # only its presence matters
    assert _order_for({}, 32, 8, 1, "cpu", lens, None) is None     # 256 workgroups: one per CU
    assert _order_for({}, 64, 8, 1, "cpu", lens, None).numel() == 1024  # unsplit, 512 workgroups
    assert _order_for({}, 64, 8, 4, "cpu", None, None) is None     # equal lengths
    assert _order_for({}, 64, 8, 4, "cpu", lens, False) is None
    assert _order_for({}, 1, 2, 32, "cpu", lens, None) is None     # 64 workgroups fit the CUs
    assert _order_for({}, 64, 8, 4, "cpu", lens, None, D=64) is None  # no ordered D=64 kernels
    assert _order_for({}, 1, 2, 32, "cpu", lens, None, G=256) is not None  # 16 head blocks each
    assert _order_for({}, 4096, 8, 1, "cpu", lens, None) is None   # past ORDER_MAX_ROWS
    ws = {}
    buf = _order_for(ws, 64, 8, 4, "cpu", lens, None)
    assert buf.dtype == torch.int32 and buf.numel() == 4096 and ws["work_order"] is buf
    assert _order_for(ws, 64, 8, 2, "cpu", lens, None) is buf      # reused when large enough
    assert _order_for({}, 2, 3, 4, "cpu", None, True).numel() == 48  # forced


def test_c_entry_points_reject_bad_arguments_without_a_gpu():
    from tritonkv_amd import _lib

    lib = _lib.load()
    a = _lib.DecodeArgs()  # all NULL / zero
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    assert lib.tkv_fp16_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    assert lib.tkv_fused_decode_split(ctypes.byref(a), None) == _lib.TKV_EINVAL
    assert lib.tkv_combine_splits(None, None, None, None, 1, 1, 1, 128, None) == _lib.TKV_EINVAL
    assert lib.tkv_quantize_pack(None, 0, 1, 1, 1, 128, 4, 32, None, 1, None, None, None,
                                 None) == _lib.TKV_EINVAL
    assert lib.tkv_pack_codes(None, 1, 128, 4, None, None) == _lib.TKV_EINVAL
    assert lib.tkv_unpack_dequant(None, None, None, 1, 128, 4, 32, 0, None, None,
                                  None) == _lib.TKV_EINVAL
    # Non-null but inconsistent arguments: HQ not a multiple of HKV, uncovered history.
    dummy = 0x1000
    a = _lib.DecodeArgs(q=dummy, k=dummy, v=dummy, k_scale=dummy, k_zero=dummy, v_scale=dummy,
                        v_zero=dummy, out=dummy, B=1, HQ=12, HKV=5, S=64, D=128, k_nbits=4,
                        v_nbits=4, group_size=32, sm_scale=0.1, split_size=64, num_splits=1)
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.HKV, a.split_size = 2, 32
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.split_size, a.group_size = 64, 48
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.group_size, a.waves = 32, 6
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.waves, a.D = 8, 96
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    # Splits are the grid's y axis: at most 65535.
    a.D, a.S, a.split_size, a.num_splits = 128, 65536 * 32, 32, 65536
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    assert lib.tkv_fp16_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.D, a.S, a.split_size, a.num_splits = 96, 64, 64, 1
    # B * HQ rows must fit a 32-bit grid
    a.D, a.B, a.HQ, a.HKV = 128, 1 << 20, 1 << 12, 1 << 12
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    assert lib.tkv_combine_splits(dummy, dummy, dummy, dummy, 1 << 20, 1 << 12, 1, 128,
                                  None) == _lib.TKV_EINVAL
    a.B, a.HQ, a.HKV = 1, 12, 2
    # Paged caches: page size a multiple of 32, a block table covering S exactly.
    a.D, a.page_size, a.num_pages, a.block_table_stride = 128, 16, 8, 4
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.page_size, a.block_table_stride = 32, 2
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL  # no table
    a.block_table = dummy
    a.block_table_stride = 3
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL  # 3*32 != S
    a.block_table_stride = 2
    assert lib.tkv_fp16_decode_attention(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    a.page_size = -32
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    # Fused append: k_new needs v_new; the fp16 control has no fused append.
    a.page_size, a.block_table, a.block_table_stride = 0, None, 0
    a.k_new = dummy
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.v_new = dummy + 1  # misaligned fp16
    assert lib.tkv_fused_decode_attention(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.v_new = dummy
    assert lib.tkv_fp16_decode_attention(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED
    assert lib.tkv_paged_quantize_pack(None, 0, 1, 1, 1, 128, 4, 32, None, None, 1, 32, 1, None,
                                       None, None, None) == _lib.TKV_EINVAL
    assert lib.tkv_paged_quantize_pack(dummy, 0, 1, 1, 1, 128, 4, 32, dummy, dummy, 1, 48, 1,
                                       dummy, dummy, dummy, None) == _lib.TKV_EINVAL
    assert _lib.status_string(_lib.TKV_EINVAL) == "invalid argument"
    # the read-ceiling probe takes the split kernel's contiguous form only
    assert lib.tkv_read_probe(None, None) == _lib.TKV_EINVAL
    a.k_new = a.v_new = dummy
    assert lib.tkv_read_probe(ctypes.byref(a), None) == _lib.TKV_EUNSUPPORTED


def test_noalloc_entry_point_rejects_before_touching_the_gpu():
    """tkv_fused_decode_attention_noalloc: no workspace accepted, partials bounded by the scratch."""
    from tritonkv_amd import _lib

    lib = _lib.load()
    assert lib.tkv_fused_decode_attention_noalloc(None, None) == _lib.TKV_EINVAL
    dummy = 0x1000
    a = _lib.DecodeArgs(q=dummy, k=dummy, v=dummy, k_scale=dummy, k_zero=dummy, v_scale=dummy,
                        v_zero=dummy, out=dummy, B=1, HQ=12, HKV=2, S=4096, D=128, k_nbits=4,
                        v_nbits=4, group_size=32, sm_scale=0.1, split_size=512, num_splits=8)
    a.acc = a.maxs = a.sums = dummy  # the partials are the library's
    assert lib.tkv_fused_decode_attention_noalloc(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.acc = a.maxs = a.sums = None
    a.counters = dummy
    assert lib.tkv_fused_decode_attention_noalloc(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.counters = None
    a.split_base, a.num_splits_total = 1, 9  # must own every split
    assert lib.tkv_fused_decode_attention_noalloc(ctypes.byref(a), None) == _lib.TKV_EINVAL
    a.split_base, a.num_splits_total = 0, 0
    # 12 rows x 4096 splits x (128 + 2) floats = 24.4 MiB > 16 MiB
    a.split_size, a.num_splits = 1, 4096
    assert lib.tkv_fused_decode_attention_noalloc(ctypes.byref(a), None) == _lib.TKV_ESCRATCH
    rows = _lib.NOALLOC_SCRATCH_BYTES // ((128 + 2) * 4)
    assert 12 * 4096 > rows
    assert "static scratch" in _lib.status_string(_lib.TKV_ESCRATCH)
    with pytest.raises(ValueError, match="static scratch"):
        _lib.check(_lib.TKV_ESCRATCH, "noalloc")


def _fake_qt(B=1, HKV=2, S=64, D=128, nbits=4, gs=32, device="cpu"):
    from tritonkv_amd.quantize import QuantizedTensor

    P = 8 // nbits
    return QuantizedTensor(torch.zeros(B, HKV, S, D // P, dtype=torch.uint8, device=device),
                           torch.ones(B, HKV, S, D // gs, dtype=torch.float16, device=device),
                           torch.zeros(B, HKV, S, D // gs, dtype=torch.float16, device=device),
                           nbits, gs, D)


def test_python_validation_precedes_backend_check():
    from tritonkv_amd.kernels import fused_decode_attention

    q = torch.zeros(1, 12, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="same nbits"):
        fused_decode_attention(q, _fake_qt(nbits=4), _fake_qt(nbits=2))
    with pytest.raises(ValueError, match="same nbits"):
        fused_decode_attention(q, _fake_qt(gs=32), _fake_qt(gs=64))
    with pytest.raises(ValueError, match="incompatible"):
        fused_decode_attention(torch.zeros(2, 12, 128), _fake_qt(), _fake_qt())
    with pytest.raises(ValueError, match="multiple of HKV"):
        fused_decode_attention(torch.zeros(1, 12, 128), _fake_qt(HKV=5), _fake_qt(HKV=5))
    with pytest.raises(ValueError, match="power of two"):
        fused_decode_attention(torch.zeros(1, 12, 96), _fake_qt(D=96), _fake_qt(D=96))
    with pytest.raises(ValueError, match="multiple of group_size"):
        fused_decode_attention(torch.zeros(1, 12, 64), _fake_qt(D=64, gs=128),
                               _fake_qt(D=64, gs=128))
    with pytest.raises(ValueError, match="fold_zp"):
        fused_decode_attention(q, _fake_qt(gs=8), _fake_qt(gs=8), fold_zp=True)
    with pytest.raises(ValueError, match="same shape"):
        fused_decode_attention(q, _fake_qt(S=64), _fake_qt(S=32))
    # every tensor on one device: a host pointer handed to a kernel would fault the GPU
    with pytest.raises(ValueError, match="same device"):
        fused_decode_attention(q, _fake_qt(), _fake_qt(device="meta"))
    # the fused append writes into the caches: a non-contiguous one (the token
    # would land in a temporary copy) or a misaligned one is refused, never copied
    kq = _fake_qt(S=64)
    view = type(kq)(kq.packed[:, :, :48], kq.scale[:, :, :48], kq.zero[:, :, :48], 4, 32, 128)
    assert not view.packed.is_contiguous()
    tok = torch.zeros(1, 2, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="contiguous"):
        fused_decode_attention(q, view, _fake_qt(S=48), k_new=tok, v_new=tok)
    flat = torch.zeros(1 + 2 * 48 * 64, dtype=torch.uint8)
    shifted = type(kq)(flat[1:].view(1, 2, 48, 64), view.scale.contiguous(),
                       view.zero.contiguous(), 4, 32, 128)
    with pytest.raises(ValueError, match="16-byte boundary"):
        fused_decode_attention(q, shifted, _fake_qt(S=48))
    from tritonkv_amd.kernels import fp16_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import _check_out

    kv = torch.zeros(1, 2, 64, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="same device"):
        fp16_decode_attention(q, kv, kv.to("meta"))
    with pytest.raises(ValueError, match="tensor on"):
        _check_out(torch.empty(1, 12, 128), 1, 12, 128, torch.device("cuda", 0))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_backend_unavailable_raises_runtime_error():
    from tritonkv_amd.kernels import fp16_decode_attention, fused_decode_attention, triton_available

    ok, why = triton_available()
    assert not ok and why
    with pytest.raises(RuntimeError):
        fused_decode_attention(torch.zeros(1, 12, 128), _fake_qt(), _fake_qt())
    with pytest.raises(RuntimeError):
        fp16_decode_attention(torch.zeros(1, 12, 128), torch.zeros(1, 2, 8, 128),
                              torch.zeros(1, 2, 8, 128))


def test_quantizer_has_no_cpu_fallback():
    from tritonkv_amd import quantize as tq

    with pytest.raises(RuntimeError, match="GPU"):
        tq.quantize_groupwise(torch.randn(2, 128), 4, 32)
    with pytest.raises(RuntimeError, match="GPU"):
        tq.unpack_codes(torch.zeros(2, 64, dtype=torch.uint8), 4, 128)
    with pytest.raises(RuntimeError, match="GPU"):
        tq.pack_codes(torch.zeros(2, 128, dtype=torch.uint8), 4)
    # argument errors still come first, as in quantize.py:68-70, :156-161, :177-178, :200-204
    with pytest.raises(ValueError):
        tq.quantize_groupwise(torch.randn(2, 128), 3, 32)
    with pytest.raises(ValueError):
        tq.quantize_groupwise(torch.randn(2, 128), 4, 48)
    with pytest.raises(TypeError):
        tq.pack_codes(torch.zeros(2, 128, dtype=torch.int32), 4)
    with pytest.raises(ValueError):
        tq.unpack_codes(torch.zeros(2, 60, dtype=torch.uint8), 4, 128)


def test_quantized_tensor_accounting():
    qt = _fake_qt(B=1, HKV=2, S=16, D=128, nbits=4, gs=32)
    assert qt.effective_bits_per_element() == 5.0
    assert qt.nbytes() * 8 / (2 * 16 * 128) == pytest.approx(5.0)
    assert qt.shape == (1, 2, 16, 128) and qt.n_groups == 4 and qt.codes_per_byte == 2
    assert _fake_qt(nbits=2).effective_bits_per_element() == 3.0


@pytest.mark.parametrize("S,block_n,ns", [(4096, 64, 5), (4096, 64, 17), (4096, 64, 64),
                                          (3000, 128, 7), (1, 64, 8), (17, 64, 3),
                                          (16384, 16, 1000), (2048, 32, 2)])
def test_plan_splits_honours_explicit_num_splits_like_the_reference(S, block_n, ns):
    from tritonkv_amd.kernels import plan_splits

    assert plan_splits(S, block_n, ns, 1, 2, 6) == osp.split_plan(S, block_n, ns)


def test_plan_splits_caps_the_split_count_at_the_grid_limit():
    from tritonkv_amd.kernels import plan_splits

    _, ns, split = plan_splits(1 << 21, 16, 100000, 1, 8, 4)
    assert ns <= 65535 and ns * split >= 1 << 21 and (ns - 1) * split < 1 << 21


def test_pick_num_splits_formula():
    from tritonkv_amd.kernels import pick_num_splits

    for B, HKV, nb, tgt in [(1, 2, 256, 1024), (32, 8, 512, 1024), (64, 8, 100, 1024),
                            (1, 1, 3, 7), (4, 8, 1, 1024)]:
        assert pick_num_splits(B, HKV, nb, tgt) == osp.pick_num_splits(B, HKV, nb, tgt)


@pytest.mark.parametrize("B,HKV,G,S", [(1, 2, 6, 512), (1, 2, 6, 16384), (32, 8, 4, 32768),
                                       (64, 8, 8, 131072), (1, 8, 1, 1), (2, 8, 4, 17)])
def test_default_split_plan_covers_history_without_empty_splits(B, HKV, G, S):
    from tritonkv_amd.kernels import plan_splits

    for ragged in (False, True):
        _, ns, size = plan_splits(S, 64, None, B, HKV, G, ragged=ragged)
        assert ns >= 1 and size * ns >= S and size * (ns - 1) < S


def test_ragged_batches_of_a_unit_per_cu_split_long_histories(monkeypatch):
    from tritonkv_amd.kernels import fused_decode_attn as fda

    monkeypatch.setattr(fda, "compute_units", lambda: 256)
    assert fda.plan_splits(131072, 64, None, 64, 8, 8)[1] == 1
    # pieces of at most 32768 tokens, at least two
    assert fda.plan_splits(131072, 64, None, 64, 8, 8, ragged=True)[1] == 4
    assert fda.plan_splits(131072 + 64, 64, None, 64, 8, 8, ragged=True)[1] == 4
    assert fda.plan_splits(32768, 64, None, 32, 8, 4, ragged=True)[1] == 2
    assert fda.plan_splits(16384, 64, None, 32, 8, 4, ragged=True)[1] == 2
    assert fda.plan_splits(8192, 64, None, 64, 8, 8, ragged=True)[1] == 1  # short: unsplit
    # below one unit per CU the ordinary policy applies either way
    assert fda.plan_splits(32768, 64, None, 4, 8, 4, ragged=True) == \
        fda.plan_splits(32768, 64, None, 4, 8, 4)


def test_timing_replicas_and_warmup_floor():
    """Rotating-set sizing (>= 768 MB of distinct caches) and the warm-up rule:
    at least W steps and at least MIN_WARMUP_S of replays, whatever the step count."""
    from tritonkv_amd.timing import MIN_WARMUP_S, replicas_for, warmup_replays_needed

    assert replicas_for(163_840, 768_000_000) == 4688
    assert replicas_for(16_777_216, 768_000_000) == 46
    assert replicas_for(768_000_000, 768_000_000) == 1
    assert replicas_for(0, 768_000_000) == 1
    assert replicas_for(1, max_replicas=8) == 8
    assert MIN_WARMUP_S >= 0.3
    # the driver's --steps 20 --warmup 5 on a 4.5 ms replay: the time floor rules
    assert warmup_replays_needed(20, 5, 0.0045, 0.5) == 112
    # many warm-up steps: the step count rules
    assert warmup_replays_needed(20, 10_000, 0.0045, 0.5) == 500
    # a replay longer than the floor still runs once
    assert warmup_replays_needed(20, 0, 2.0, 0.5) == 1


def test_prepared_call_key_tracks_what_the_argument_block_depends_on():
    """The workspace's checked argument block is reused only under an equal
    key: a tensor's key changes with its storage address, shape, dtype and
    layout -- also when the same tensor object is resized or restrided in
    place -- and a workspace without a prepared call, or with another key,
    yields none."""
    from tritonkv_amd.kernels.fused_decode_attn import _new_key, _prepared, _tensor_key

    t = torch.zeros(2, 3, 64, 16, dtype=torch.uint8)
    k0 = _tensor_key(t)
    assert _tensor_key(t) == k0
    assert _tensor_key(torch.zeros_like(t)) != k0                 # another storage
    t2 = torch.zeros(2, 3, 64, 16, dtype=torch.uint8)
    ptr = t2.data_ptr()
    t2.resize_(2, 3, 32, 16)                                      # same storage, new shape
    assert t2.data_ptr() == ptr and _tensor_key(t2)[1] != k0[1]
    v = t.view(torch.int8)
    assert v.data_ptr() == t.data_ptr() and _tensor_key(v) != k0  # dtype view
    tt = t.transpose(2, 3)
    assert tt.data_ptr() == t.data_ptr() and _tensor_key(tt) != k0  # layout
    assert _tensor_key(None) is None and _new_key(None) is None
    assert _new_key(t) == _new_key(torch.ones_like(t))             # new rows may move
    assert _new_key(t) != _new_key(t.half())

    class Prep:
        key = ("a", 1)
    assert _prepared(None, ("a", 1)) is None
    assert _prepared({}, ("a", 1)) is None
    ws = {"call": Prep()}
    assert _prepared(ws, ("a", 1)) is ws["call"]
    assert _prepared(ws, ("a", 2)) is None
