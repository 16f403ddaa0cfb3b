"""ctypes binding of ``libtkv_hip.so``, the gfx950 kernels' C ABI (``include/tkv.h``).

The library is loaded after ``torch``: torch's bundled HIP runtime carries the
same soname (``libamdhip64.so.7``) that the library links against, so the
dynamic linker resolves both to the one runtime already in the process and
torch's streams are valid handles for the kernels launched here.

There is no fallback: if the library is missing or fails to load, every entry
point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be imported before the library, see above)

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libtkv_hip.so")

TKV_OK = 0
TKV_EINVAL = -1
TKV_EUNSUPPORTED = -2
TKV_ENODEVICE = -3
TKV_ESCRATCH = -4
NOALLOC_SCRATCH_BYTES = 16 << 20  # TKV_NOALLOC_SCRATCH_BYTES


class DecodeArgs(ctypes.Structure):
    """Mirror of ``tkv_decode_args`` (include/tkv.h)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_is_fp32", ctypes.c_int32),
        ("k", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("k_zero", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("v_zero", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("acc", ctypes.c_void_p),
        ("maxs", ctypes.c_void_p),
        ("sums", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("B", ctypes.c_int32),
        ("HQ", ctypes.c_int32),
        ("HKV", ctypes.c_int32),
        ("S", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("k_nbits", ctypes.c_int32),
        ("v_nbits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("sm_scale", ctypes.c_float),
        ("split_size", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("counters", ctypes.c_void_p),
        ("waves", ctypes.c_int32),
        ("block_table", ctypes.c_void_p),
        ("block_table_stride", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("k_new", ctypes.c_void_p),
        ("v_new", ctypes.c_void_p),
        ("new_is_fp32", ctypes.c_int32),
        ("key_block", ctypes.c_int32),
        ("split_base", ctypes.c_int32),
        ("num_splits_total", ctypes.c_int32),
        ("work_order", ctypes.c_void_p),
    ]


class DeviceInfo(ctypes.Structure):
    """Mirror of ``tkv_device_info_t``."""

    _fields_ = [
        ("device", ctypes.c_int32),
        ("compute_units", ctypes.c_int32),
        ("warp_size", ctypes.c_int32),
        ("l2_bytes", ctypes.c_int32),
        ("global_mem_bytes", ctypes.c_int64),
        ("clock_khz", ctypes.c_int32),
        ("mem_clock_khz", ctypes.c_int32),
        ("mem_bus_bits", ctypes.c_int32),
        ("gcn_arch", ctypes.c_char * 64),
    ]


# name -> (argtypes, restype); every symbol include/tkv.h declares.
_P, _I32, _I64, _F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    "tkv_fused_decode_attention": ([ctypes.POINTER(DecodeArgs), _P], ctypes.c_int),
    "tkv_fp16_decode_attention": ([ctypes.POINTER(DecodeArgs), _P], ctypes.c_int),
    "tkv_fused_decode_attention_noalloc": ([ctypes.POINTER(DecodeArgs), _P], ctypes.c_int),
    "tkv_fused_decode_split": ([ctypes.POINTER(DecodeArgs), _P], ctypes.c_int),
    "tkv_read_probe": ([ctypes.POINTER(DecodeArgs), _P], ctypes.c_int),
    "tkv_fp16_decode_split": ([ctypes.POINTER(DecodeArgs), _P], ctypes.c_int),
    "tkv_combine_splits": ([_P, _P, _P, _P, _I32, _I32, _I32, _I32, _P], ctypes.c_int),
    "tkv_quantize_pack": ([_P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _P],
                          ctypes.c_int),
    "tkv_paged_quantize_pack": ([_P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _I32, _I32,
                                 _I32, _P, _P, _P, _P], ctypes.c_int),
    "tkv_quantize_keys_channel": ([_P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I32, _P, _P, _P,
                                   _P], ctypes.c_int),
    "tkv_channel_decode_attention": ([ctypes.POINTER(DecodeArgs), _P, _P, _P, _I32, _P],
                                     ctypes.c_int),
    "tkv_channel_window_append": ([_P, _P, _I32, _I32, _I32, _P, _P, _I32, _P, _P], ctypes.c_int),
    "tkv_channel_window_flush": ([_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _I32,
                                  _P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "tkv_pack_codes": ([_P, _I64, _I32, _I32, _P, _P], ctypes.c_int),
    "tkv_unpack_dequant": ([_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P], ctypes.c_int),
    "tkv_device_info": ([ctypes.POINTER(DeviceInfo)], ctypes.c_int),
    "tkv_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "tkv_abi_version": ([], ctypes.c_int),
}

_LIB = None
_LOAD_ERROR: str | None = None


def load():
    """Load the library (once).  Raises RuntimeError if it is absent or broken."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        _LOAD_ERROR = (f"{LIB_PATH} is not built; run `python -m tritonkv_amd.build` "
                       "(hipcc --offload-arch=gfx950)")
        raise RuntimeError(_LOAD_ERROR)
    try:
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    except OSError as exc:
        _LOAD_ERROR = f"failed to load {LIB_PATH}: {exc}"
        raise RuntimeError(_LOAD_ERROR) from exc
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _LIB = lib
    return lib


def load_error() -> str | None:
    try:
        load()
    except RuntimeError:
        pass
    return _LOAD_ERROR


def status_string(rc: int) -> str:
    return load().tkv_status_string(rc).decode()


def check(rc: int, what: str) -> None:
    """Raise on a non-zero status: ValueError for argument errors, RuntimeError otherwise."""
    if rc == TKV_OK:
        return
    msg = f"{what}: {status_string(rc)} (status {rc})"
    if rc in (TKV_EINVAL, TKV_EUNSUPPORTED, TKV_ESCRATCH):
        raise ValueError(msg)
    raise RuntimeError(msg)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def device_info() -> DeviceInfo:
    info = DeviceInfo()
    check(load().tkv_device_info(ctypes.byref(info)), "tkv_device_info")
    return info
