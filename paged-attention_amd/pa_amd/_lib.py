"""ctypes binding of libpa_decode.so (include/pa_decode.h).

Loading fails loudly: there is no CPU fallback for any entry point. Status
codes become exceptions with the library's own message:

    PA_ERR_INVALID_ARGUMENT -> InvalidArgument (a ValueError; std::invalid_argument)
    PA_ERR_LENGTH           -> LengthError     (std::length_error)
    PA_ERR_DEVICE           -> DeviceError     (a RuntimeError; CUDA_CHECK abort in the reference)
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import re

PKG_DIR = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = pathlib.Path(os.environ.get("PA_DECODE_LIB", PKG_DIR / "lib" / "libpa_decode.so"))
HEADER = PKG_DIR.parent / "include" / "pa_decode.h"

PA_OK = 0
PA_ERR_INVALID_ARGUMENT = 1
PA_ERR_LENGTH = 2
PA_ERR_DEVICE = 3

PA_KV_FP16 = 0
PA_KV_FP8_E4M3 = 1


class PaError(Exception):
    """Base class of every error the library reports."""


class InvalidArgument(PaError, ValueError):
    pass


class LengthError(PaError, ValueError):
    pass


class DeviceError(PaError, RuntimeError):
    pass


class DecodeParams(ctypes.Structure):
    """pa_decode_params (decode_types.hpp:14-45 DecodeParams)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("slot_ids", ctypes.c_void_p),
        ("block_table_stride", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("sm_scale", ctypes.c_float),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
        ("segments", ctypes.c_void_p),
        ("cta_seg_begin", ctypes.c_void_p),
        ("item_seg_begin", ctypes.c_void_p),
        ("num_ctas", ctypes.c_int32),
        ("needs_merge", ctypes.c_int32),
        ("partial_out", ctypes.c_void_p),
        ("partial_lse", ctypes.c_void_p),
        ("max_item_segments", ctypes.c_int32),
        ("block_merge", ctypes.c_int32),
        ("num_segments", ctypes.c_int32),
        ("merge_counters", ctypes.c_void_p),
    ]


class CacheConfig(ctypes.Structure):
    """pa_cache_config (paged_kv_cache.hpp:19-29 PagedKVCache::Config)."""

    _fields_ = [
        ("num_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_slots", ctypes.c_int32),
        ("max_pages_per_slot", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint
_F = ctypes.c_float
_S = ctypes.c_size_t
_PI = ctypes.POINTER(ctypes.c_int)
_PP = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); every function pa_decode.h declares.
SIGNATURES: dict[str, tuple] = {
    "pa_last_error": (ctypes.c_char_p, []),
    "pa_kv_dtype_bytes": (_I, [_I]),
    "pa_kv_dtype_name": (ctypes.c_char_p, [_I]),
    "pa_tile_tokens": (_I, [_I, _I, _I, _PI]),
    "pa_wave_ctas": (_I, [_I, _I, _I, _PI]),
    "pa_default_ctas": (_I, [_I, _I, _I, _PI]),
    "pa_plan_build": (_I, [_I, _P, _I, _I, _I, _I, _I, _PP]),
    "pa_plan_build_tiled": (_I, [_I, _P, _I, _I, _I, _PP]),
    "pa_plan_create": (_I, [_I, _I, _P, _I, _P, _P, _I, _I, _PP]),
    "pa_plan_destroy": (None, [_P]),
    "pa_plan_num_ctas": (_I, [_P]),
    "pa_plan_tile": (_I, [_P]),
    "pa_plan_num_segments": (_I, [_P]),
    "pa_plan_num_items": (_I, [_P]),
    "pa_plan_merge_mode": (_I, [_P, _PI]),
    "pa_plan_copy": (_I, [_P, _P, _P, _P]),
    "pa_device_plan_create": (_I, [_PP]),
    "pa_device_plan_destroy": (None, [_P]),
    "pa_device_plan_upload": (_I, [_P, _P, _I, _I, _P]),
    "pa_device_plan_bind": (_I, [_P, ctypes.POINTER(DecodeParams)]),
    "pa_decode": (_I, [_I, ctypes.POINTER(DecodeParams), _P]),
    "pa_decode_split": (_I, [_I, ctypes.POINTER(DecodeParams), _P]),
    "pa_decode_merge": (_I, [_I, ctypes.POINTER(DecodeParams), _P]),
    "pa_decode_static": (_I, [_I, ctypes.POINTER(DecodeParams), _I, _P]),
    "pa_append_quantize": (_I, [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P]),
    "pa_gather_kv": (_I, [_I, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "pa_stream_read": (_I, [_P, _S, _I, _P, _P]),
    "pa_stream_read_ex": (_I, [_P, _S, _I, _I, _I, _I, _P, _P]),
    "pa_stream_read_chunked": (_I, [_P, _S, _I, _I, _I, _P, _P]),
    "pa_fill_bytes": (_I, [_P, _S, _I, _P]),
    "pa_f32_to_f16": (_I, [_P, _P, _S, _P]),
    "pa_f16_to_f32": (_I, [_P, _P, _S, _P]),
    "pa_pool_create": (_I, [_I, _I, _I, _I, _PP]),
    "pa_pool_destroy": (None, [_P]),
    "pa_pool_admit": (_I, [_P]),
    "pa_pool_reserve": (_I, [_P, _I, _I, _PI, _PI, _PI]),
    "pa_pool_reserve_batch": (_I, [_P, _P, _P, _I, _PI]),
    "pa_pool_release": (_I, [_P, _I]),
    "pa_pool_shuffle_free_pages": (None, [_P, _U]),
    "pa_pool_free_pages": (_I, [_P]),
    "pa_pool_seq_len": (_I, [_P, _I]),
    "pa_pool_occupied": (_I, [_P, _I]),
    "pa_pool_max_seq_len": (_I, [_P]),
    "pa_pool_num_pages_of": (_I, [_P, _I]),
    "pa_pool_block_table": (_I, [_P, _I, _P, _I]),
    "pa_cache_bytes_per_page": (_S, [ctypes.POINTER(CacheConfig)]),
    "pa_kv_pool_stagger": (_S, []),
    "pa_cache_pages_for_budget": (_I, [ctypes.POINTER(CacheConfig), _S]),
    "pa_cache_create": (_I, [ctypes.POINTER(CacheConfig), _PP]),
    "pa_cache_destroy": (None, [_P]),
    "pa_cache_pool": (_P, [_P]),
    "pa_cache_admit": (_I, [_P]),
    "pa_cache_append": (_I, [_P, _I, _P, _P, _I, _P, _PI]),
    "pa_cache_append_batch": (_I, [_P, _P, _P, _I, _P, _P, _P, _PI]),
    "pa_cache_release": (_I, [_P, _I]),
    "pa_cache_shuffle_free_pages": (None, [_P, _U]),
    "pa_cache_params": (_I, [_P, ctypes.POINTER(DecodeParams)]),
    "pa_cache_plan": (_I, [_P, _P, _I, _I, _I, _P]),
    "pa_cache_run": (_I, [_P, _P, _P, _P]),
    "pa_cache_decode": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "pa_cache_last_plan": (_P, [_P]),
    "pa_cache_total_bytes": (_S, [_P]),
}

_lib: ctypes.CDLL | None = None


def _init_torch_device_state() -> None:
    """Loads torch's HIP runtime before this library's.

    torch ships its own libamdhip64 (soname libamdhip64.so.7), and its
    libraries ask for it as `libamdhip64.so`; this library asks for
    `libamdhip64.so.7`. Loaded after torch, the library's request matches
    torch's copy by soname and the process has one HIP runtime. Loaded first,
    it brings in the system's copy (/opt/rocm), and torch's request, which no
    loaded soname matches, then maps torch's own copy beside it: two HIP
    runtimes in one process, of which the second finds no device
    (hipErrorNoDevice, torch.cuda.is_available() False on the GPU boxes).
    So torch goes first (a no-op when torch is absent)."""
    try:
        import torch
    except ImportError:
        return
    torch.cuda.is_available()


def hip_runtimes() -> list[str]:
    """Distinct HIP runtime libraries mapped into this process (Linux)."""
    try:
        maps = pathlib.Path("/proc/self/maps").read_text()
    except OSError:
        return []
    paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    return sorted({os.path.realpath(p) for p in paths})


def load() -> ctypes.CDLL:
    """Loads the library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python paged-attention_amd/build.py` "
            "(or __graft_entry__.build()); there is no fallback path")
    _init_torch_device_state()
    lib = ctypes.CDLL(str(LIB_PATH))
    runtimes = hip_runtimes()
    if len(runtimes) > 1:
        raise RuntimeError(
            "two HIP runtimes are loaded in this process (" + ", ".join(runtimes) + "): libpa_decode.so was "
            "loaded before torch; import torch (and query a device) before loading it")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def header_functions() -> list[str]:
    """Names of the functions include/pa_decode.h declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text)))


def check(status: int) -> None:
    if status == PA_OK:
        return
    msg = load().pa_last_error().decode(errors="replace")
    if status == PA_ERR_INVALID_ARGUMENT:
        raise InvalidArgument(msg)
    if status == PA_ERR_LENGTH:
        raise LengthError(msg)
    raise DeviceError(msg or f"pa_decode error {status}")


def call(name: str, *args):
    """Calls a status-returning entry point and raises on failure."""
    check(getattr(load(), name)(*args))

