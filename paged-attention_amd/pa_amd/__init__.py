"""MI355X (gfx950) paged flash-decoding: Python side of libpa_decode.so.

`core` mirrors decode.hpp / paged_kv_cache.hpp over the C ABI; `decoder`
mirrors the reference's torch binding (`Decoder`). Importing this package does
not load the library; the first call does, and fails loudly if it is missing.
"""

from . import _lib
from ._lib import DecodeParams, CacheConfig, PaError, InvalidArgument, LengthError, DeviceError
from .core import (FP16, FP8_E4M3, DecodePlan, DevicePlan, PagePool, PagedKVCache, make_plan,
                   make_plan_tiled, paged_decode, decode_split, decode_merge, append_quantize,
                   gather_kv, stream_read, stream_read_chunked, fill_bytes, tile_tokens, wave_ctas, default_ctas, kv_dtype_bytes,
                   kv_dtype_name, sm_scale, kv_pool_stagger, alloc_kv_pools)


def Decoder(*args, **kwargs):
    """bindings/torch_decode.cu:14-81 Decoder (imports torch lazily)."""
    from .decoder import Decoder as _Decoder
    return _Decoder(*args, **kwargs)


__all__ = [
    "_lib", "DecodeParams", "CacheConfig", "PaError", "InvalidArgument", "LengthError",
    "DeviceError", "FP16", "FP8_E4M3", "DecodePlan", "DevicePlan", "PagePool", "PagedKVCache",
    "make_plan", "make_plan_tiled", "paged_decode", "decode_split", "decode_merge",
    "append_quantize", "gather_kv", "stream_read", "stream_read_chunked", "fill_bytes", "tile_tokens", "wave_ctas", "default_ctas",
    "kv_dtype_bytes", "kv_dtype_name", "sm_scale", "kv_pool_stagger", "alloc_kv_pools", "Decoder",
]
