"""MI355X (gfx950) paged flash-decoding: Python side of libpa_decode.so.

`core` mirrors decode.hpp / paged_kv_cache.hpp over the C ABI; `Decoder` is
the reference's torch binding (compiled, `_pa_torch`, with a ctypes twin in
`decoder`). Importing this package does not load the library; the first call
does, and fails loudly if it is missing.
"""

from . import _lib
from ._lib import DecodeParams, CacheConfig, PaError, InvalidArgument, LengthError, DeviceError
from .core import (FP16, FP8_E4M3, DecodePlan, DevicePlan, PagePool, PagedKVCache, make_plan,
                   make_plan_tiled, paged_decode, decode_split, decode_merge, append_quantize,
                   gather_kv, stream_read, stream_read_chunked, fill_bytes, tile_tokens, wave_ctas, default_ctas, kv_dtype_bytes,
                   kv_dtype_name, sm_scale, kv_pool_stagger, alloc_kv_pools)


def Decoder(*args, **kwargs):
    """bindings/torch_decode.cu:14-81 Decoder (imports torch lazily): the
    compiled binding (pa_amd/_pa_torch*.so, built from csrc/pa_torch.cpp) when
    it was built, else the ctypes one (decoder.Decoder); both drive the same
    library and kernels."""
    from .decoder import decoder_class
    return decoder_class()(*args, **kwargs)


__all__ = [
    "_lib", "DecodeParams", "CacheConfig", "PaError", "InvalidArgument", "LengthError",
    "DeviceError", "FP16", "FP8_E4M3", "DecodePlan", "DevicePlan", "PagePool", "PagedKVCache",
    "make_plan", "make_plan_tiled", "paged_decode", "decode_split", "decode_merge",
    "append_quantize", "gather_kv", "stream_read", "stream_read_chunked", "fill_bytes", "tile_tokens", "wave_ctas", "default_ctas",
    "kv_dtype_bytes", "kv_dtype_name", "sm_scale", "kv_pool_stagger", "alloc_kv_pools", "Decoder",
]
