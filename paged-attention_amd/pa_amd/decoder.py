"""The torch binding's `Decoder` (bindings/torch_decode.cu:14-81), same signature:

    dec = Decoder(num_q_heads, num_kv_heads, head_dim, page_size, fp8)
    dec.plan(seq_lens_cpu_int32, num_ctas=0)
    out = dec.run(q, k_cache, v_cache, block_table, seq_lens_dev, k_scale, v_scale)
    dec.num_ctas, dec.num_segments

It runs libpa_decode.so's HIP kernels on the current torch stream. Argument
checks raise RuntimeError, as TORCH_CHECK does in the reference.

Two implementations: the compiled extension `pa_amd._pa_torch` (csrc/pa_torch.cpp,
built by build.py's build_torch_ext; the one `pa_amd.Decoder` returns when it
was built) and this module's ctypes class, which needs no build against torch.
"""

from __future__ import annotations

import ctypes

import torch

from . import core
from ._lib import DecodeParams, check, load


# The current stream's raw handle without building a torch.cuda.Stream object
# (that costs ~2.5 us a call, a quarter of a small decode step); the public
# call is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(device_index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def _require(cond: bool, msg: str = "Expected condition to hold") -> None:
    if not cond:
        raise RuntimeError(msg)


class Decoder:
    def __init__(self, num_q_heads: int, num_kv_heads: int, head_dim: int, page_size: int, fp8: bool):
        self._hq = int(num_q_heads)
        self._hkv = int(num_kv_heads)
        self._dim = int(head_dim)
        self._page = int(page_size)
        self._dtype = core.FP8_E4M3 if fp8 else core.FP16
        self._batch = 0
        self._table_cols = 0   # block-table columns the plan's longest row needs
        self._plan: core.DecodePlan | None = None
        self._device_plan = core.DevicePlan()
        # The launch parameters that do not change between run() calls of one
        # plan (shapes, scale, the bound device plan), filled by plan(); run()
        # copies them and sets the tensors. Keeps a small decode host-cheap.
        self._params: DecodeParams | None = None
        self._elem = 2 if self._dtype == core.FP16 else 1
        self._cache_shape = (self._hkv, self._page, self._dim)

    # torch_decode.cu:21-27
    def plan(self, seq_lens: torch.Tensor, num_ctas: int = 0) -> None:
        _require(seq_lens.device.type == "cpu" and seq_lens.dtype == torch.int32,
                 "seq_lens must be a CPU int32 tensor")
        lens = seq_lens.contiguous().numpy()
        self._plan = core.make_plan(self._dtype, lens, self._hq, self._hkv, self._dim, num_ctas)
        self._table_cols = int((int(lens.max()) + self._page - 1) // self._page) if lens.size else 0
        self._device_plan.upload(self._plan, self._hq // self._hkv, self._dim,
                                 torch.cuda.current_stream())
        self._batch = int(lens.shape[0])
        p = DecodeParams()
        p.slot_ids = None
        p.batch = self._batch
        p.num_q_heads = self._hq
        p.num_kv_heads = self._hkv
        p.head_dim = self._dim
        p.page_size = self._page
        p.sm_scale = core.sm_scale(self._dim)
        self._device_plan.bind(p)
        self._params = p

    # torch_decode.cu:31-59
    def run(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
            block_table: torch.Tensor, seq_lens_dev: torch.Tensor, k_scale: float,
            v_scale: float) -> torch.Tensor:
        _require(q.is_cuda and q.dtype == torch.float16 and q.is_contiguous(),
                 "q must be a contiguous CUDA fp16 tensor")
        _require(k_cache.is_contiguous() and v_cache.is_contiguous() and block_table.is_contiguous(),
                 "caches and block_table must be contiguous")
        _require(self._params is not None and q.size(0) == self._batch, "q batch does not match the plan")
        _require(block_table.dtype == torch.int32, "block_table must be int32")
        # Shape checks beyond the reference's: a mismatch here would otherwise
        # become out-of-range device reads.
        _require(q.shape[1:] == (self._hq, self._dim), "q must be [batch, num_q_heads, head_dim]")
        for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
            _require(c.is_cuda and c.dim() == 4 and c.shape[1:] == self._cache_shape
                     and c.element_size() == self._elem,
                     f"{name} must be a CUDA [pages, num_kv_heads, page_size, head_dim] tensor of "
                     f"{'fp16' if self._elem == 2 else 'one-byte FP8'} elements")
        _require(block_table.is_cuda and block_table.dim() == 2 and block_table.size(0) >= self._batch
                 and block_table.size(1) >= self._table_cols,
                 "block_table must be a CUDA [batch, >= ceil(max seq_len / page_size)] tensor")
        _require(seq_lens_dev.is_cuda and seq_lens_dev.dtype == torch.int32, "seq_lens must be a CUDA int32 tensor")
        out = torch.empty_like(q)
        p = DecodeParams.from_buffer_copy(self._params)
        p.q = q.data_ptr()
        p.out = out.data_ptr()
        p.k_cache = k_cache.data_ptr()
        p.v_cache = v_cache.data_ptr()
        p.block_table = block_table.data_ptr()
        p.seq_lens = seq_lens_dev.data_ptr()
        p.block_table_stride = block_table.size(1)
        p.k_scale = float(k_scale)
        p.v_scale = float(v_scale)
        check(load().pa_decode(self._dtype, ctypes.byref(p), _current_stream(q.get_device())))
        return out

    @property
    def num_ctas(self) -> int:
        return self._plan.num_ctas if self._plan is not None else 0

    @property
    def num_segments(self) -> int:
        return len(self._plan.segments) if self._plan is not None else 0


_compiled = None


def decoder_class():
    """The compiled binding's Decoder class if its module was built, else this
    module's ctypes Decoder. A built module that fails to import raises. With
    PA_DECODE_LIB naming another library build, the ctypes Decoder (the
    compiled module is linked against the in-tree library)."""
    global _compiled
    if _compiled is None:
        import os
        from ._lib import PKG_DIR, _init_torch_device_state
        if "PA_DECODE_LIB" not in os.environ and any((PKG_DIR / "pa_amd").glob("_pa_torch*.so")):
            _init_torch_device_state()     # torch's HIP state before the library loads
            from . import _pa_torch
            _compiled = _pa_torch.Decoder
        else:
            _compiled = False
    return _compiled or Decoder
