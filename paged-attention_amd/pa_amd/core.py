"""Python mirror of the reference's decode interface over the C ABI.

Names and argument meanings follow the reference headers:
  decode.hpp:21-66         make_plan / DecodePlan / DevicePlan / paged_decode /
                           tile_tokens / wave_ctas / default_ctas
  paged_kv_cache.hpp:17-93 PagedKVCache
Device memory is passed as torch tensors (or raw integer addresses); every call
runs the HIP kernels of libpa_decode.so on the given (default: current) stream.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import CacheConfig, DecodeParams, InvalidArgument, call, check, load

FP16 = _lib.PA_KV_FP16
FP8_E4M3 = _lib.PA_KV_FP8_E4M3


def _ptr(x) -> int | None:
    """Device/host address of a tensor, ndarray or int (None for None)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)!r}")


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        if torch.cuda.is_available():
            raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)   # no Stream object: ~0.1 us
            if raw is not None:
                return raw(torch.cuda.current_device())
            return torch.cuda.current_stream().cuda_stream
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def kv_dtype_bytes(dtype: int) -> int:
    return load().pa_kv_dtype_bytes(dtype)


def kv_dtype_name(dtype: int) -> str:
    return load().pa_kv_dtype_name(dtype).decode()


def kv_pool_stagger() -> int:
    """Bytes between the end of the K pool and the start of the V pool that
    the library leaves in its own caches (pa_kv_pool_stagger)."""
    return load().pa_kv_pool_stagger()


def alloc_kv_pools(num_pages: int, num_kv_heads: int, page_size: int, head_dim: int, fp8: bool,
                   device=None):
    """K and V pools ([num_pages][num_kv_heads][page_size][head_dim], fp16 or
    E4M3 bytes as uint8) as two views of one allocation, V starting
    kv_pool_stagger() bytes after the end of K: the placement the library's own
    caches use (separately allocated pools tend to share their offset modulo a
    large power of two, which costs a decode step 3-7% on MI355X)."""
    import torch
    elem = 1 if fp8 else 2
    n = num_pages * num_kv_heads * page_size * head_dim
    gap = kv_pool_stagger()
    if gap % elem:
        raise InvalidArgument("pool stagger is not a whole number of elements")
    dt = torch.uint8 if fp8 else torch.float16
    flat = torch.empty(2 * n + gap // elem, dtype=dt, device=device if device is not None else "cuda")
    shape = (num_pages, num_kv_heads, page_size, head_dim)
    return flat[:n].view(shape), flat[n + gap // elem:].view(shape)


def tile_tokens(dtype: int, head_dim: int, group: int) -> int:
    out = ctypes.c_int(0)
    call("pa_tile_tokens", dtype, head_dim, group, ctypes.byref(out))
    return out.value


def wave_ctas(dtype: int, head_dim: int, group: int) -> int:
    out = ctypes.c_int(0)
    call("pa_wave_ctas", dtype, head_dim, group, ctypes.byref(out))
    return out.value


def default_ctas(dtype: int, head_dim: int, group: int) -> int:
    out = ctypes.c_int(0)
    call("pa_default_ctas", dtype, head_dim, group, ctypes.byref(out))
    return out.value


@dataclass
class DecodePlan:
    """decode.hpp:21-27: num_ctas, tile, segments [n,4], cta_seg_begin, item_seg_begin."""

    num_ctas: int
    tile: int
    segments: np.ndarray
    cta_seg_begin: np.ndarray
    item_seg_begin: np.ndarray
    handle: ctypes.c_void_p | None = None   # owning pa_plan*, kept for upload

    @classmethod
    def _from_handle(cls, handle: int, owned: bool) -> "DecodePlan":
        lib = load()
        nseg = lib.pa_plan_num_segments(handle)
        nctas = lib.pa_plan_num_ctas(handle)
        items = lib.pa_plan_num_items(handle)
        seg = np.zeros((nseg, 4), dtype=np.int32)
        cta = np.zeros(nctas + 1, dtype=np.int32)
        itm = np.zeros(items + 1, dtype=np.int32)
        check(lib.pa_plan_copy(handle, seg.ctypes.data, cta.ctypes.data, itm.ctypes.data))
        plan = cls(nctas, lib.pa_plan_tile(handle), seg, cta, itm)
        if owned:
            plan.handle = _PlanHandle(handle)
        return plan

    @property
    def needs_merge(self) -> bool:
        return len(self.segments) > len(self.item_seg_begin) - 1

    @property
    def merge_mode(self) -> int:
        """pa_decode_params.block_merge that DevicePlan.bind sets for this plan:
        0 (merge kernel), 1 (split items merged inside one block), 2 (items
        spanning blocks merged by the split kernel too)."""
        if self.handle is None:
            raise ValueError("plan has no native handle")
        out = ctypes.c_int(0)
        call("pa_plan_merge_mode", self.handle.value, ctypes.byref(out))
        return out.value


class _PlanHandle:
    def __init__(self, h: int):
        self.value = h

    def __del__(self):
        try:
            load().pa_plan_destroy(self.value)
        except Exception:
            pass


def _lens_array(seq_lens) -> np.ndarray:
    if hasattr(seq_lens, "cpu"):
        seq_lens = seq_lens.cpu().numpy()
    return np.ascontiguousarray(np.asarray(seq_lens, dtype=np.int32))


def make_plan(dtype: int, seq_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
              num_ctas: int = 0) -> DecodePlan:
    """decode.cu:65-108 make_plan."""
    lens = _lens_array(seq_lens)
    h = ctypes.c_void_p()
    call("pa_plan_build", dtype, lens.ctypes.data, len(lens), num_q_heads, num_kv_heads, head_dim,
         num_ctas, ctypes.byref(h))
    return DecodePlan._from_handle(h.value, owned=True)


def make_plan_tiled(tile: int, seq_lens, num_kv_heads: int, num_ctas: int) -> DecodePlan:
    """The same cut at an explicit tile and grid (pure host, no device needed)."""
    lens = _lens_array(seq_lens)
    h = ctypes.c_void_p()
    call("pa_plan_build_tiled", tile, lens.ctypes.data, len(lens), num_kv_heads, num_ctas,
         ctypes.byref(h))
    return DecodePlan._from_handle(h.value, owned=True)


class DevicePlan:
    """decode.hpp:44-63: device copy of a plan + partial workspace (RAII)."""

    def __init__(self):
        h = ctypes.c_void_p()
        call("pa_device_plan_create", ctypes.byref(h))
        self._h = h.value

    def upload(self, plan: DecodePlan, group: int, head_dim: int, stream=None) -> None:
        if plan.handle is None:
            raise ValueError("plan has no native handle")
        call("pa_device_plan_upload", self._h, plan.handle.value, group, head_dim, _stream(stream))

    def bind(self, p: DecodeParams) -> None:
        call("pa_device_plan_bind", self._h, ctypes.byref(p))

    def __del__(self):
        try:
            if self._h:
                load().pa_device_plan_destroy(self._h)
        except Exception:
            pass


def paged_decode(dtype: int, p: DecodeParams, stream=None) -> None:
    """decode.cu:158-165: split kernel, then the merge when rows were split."""
    call("pa_decode", dtype, ctypes.byref(p), _stream(stream))


def decode_split(dtype: int, p: DecodeParams, stream=None) -> None:
    call("pa_decode_split", dtype, ctypes.byref(p), _stream(stream))


def decode_merge(dtype: int, p: DecodeParams, stream=None) -> None:
    call("pa_decode_merge", dtype, ctypes.byref(p), _stream(stream))


def append_quantize(dtype: int, k, v, k_cache, v_cache, block_table_row, start_pos: int, n: int,
                    num_kv_heads: int, head_dim: int, page_size: int, inv_k_scale: float = 1.0,
                    inv_v_scale: float = 1.0, stream=None) -> None:
    """paged_kv_cache.cu:25-39 append_kernel (fp16 copy / FP8 quantize + scatter)."""
    call("pa_append_quantize", dtype, _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
         _ptr(block_table_row), start_pos, n, num_kv_heads, head_dim, page_size,
         float(inv_k_scale), float(inv_v_scale), _stream(stream))


def gather_kv(dtype: int, cache, block_table_row, num_kv_heads: int, head_dim: int, page_size: int,
              kv_head: int, length: int, out, stream=None) -> None:
    call("pa_gather_kv", dtype, _ptr(cache), _ptr(block_table_row), num_kv_heads, head_dim,
         page_size, kv_head, length, _ptr(out), _stream(stream))


def stream_read_chunked(buf, nbytes: int, blocks: int, sink, stream=None, threads: int = 512,
                        unroll: int = 16) -> None:
    """Streaming read with one contiguous span per wave (the best read shape)."""
    call("pa_stream_read_chunked", _ptr(buf), nbytes, blocks, threads, unroll, _ptr(sink), _stream(stream))


def stream_read(buf, nbytes: int, blocks: int, sink, stream=None, threads: int = 256, unroll: int = 1,
                nontemporal: bool = False) -> None:
    """bench_decode.cu:70-78 read_kernel (threads=256, unroll=1) and its unrolled variants."""
    call("pa_stream_read_ex", _ptr(buf), nbytes, blocks, threads, unroll, int(nontemporal), _ptr(sink),
         _stream(stream))


def fill_bytes(buf, nbytes: int, value: int, stream=None) -> None:
    """Streaming write of one byte value (a write of known size)."""
    call("pa_fill_bytes", _ptr(buf), nbytes, value, _stream(stream))


class PagePool:
    """Host page allocator + block tables (paged_kv_cache.cu:84-151), no device memory."""

    def __init__(self, num_pages: int, page_size: int, max_slots: int, max_pages_per_slot: int,
                 _handle: int | None = None, _owner=None):
        if _handle is not None:
            self._h, self._owned, self._owner = _handle, False, _owner
            return
        h = ctypes.c_void_p()
        call("pa_pool_create", num_pages, page_size, max_slots, max_pages_per_slot, ctypes.byref(h))
        self._h, self._owned, self._owner = h.value, True, None

    def admit(self) -> int:
        return load().pa_pool_admit(self._h)

    def reserve(self, slot: int, n: int) -> tuple[bool, int, int]:
        ok, first, num = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        call("pa_pool_reserve", self._h, slot, n, ctypes.byref(ok), ctypes.byref(first),
             ctypes.byref(num))
        return bool(ok.value), first.value, num.value

    def reserve_batch(self, slots, counts) -> bool:
        """reserve(slots[i], counts[i]) for every i in order, all-or-nothing."""
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        counts = np.ascontiguousarray(counts, dtype=np.int32)
        if slots.shape != counts.shape or slots.ndim != 1:
            raise ValueError("slots and counts must be 1-D of one length")
        ok = ctypes.c_int()
        call("pa_pool_reserve_batch", self._h, slots.ctypes.data, counts.ctypes.data, slots.size,
             ctypes.byref(ok))
        return bool(ok.value)

    def release(self, slot: int) -> None:
        call("pa_pool_release", self._h, slot)

    def shuffle_free_pages(self, seed: int) -> None:
        load().pa_pool_shuffle_free_pages(self._h, seed)

    def free_pages(self) -> int:
        return load().pa_pool_free_pages(self._h)

    def seq_len(self, slot: int) -> int:
        return load().pa_pool_seq_len(self._h, slot)

    def occupied(self, slot: int) -> bool:
        return bool(load().pa_pool_occupied(self._h, slot))

    def max_seq_len(self) -> int:
        return load().pa_pool_max_seq_len(self._h)

    def block_table(self, slot: int) -> np.ndarray:
        n = load().pa_pool_num_pages_of(self._h, slot)
        out = np.zeros(n, dtype=np.int32)
        call("pa_pool_block_table", self._h, slot, out.ctypes.data, n)
        return out

    def __del__(self):
        try:
            if self._owned and self._h:
                load().pa_pool_destroy(self._h)
        except Exception:
            pass


class PagedKVCache:
    """paged_kv_cache.hpp:17-93: HND page pool on the device, free list, block
    tables, append-time FP8 quantization, plan/run/decode."""

    def __init__(self, num_pages: int, page_size: int, num_kv_heads: int, head_dim: int,
                 max_slots: int, max_pages_per_slot: int, dtype: int = FP16,
                 k_scale: float = 1.0, v_scale: float = 1.0):
        self.cfg = CacheConfig(num_pages, page_size, num_kv_heads, head_dim, max_slots,
                               max_pages_per_slot, dtype, k_scale, v_scale)
        h = ctypes.c_void_p()
        call("pa_cache_create", ctypes.byref(self.cfg), ctypes.byref(h))
        self._h = h.value
        self.pool = PagePool(0, 0, 0, 0, _handle=load().pa_cache_pool(self._h), _owner=self)

    @staticmethod
    def bytes_per_page(cfg: CacheConfig) -> int:
        return load().pa_cache_bytes_per_page(ctypes.byref(cfg))

    @staticmethod
    def pages_for_budget(cfg: CacheConfig, budget_bytes: int) -> int:
        return load().pa_cache_pages_for_budget(ctypes.byref(cfg), budget_bytes)

    def admit(self) -> int:
        return load().pa_cache_admit(self._h)

    def append(self, slot: int, k, v, n: int, stream=None) -> bool:
        done = ctypes.c_int(0)
        call("pa_cache_append", self._h, slot, _ptr(k), _ptr(v), n, _stream(stream), ctypes.byref(done))
        return bool(done.value)

    def append_batch(self, slots, counts, k, v, stream=None) -> bool:
        """Appends counts[i] tokens to slots[i] for every i in one copy + one
        kernel; k / v hold the tokens concatenated in entry order
        ([sum(counts)][Hkv][D] fp16, device). All-or-nothing on pages."""
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        counts = np.ascontiguousarray(counts, dtype=np.int32)
        if slots.shape != counts.shape or slots.ndim != 1:
            raise ValueError("slots and counts must be 1-D of one length")
        done = ctypes.c_int(0)
        call("pa_cache_append_batch", self._h, slots.ctypes.data, counts.ctypes.data, slots.size,
             _ptr(k), _ptr(v), _stream(stream), ctypes.byref(done))
        return bool(done.value)

    def release(self, slot: int) -> None:
        call("pa_cache_release", self._h, slot)

    def shuffle_free_pages(self, seed: int) -> None:
        load().pa_cache_shuffle_free_pages(self._h, seed)

    def params(self) -> DecodeParams:
        p = DecodeParams()
        call("pa_cache_params", self._h, ctypes.byref(p))
        return p

    def plan(self, slots, num_q_heads: int, num_ctas: int = 0, stream=None) -> None:
        s = np.ascontiguousarray(np.asarray(slots, dtype=np.int32))
        call("pa_cache_plan", self._h, s.ctypes.data, len(s), num_q_heads, num_ctas, _stream(stream))

    def run(self, q, out, stream=None) -> None:
        call("pa_cache_run", self._h, _ptr(q), _ptr(out), _stream(stream))

    def decode(self, q, out, batch: int, num_q_heads: int, num_ctas: int = 0, stream=None) -> None:
        call("pa_cache_decode", self._h, _ptr(q), _ptr(out), batch, num_q_heads, num_ctas,
             _stream(stream))

    def last_plan(self) -> DecodePlan:
        return DecodePlan._from_handle(load().pa_cache_last_plan(self._h), owned=False)

    def seq_len(self, slot: int) -> int:
        return self.pool.seq_len(slot)

    def occupied(self, slot: int) -> bool:
        return self.pool.occupied(slot)

    def free_pages(self) -> int:
        return self.pool.free_pages()

    def max_seq_len(self) -> int:
        return self.pool.max_seq_len()

    def total_bytes(self) -> int:
        return load().pa_cache_total_bytes(self._h)

    def config(self) -> CacheConfig:
        return self.cfg

    def block_table(self, slot: int) -> np.ndarray:
        return self.pool.block_table(slot)

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().pa_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sm_scale(head_dim: int) -> float:
    """1/sqrt(head_dim) rounded to fp32, as the reference computes it."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


__all__ = [
    "FP16", "FP8_E4M3", "DecodeParams", "CacheConfig", "DecodePlan", "DevicePlan", "PagePool",
    "PagedKVCache", "make_plan", "make_plan_tiled", "paged_decode", "decode_split", "decode_merge",
    "append_quantize", "gather_kv", "stream_read", "stream_read_chunked", "fill_bytes", "tile_tokens", "wave_ctas", "default_ctas",
    "kv_dtype_bytes", "kv_dtype_name", "sm_scale",
]
