"""CPU oracle of the paged flash-decoding path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline). The product
library (libpa_decode.so) never calls it.

Wraps oracle/_build/libpa_oracle.so (plain C, see pa_oracle.h for the reference
lines each function restates) and, when it was built from the reference tree,
oracle/_ref/libref_cpu_attention.so (the reference's own cpu_attention,
src/attention/cpu/attention.cpp:14-34, compiled unchanged).

Pinning (what checks each function; the tests are named in parentheses):
  f16 codec        numpy float16 over all 65536 codes and random floats
                   (test_oracle_codecs)
  e4m3 codec       torch.float8_e4m3fn table of all 256 codes and torch's
                   encoder for |x| < 464, golden fixture tests/golden/e4m3_*.npy
                   (test_oracle_codecs)
  cpu_attention    bit-exact against the reference's compiled cpu_attention
                   (oracle/_ref) and its known-answer tests
                   (tests/test_cpu_attention.cpp:7-67) (test_oracle_attention)
  paged_decode     float64 numpy attention on tiny inputs, GQA mapping and
                   permutation invariance (test_oracle_attention)
  append/gather    closed-form address on brute-force tiny pools (test_oracle_paging)
  e4m3 table       equal to orc_append's FP8 store for all 65536 fp16 codes at
                   several scales (test_oracle_paging)
  attention_pairs  every (row, query head) pair equal to paged_decode and to
                   cpu_attention on the same gathered inputs, with and without
                   the reference's compiled cpu_attention (test_oracle_attention)
  make_plan        68 (ctas, segments) rows of the reference's results/*.csv,
                   fixture tests/golden/planner_rows.csv (test_planner)
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "_build" / "libpa_oracle.so"
REF_LIB = HERE / "_ref" / "libref_cpu_attention.so"

_lib: ctypes.CDLL | None = None
_ref: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


def build() -> None:
    """Compiles the oracle (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if pathlib.Path(os.environ.get("PA_REFERENCE", "/root/reference")).joinpath(
            "src/attention/cpu/attention.cpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.orc_f16_to_f32.restype = _F
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [_F]
        L.orc_e4m3_to_f32.restype = _F
        L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_f32_to_e4m3.restype = ctypes.c_uint8
        L.orc_f32_to_e4m3.argtypes = [_F]
        L.orc_f32_to_f16_array.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_f16_to_f32_array.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_append.argtypes = [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F]
        L.orc_e4m3_quantize_table.argtypes = [_F, _P]
        L.orc_gather_raw.argtypes = [_I, _P, _P, _I, _I, _I, _I, _I, _P]
        L.orc_gather_dequant.argtypes = [_I, _P, _P, _I, _I, _I, _I, _I, _F, _P]
        L.orc_cpu_attention.argtypes = [_P, _P, _P, _P, _I, _I]
        L.orc_paged_decode.argtypes = [_I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P, _I]
        L.orc_attention_pairs.restype = ctypes.c_double
        L.orc_attention_pairs.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I]
        L.orc_make_plan.restype = _I
        L.orc_make_plan.argtypes = [_I, _P, _I, _I, _I, _P, _I, _P, _I, _P, ctypes.POINTER(_I)]
        _lib = L
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's compiled cpu_attention, or None if it was not built."""
    global _ref
    if _ref is None and REF_LIB.exists():
        R = ctypes.CDLL(str(REF_LIB))
        fn = getattr(R, "_Z13cpu_attentionPKfS0_S0_Pfii")
        fn.argtypes = [_P, _P, _P, _P, _I, _I]
        fn.restype = None
        _ref = R
    return _ref


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(h.ctypes.data, out.ctypes.data, h.size)
    return out


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.orc_e4m3_to_f32(int(c)) for c in np.asarray(codes).ravel()],
                    dtype=np.float32).reshape(np.shape(codes))


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.asarray(x, dtype=np.float32)
    return np.array([L.orc_f32_to_e4m3(float(v)) for v in x.ravel()], dtype=np.uint8).reshape(x.shape)


def append(dtype: int, k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
           bt_row: np.ndarray, start_pos: int, hkv: int, hd: int, page_size: int,
           inv_k: float = 1.0, inv_v: float = 1.0) -> None:
    """In-place CPU append into numpy pools (uint16 for fp16, uint8 for fp8)."""
    k, v = _c(k, np.uint16), _c(v, np.uint16)
    bt = _c(bt_row, np.int32)
    n = k.shape[0]
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    lib().orc_append(dtype, k.ctypes.data, v.ctypes.data, k_cache.ctypes.data, v_cache.ctypes.data,
                     bt.ctypes.data, start_pos, n, hkv, hd, page_size, inv_k, inv_v)


def e4m3_quantize_table(inv_scale: float) -> np.ndarray:
    """uint8[65536]: the E4M3 byte orc_append stores for each fp16 code at
    reciprocal scale inv_scale (index the table with the fp16 bit patterns)."""
    out = np.zeros(65536, dtype=np.uint8)
    lib().orc_e4m3_quantize_table(float(inv_scale), out.ctypes.data)
    return out


def gather_raw(dtype: int, cache: np.ndarray, bt_row: np.ndarray, hkv: int, hd: int,
               page_size: int, h: int, length: int) -> np.ndarray:
    out = np.zeros((length, hd), dtype=np.uint16 if dtype == 0 else np.uint8)
    bt = _c(bt_row, np.int32)
    lib().orc_gather_raw(dtype, cache.ctypes.data, bt.ctypes.data, hkv, hd, page_size, h, length,
                         out.ctypes.data)
    return out


def gather_dequant(dtype: int, cache: np.ndarray, bt_row: np.ndarray, hkv: int, hd: int,
                   page_size: int, h: int, length: int, scale: float = 1.0) -> np.ndarray:
    out = np.zeros((length, hd), dtype=np.float32)
    bt = _c(bt_row, np.int32)
    lib().orc_gather_dequant(dtype, cache.ctypes.data, bt.ctypes.data, hkv, hd, page_size, h,
                             length, scale, out.ctypes.data)
    return out


def cpu_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    q, K, V = _c(q, np.float32), _c(K, np.float32), _c(V, np.float32)
    T, d = K.shape
    out = np.zeros(d, dtype=np.float32)
    lib().orc_cpu_attention(q.ctypes.data, K.ctypes.data, V.ctypes.data, out.ctypes.data, T, d)
    return out


def ref_cpu_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    """The reference's own compiled cpu_attention (requires oracle/_ref)."""
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref was not built")
    q, K, V = _c(q, np.float32), _c(K, np.float32), _c(V, np.float32)
    T, d = K.shape
    out = np.zeros(d, dtype=np.float32)
    R._Z13cpu_attentionPKfS0_S0_Pfii(q.ctypes.data, K.ctypes.data, V.ctypes.data, out.ctypes.data, T, d)
    return out


def paged_decode(dtype: int, q_bits: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                 block_table: np.ndarray, seq_lens: np.ndarray, num_q_heads: int,
                 num_kv_heads: int, head_dim: int, page_size: int, k_scale: float = 1.0,
                 v_scale: float = 1.0, slot_ids: np.ndarray | None = None,
                 threads: int = 1) -> np.ndarray:
    """fp32 reference output [batch][num_q_heads][head_dim] over numpy pools."""
    q_bits = _c(q_bits, np.uint16)
    bt = _c(block_table, np.int32)
    lens = _c(seq_lens, np.int32)
    batch = len(lens)
    sid = None if slot_ids is None else _c(slot_ids, np.int32)
    out = np.zeros((batch, num_q_heads, head_dim), dtype=np.float32)
    lib().orc_paged_decode(dtype, q_bits.ctypes.data, k_cache.ctypes.data, v_cache.ctypes.data,
                           bt.ctypes.data, bt.shape[1], None if sid is None else sid.ctypes.data,
                           lens.ctypes.data, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                           k_scale, v_scale, out.ctypes.data, threads)
    return out


def attention_pairs(q: np.ndarray, K: list, V: list, seq_lens, num_kv_heads: int,
                    threads: int = 1, use_reference: bool = False) -> tuple[np.ndarray, float]:
    """Runs cpu_attention for every (row, query head) pair over gathered fp32
    K/V (one [len][d] array per (row, kv head) item) on `threads` threads.

    use_reference=True calls the reference's own compiled cpu_attention
    (oracle/_ref); otherwise the restatement. Returns (out [B][Hq][d], seconds
    of the threaded loop)."""
    q = _c(q, np.float32)
    B, hq, d = q.shape
    lens = _c(np.asarray(seq_lens), np.int32)
    items = B * num_kv_heads
    assert len(K) == items and len(V) == items
    Ks = [_c(k, np.float32) for k in K]
    Vs = [_c(v, np.float32) for v in V]
    kp = (ctypes.c_void_p * items)(*[k.ctypes.data for k in Ks])
    vp = (ctypes.c_void_p * items)(*[v.ctypes.data for v in Vs])
    fn = None
    if use_reference:
        R = ref_lib()
        if R is None:
            raise RuntimeError("oracle/_ref was not built")
        fn = ctypes.cast(R._Z13cpu_attentionPKfS0_S0_Pfii, ctypes.c_void_p).value
    out = np.zeros((B, hq, d), dtype=np.float32)
    secs = lib().orc_attention_pairs(fn, q.ctypes.data, ctypes.addressof(kp), ctypes.addressof(vp),
                                     lens.ctypes.data, B, hq, num_kv_heads, d, out.ctypes.data, threads)
    return out, float(secs)


def make_plan(tile: int, seq_lens, num_kv_heads: int, requested: int):
    """Returns (num_ctas, segments [n,4], cta_seg_begin, item_seg_begin)."""
    lens = _c(np.asarray(seq_lens), np.int32)
    batch = len(lens)
    total = int(sum((int(l) + tile - 1) // tile for l in lens)) * num_kv_heads
    seg_cap = total + requested + 8
    segs = np.zeros((seg_cap, 4), dtype=np.int32)
    cta = np.zeros(requested + 2, dtype=np.int32)
    item = np.zeros(batch * num_kv_heads + 1, dtype=np.int32)
    nctas = _I(0)
    n = lib().orc_make_plan(tile, lens.ctypes.data, batch, num_kv_heads, requested, segs.ctypes.data,
                            seg_cap, cta.ctypes.data, len(cta), item.ctypes.data, ctypes.byref(nctas))
    if n < 0:
        raise ValueError("orc_make_plan rejected the input")
    return nctas.value, segs[:n].copy(), cta[: nctas.value + 1].copy(), item
