"""Pins the oracle's append scatter and gather against the closed-form HND
address ((page * Hkv + h) * P + pos % P) * D + d (paged_kv_cache.cu:33-35,
decode_kernels.cuh:175-177), by brute force on tiny pools."""

import numpy as np
import pytest

import oracle


@pytest.mark.parametrize("P,start", [(1, 0), (2, 3), (4, 1), (16, 0), (16, 13)])
def test_append_scatter_closed_form(P, start):
    rng = np.random.default_rng(P + start)
    hkv, D, n = 3, 128, 21
    pages = (start + n + P - 1) // P
    npool = pages + 4
    table = rng.permutation(npool)[:pages].astype(np.int32)
    k = rng.integers(0, 65535, size=(n, hkv * D), dtype=np.uint16)
    v = rng.integers(0, 65535, size=(n, hkv * D), dtype=np.uint16)
    kc = np.zeros(npool * hkv * P * D, np.uint16)
    vc = np.zeros_like(kc)
    oracle.append(0, k, v, kc, vc, table, start, hkv, D, P)
    exp_k = np.zeros_like(kc)
    for i in range(n):
        pos = start + i
        for h in range(hkv):
            base = ((table[pos // P] * hkv + h) * P + pos % P) * D
            exp_k[base: base + D] = k[i, h * D:(h + 1) * D]
    assert np.array_equal(kc, exp_k)
    for h in range(hkv):
        g = oracle.gather_raw(0, vc, table, hkv, D, P, h, start + n)
        assert np.array_equal(g[start:], v[:, h * D:(h + 1) * D])


def test_fp8_append_uses_reciprocal_multiply():
    # paged_kv_cache.cu:21,:130: stored = e4m3(x * fp32(1/scale)), not x / scale.
    scale = np.float32(3.0 / 448.0)
    inv = np.float32(1.0) / scale
    x = np.arange(65536, dtype=np.uint16)
    xf = oracle.f16_bits_to_f32(x)
    finite = np.isfinite(xf)
    n = 512
    kc = np.zeros(n * 128, np.uint8)
    vc = np.zeros_like(kc)
    table = np.arange(n // 16, dtype=np.int32)
    oracle.append(1, x.reshape(n, 128), x.reshape(n, 128), kc, vc, table, 0, 1, 128, 16, float(inv), float(inv))
    exp = oracle.f32_to_e4m3((xf * inv).astype(np.float32))
    assert np.array_equal(kc[finite], exp[finite])


@pytest.mark.parametrize("scale", [1.0, 3.0 / 448.0, 4.0 / 448.0, 4.8125 / 448.0, 5.3271484375 / 448.0, 1e-3])
def test_e4m3_quantize_table_equals_append(scale):
    """The quantize table (one byte per fp16 code at a fixed scale) holds, for
    every one of the 65536 fp16 codes, the byte orc_append stores for that code
    through its address path (one token row of 128 dims per 128 codes), and
    the byte of the scalar encoder applied to the fp32 product."""
    inv = float(np.float32(1.0) / np.float32(scale))
    table = oracle.e4m3_quantize_table(inv)
    x = np.arange(65536, dtype=np.uint16)
    n = 512
    kc = np.zeros(n * 128, np.uint8)
    vc = np.zeros_like(kc)
    pages = np.arange(n // 16, dtype=np.int32)[::-1].copy()     # reversed pages: the scatter matters
    oracle.append(1, x.reshape(n, 128), x.reshape(n, 128), kc, vc, pages, 0, 1, 128, 16, inv, inv)
    stored = oracle.gather_raw(1, kc, pages, 1, 128, 16, 0, n).ravel()
    assert np.array_equal(stored, table)
    sample = x[::97]
    prod = (oracle.f16_bits_to_f32(sample) * np.float32(inv)).astype(np.float32)
    assert np.array_equal(table[sample], oracle.f32_to_e4m3(prod))
