"""Pins the oracle's attention.

* Bit-exact against the reference's own cpu_attention compiled from
  src/attention/cpu/attention.cpp (oracle/_ref), when it was built here.
* The reference's known-answer tests (tests/test_cpu_attention.cpp:7-67).
* The multi-head paged decode against float64 numpy attention on small inputs,
  including the GQA head mapping h = hq / G and slot indirection.
"""

import math

import numpy as np
import pytest

import oracle


def _rand(rng, *shape):
    return rng.uniform(-1, 1, shape).astype(np.float32)


def test_matches_reference_cpu_attention_bitwise():
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(3)
    for T, d in [(1, 128), (7, 8), (300, 128), (2049, 64), (4096, 128)]:
        q, K, V = _rand(rng, d), _rand(rng, T, d), _rand(rng, T, d)
        assert np.array_equal(oracle.cpu_attention(q, K, V), oracle.ref_cpu_attention(q, K, V))


def test_zero_values_give_zero():
    d, T = 8, 16
    out = oracle.cpu_attention(np.full(d, 0.5, np.float32), np.full((T, d), 0.25, np.float32),
                               np.zeros((T, d), np.float32))
    assert np.all(out == 0.0)


def test_uniform_keys_give_column_mean():
    d, T = 8, 16
    V = np.repeat(np.arange(T, dtype=np.float32)[:, None], d, axis=1)
    out = oracle.cpu_attention(np.ones(d, np.float32), np.ones((T, d), np.float32), V)
    assert np.allclose(out, (T - 1) / 2.0, atol=1e-5)


def test_two_token_closed_form():
    q = np.array([10, 0, 0, 0], np.float32)
    K = np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32)
    V = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float32)
    s0, s1 = 10 / math.sqrt(4), 0.0
    w0 = 1 / (1 + math.exp(s1 - s0))
    exp = w0 * V[0] + (1 - w0) * V[1]
    assert np.allclose(oracle.cpu_attention(q, K, V), exp, atol=1e-5)


def _numpy_decode(q, K, V, lens, hq, hkv):
    G = hq // hkv
    out = np.zeros((len(lens), hq, q.shape[-1]))
    for b, L in enumerate(lens):
        for h in range(hq):
            kh = K[b][:L, h // G].astype(np.float64)
            vh = V[b][:L, h // G].astype(np.float64)
            s = kh @ q[b, h].astype(np.float64) / math.sqrt(q.shape[-1])
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ vh
    return out


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("hq,hkv,P", [(8, 8, 16), (8, 2, 3), (16, 4, 1), (8, 1, 5)])
def test_paged_decode_matches_float64(fp8, hq, hkv, P):
    rng = np.random.default_rng(hq * 10 + P)
    D = 128
    lens = [1, 37, 90]
    K = [rng.standard_normal((L, hkv, D)).astype(np.float32) for L in lens]
    V = [rng.standard_normal((L, hkv, D)).astype(np.float32) for L in lens]
    qb = oracle.f32_to_f16_bits(rng.standard_normal((len(lens), hq, D)).astype(np.float32))
    pages = [math.ceil(L / P) for L in lens]
    npages = sum(pages) + 2
    perm = rng.permutation(npages).astype(np.int32)
    table = np.zeros((len(lens) + 1, max(pages) + 1), np.int32)
    slot_ids = np.array([2, 0, 1], np.int32)            # batch row b reads table row slot_ids[b]
    off = 0
    dt = 1 if fp8 else 0
    eb = 1 if fp8 else 2
    kc = np.zeros(npages * hkv * P * D * eb, np.uint8)
    vc = np.zeros_like(kc)
    scale = 4.0 / 448.0 if fp8 else 1.0
    inv = float(np.float32(1) / np.float32(scale))
    Kq, Vq = [], []
    for b, L in enumerate(lens):
        row = table[slot_ids[b]]
        row[: pages[b]] = perm[off: off + pages[b]]
        off += pages[b]
        kb = oracle.f32_to_f16_bits(K[b].reshape(L, -1))
        vb = oracle.f32_to_f16_bits(V[b].reshape(L, -1))
        view = (lambda a: a) if fp8 else (lambda a: a.view(np.uint16))
        oracle.append(dt, kb, vb, view(kc), view(vc), row, 0, hkv, D, P, inv, inv)
        # the values the cache holds, dequantized
        kf = oracle.f16_bits_to_f32(kb)
        vf = oracle.f16_bits_to_f32(vb)
        if fp8:
            kf = oracle.e4m3_to_f32(oracle.f32_to_e4m3(kf * np.float32(inv))) * np.float32(scale)
            vf = oracle.e4m3_to_f32(oracle.f32_to_e4m3(vf * np.float32(inv))) * np.float32(scale)
        Kq.append(kf.reshape(L, hkv, D))
        Vq.append(vf.reshape(L, hkv, D))
    view = (lambda a: a) if fp8 else (lambda a: a.view(np.uint16))
    got = oracle.paged_decode(dt, qb, view(kc), view(vc), table, np.array(lens, np.int32), hq, hkv, D, P,
                              scale, scale, slot_ids=slot_ids, threads=3)
    exp = _numpy_decode(oracle.f16_bits_to_f32(qb), Kq, Vq, lens, hq, hkv)
    assert np.max(np.abs(got - exp)) < 1e-5


@pytest.mark.parametrize("use_reference", [False, True], ids=["restatement", "reference"])
def test_attention_pairs_equal_paged_decode_and_cpu_attention(use_reference):
    """orc_attention_pairs (the threaded loop the CPU baseline times) computes,
    for every (row, query head) pair of a ragged GQA batch, bitwise what
    orc_paged_decode and a direct cpu_attention call compute over the same
    gathered K/V: the pairs reach the right item (h = hq / G), the right length
    and the right output row, whatever the thread count."""
    if use_reference and oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(8)
    hq, hkv, D, P = 16, 4, 128, 16
    lens = [1, 17, 300, 64, 129]
    B = len(lens)
    pages = [-(-L // P) for L in lens]
    npool = sum(pages) + 2
    order = rng.permutation(npool).astype(np.int32)
    table = np.zeros((B, max(pages)), np.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = order[off:off + n]
        off += n
    kc = oracle.f32_to_f16_bits(rng.standard_normal(npool * hkv * P * D).astype(np.float32))
    vc = oracle.f32_to_f16_bits(rng.standard_normal(npool * hkv * P * D).astype(np.float32))
    qb = oracle.f32_to_f16_bits(rng.standard_normal((B, hq, D)).astype(np.float32))
    ref = oracle.paged_decode(0, qb, kc, vc, table, np.asarray(lens, np.int32), hq, hkv, D, P, threads=3)
    K = [oracle.gather_dequant(0, kc, table[b], hkv, D, P, h, lens[b]) for b in range(B) for h in range(hkv)]
    V = [oracle.gather_dequant(0, vc, table[b], hkv, D, P, h, lens[b]) for b in range(B) for h in range(hkv)]
    qf = oracle.f16_bits_to_f32(qb)
    for threads in (1, 5):
        out, secs = oracle.attention_pairs(qf, K, V, lens, hkv, threads=threads, use_reference=use_reference)
        assert secs >= 0.0
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    G = hq // hkv
    for b in range(B):
        for h in range(hq):
            one = oracle.cpu_attention(qf[b, h], K[b * hkv + h // G], V[b * hkv + h // G])
            assert np.array_equal(one.view(np.uint32), ref[b, h].view(np.uint32))
