"""Shared helpers for the parity tests (device copies, seeded inputs, cases)."""

from __future__ import annotations

import ctypes
import math

import numpy as np

import oracle
import pa_amd

D = 128
TOL = 2e-3          # max-abs bound against the fp32 CPU oracle (fp16 and dequantized FP8 KV)
FP8_TEST_SCALE = 4.0 / 448.0   # tests/test_paged_decode.cu:79: |x| <= 4 fits

_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipDeviceSynchronize.restype = ctypes.c_int
    return _hip


def d2h(ptr: int, nbytes: int, dtype=np.uint8) -> np.ndarray:
    """Copies nbytes of device memory at ptr into a new numpy array."""
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
    assert hip().hipDeviceSynchronize() == 0
    assert hip().hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0   # hipMemcpyDeviceToHost
    return out


def to_device(a: np.ndarray):
    """numpy array -> torch CUDA tensor with the same bytes."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16))
    elif a.dtype == np.uint8:
        t = torch.from_numpy(a)
    else:
        t = torch.from_numpy(a)
    return t.cuda()


def normal_f16(rng: np.random.Generator, shape) -> np.ndarray:
    """N(0,1) samples rounded to fp16 (RNE), as fp16 bit patterns."""
    return oracle.f32_to_f16_bits(rng.standard_normal(shape, dtype=np.float32))


def dtype_of(fp8: bool) -> int:
    return pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16


def run_cache_case(fp8: bool, hq: int, hkv: int, page_size: int, seq_lens, num_ctas: int = 0,
                   chunk: int = 0, seed: int = 1234, quantized_reference: bool = True,
                   shuffle_seed: int | None = None, threads: int = 8, batched: bool = False):
    """tests/test_paged_decode.cu:50-151 run_case through the C ABI's cache.

    Builds a PagedKVCache, appends per-sequence K/V (whole or round-robin
    chunks; with batched=True each round of chunks is one append_batch call,
    as a decode step grows every sequence at once), decodes, and checks (1)
    every stored byte against the oracle's append (bit-exact block-table
    scatter and FP8 bytes) and (2) the output against the oracle's fp32
    attention over the stored (dequantized) values.
    Returns (max_abs_err, out fp32, plan).
    """
    import torch
    dt = dtype_of(fp8)
    rng = np.random.default_rng(seed)
    B, G = len(seq_lens), hq // hkv
    Ks = [normal_f16(rng, (L, hkv, D)) for L in seq_lens]
    Vs = [normal_f16(rng, (L, hkv, D)) for L in seq_lens]
    q = normal_f16(rng, (B, hq, D))
    pages = [math.ceil(L / page_size) for L in seq_lens]
    scale = FP8_TEST_SCALE if fp8 else 1.0
    cache = pa_amd.PagedKVCache(sum(pages) + 3, page_size, hkv, D, B, max(pages), dt, scale, scale)
    if shuffle_seed is not None:
        cache.shuffle_free_pages(shuffle_seed)
    dK = [to_device(k) for k in Ks]
    dV = [to_device(v) for v in Vs]
    for b in range(B):
        assert cache.admit() == b
    row = hkv * D
    done = [0] * B
    progress = True
    while progress:
        progress = False
        slots, counts, kparts, vparts = [], [], [], []
        for b in range(B):
            n = min(chunk if chunk > 0 else seq_lens[b], seq_lens[b] - done[b])
            if n <= 0:
                continue
            if batched:
                slots.append(b)
                counts.append(n)
                kparts.append(dK[b][done[b]:done[b] + n])
                vparts.append(dV[b][done[b]:done[b] + n])
            else:
                ok = cache.append(b, dK[b].data_ptr() + done[b] * row * 2, dV[b].data_ptr() + done[b] * row * 2, n)
                assert ok
            done[b] += n
            progress = True
        if slots:
            kb, vb = torch.cat(kparts).contiguous(), torch.cat(vparts).contiguous()
            assert cache.append_batch(slots, counts, kb, vb, torch.cuda.current_stream().cuda_stream)
    dq = to_device(q)
    dout = torch.empty((B, hq, D), dtype=torch.float16, device="cuda")
    cache.decode(dq, dout, B, hq, num_ctas)
    torch.cuda.synchronize()
    out = oracle.f16_bits_to_f32(dout.cpu().view(torch.int16).numpy().view(np.uint16))

    p = cache.params()
    eb = 1 if fp8 else 2
    pool_bytes = (sum(pages) + 3) * hkv * page_size * D * eb
    gk = d2h(p.k_cache, pool_bytes)
    gv = d2h(p.v_cache, pool_bytes)
    table = np.zeros((B, max(pages)), dtype=np.int32)
    for b in range(B):
        t = cache.block_table(b)
        assert len(t) == pages[b]
        table[b, : len(t)] = t
    # (1) bit-exact storage: CPU append of the same inputs into the same pages
    ck = np.zeros(pool_bytes, dtype=np.uint8)
    cv = np.zeros(pool_bytes, dtype=np.uint8)
    inv = float(np.float32(1.0) / np.float32(scale))
    for b in range(B):
        _append_all(dt, Ks[b], Vs[b], ck, cv, table[b], hkv, page_size, inv, fp8)
    for b in range(B):
        for h in range(hkv):
            a = oracle.gather_raw(dt, gk.view(np.uint16) if not fp8 else gk, table[b], hkv, D, page_size, h, seq_lens[b])
            c = oracle.gather_raw(dt, ck.view(np.uint16) if not fp8 else ck, table[b], hkv, D, page_size, h, seq_lens[b])
            assert np.array_equal(a, c), f"stored K bytes differ (b={b}, h={h})"
            a = oracle.gather_raw(dt, gv.view(np.uint16) if not fp8 else gv, table[b], hkv, D, page_size, h, seq_lens[b])
            c = oracle.gather_raw(dt, cv.view(np.uint16) if not fp8 else cv, table[b], hkv, D, page_size, h, seq_lens[b])
            assert np.array_equal(a, c), f"stored V bytes differ (b={b}, h={h})"
    # (2) attention over the stored values (or the unquantized fp16 values)
    lens = np.asarray(seq_lens, dtype=np.int32)
    if quantized_reference or not fp8:
        ref = oracle.paged_decode(dt, q, gk.view(np.uint16) if not fp8 else gk,
                                  gv.view(np.uint16) if not fp8 else gv, table, lens, hq, hkv, D, page_size,
                                  scale, scale, threads=threads)
    else:
        fk = np.zeros(pool_bytes * 2 if fp8 else pool_bytes, dtype=np.uint8)
        fv = np.zeros_like(fk)
        for b in range(B):
            _append_all(pa_amd.FP16, Ks[b], Vs[b], fk, fv, table[b], hkv, page_size, 1.0, False)
        ref = oracle.paged_decode(pa_amd.FP16, q, fk.view(np.uint16), fv.view(np.uint16), table, lens, hq, hkv,
                                  D, page_size, threads=threads)
    assert np.all(np.isfinite(out))
    err = float(np.max(np.abs(out - ref)))
    plan = cache.last_plan()
    cache.close()
    return err, out, plan


def _append_all(dt, K, V, ck, cv, bt_row, hkv, page_size, inv, fp8):
    kc = ck if fp8 else ck.view(np.uint16)
    vc = cv if fp8 else cv.view(np.uint16)
    oracle.append(dt, K.reshape(K.shape[0], -1), V.reshape(V.shape[0], -1), kc, vc, bt_row, 0, hkv, D,
                  page_size, inv, inv)


def paged_inputs(batch, seq_lens, hq, hkv, page_size, fp8, seed, keep_sources=False):
    """compare_flashinfer.py:80-97 style inputs: N(0,1) pools filled on the
    device, a random page permutation as block table, per-tensor amax/448
    scales with append-time quantization for FP8. With keep_sources (FP8
    only) the per-row fp16 sources [L][Hkv][D] of K and V come back as a
    seventh value, a list of (k, v) device tensors."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    pages_per = [math.ceil(L / page_size) for L in seq_lens]
    num_pages = sum(pages_per)
    max_pages = max(pages_per)
    perm = torch.randperm(num_pages, device="cuda", generator=g).to(torch.int32)
    table = torch.zeros(batch, max_pages, dtype=torch.int32, device="cuda")
    off = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[off:off + n]
        off += n
    q = torch.randn(batch, hq, D, device="cuda", dtype=torch.float16, generator=g)
    if not fp8:
        k = torch.randn(num_pages, hkv, page_size, D, device="cuda", dtype=torch.float16, generator=g)
        v = torch.randn(num_pages, hkv, page_size, D, device="cuda", dtype=torch.float16, generator=g)
        return q, k, v, table, 1.0, 1.0
    kc = torch.zeros(num_pages, hkv, page_size, D, device="cuda", dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    srcs = []
    for b, L in enumerate(seq_lens):
        srcs.append((torch.randn(L, hkv, D, device="cuda", dtype=torch.float16, generator=g),
                     torch.randn(L, hkv, D, device="cuda", dtype=torch.float16, generator=g)))
    k_scale = max(float(s[0].abs().max()) for s in srcs) / 448.0
    v_scale = max(float(s[1].abs().max()) for s in srcs) / 448.0
    ik = float(np.float32(1.0) / np.float32(k_scale))
    iv = float(np.float32(1.0) / np.float32(v_scale))
    for b, (ks, vs) in enumerate(srcs):
        pa_amd.append_quantize(pa_amd.FP8_E4M3, ks, vs, kc, vc, table[b], 0, seq_lens[b], hkv, D, page_size, ik, iv)
    if keep_sources:
        return q, kc, vc, table, k_scale, v_scale, srcs
    return q, kc, vc, table, k_scale, v_scale


def decoder_case(batch, seq_lens, fp8, page_size=16, hq=32, hkv=8, seed=0, threads=16, rows=None):
    """Decodes the whole batch on the GPU; checks every row against the oracle,
    or only `rows` (a sample, for batches whose full oracle would take minutes)."""
    import torch
    q, k, v, table, ks, vs = paged_inputs(batch, seq_lens, hq, hkv, page_size, fp8, seed)
    dec = pa_amd.Decoder(hq, hkv, D, page_size, fp8)
    lens = torch.tensor(seq_lens, dtype=torch.int32)
    dec.plan(lens, 0)
    out = dec.run(q, k, v, table, lens.cuda(), ks, vs)
    torch.cuda.synchronize()
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    kb = k.view(torch.uint8).cpu().numpy() if fp8 else k.view(torch.int16).cpu().numpy().view(np.uint16)
    vb = v.view(torch.uint8).cpu().numpy() if fp8 else v.view(torch.int16).cpu().numpy().view(np.uint16)
    sel = np.arange(batch) if rows is None else np.asarray(rows)
    qb = q.view(torch.int16).cpu().numpy().view(np.uint16)[sel]
    ref = oracle.paged_decode(dt, qb, kb, vb, table.cpu().numpy()[sel], np.asarray(seq_lens, np.int32)[sel], hq,
                              hkv, D, page_size, ks, vs, threads=threads)
    got = out.float().cpu().numpy()[sel]
    return float(np.max(np.abs(got - ref))), dec
