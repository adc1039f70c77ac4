"""The five benchmark configurations (C1-C5) through the torch `Decoder` binding
(bindings/torch_decode.cu:14-81): C1-C5 at full size against the oracle,
config 2's page-size sweep at full size (bitwise equal across page sizes, the
contiguous point against the oracle), config 3's stored FP8 bytes at its own
amax/448 scales, a full-size placement-invariance check, and the binding's
argument checks.
"""

from __future__ import annotations

import numpy as np
import pytest

import pa_amd
import oracle
from helpers import D, TOL, decoder_case, paged_inputs

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu_device")]

DTYPES = [False, True]   # fp8?
IDS = ["fp16", "fp8"]


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_decoder_binding_config1(fp8):
    """Config C1 shape (4 x 1024, P=16, scattered) via the torch_decode
    `Decoder` signature."""
    err, dec = decoder_case(4, [1024] * 4, fp8)
    assert dec.num_ctas > 0 and dec.num_segments >= 32
    assert err < TOL, err

def test_decoder_full_size_config2():
    """Config C2 at full size: 32 x 8192 fp16, 16-token scattered pages."""
    err, _ = decoder_case(32, [8192] * 32, False, threads=16)
    assert err < TOL, err

@pytest.mark.parametrize("batch,length,hq,hkv,fp8", [
    (32, 8192, 4, 1, False),     # C2 sharded over 8 GPUs by kv head: one GPU's share
    (4, 8192, 32, 8, False),     # C2 sharded by row
    (64, 8192, 4, 1, True),      # C3 sharded by kv head
    (1, 16384, 32, 8, True),     # C5 FP8 sharded by tokens (one eighth of the sequence)
], ids=["c2_heads8", "c2_rows8", "c3_heads8", "c5fp8_tokens8"])
def test_decoder_shard_shapes(batch, length, hq, hkv, fp8):
    """One GPU's share of an 8-way sharded BASELINE step at its real shape
    (the shapes the sharding design is timed at), against the oracle: rows
    cut over 4 or 8 blocks and merged across them in the split kernel, or
    over 32 blocks and merged by the merge kernel."""
    err, dec = decoder_case(batch, [length] * batch, fp8, hq=hq, hkv=hkv, threads=16)
    assert dec.num_segments > batch * hkv   # split rows
    assert err < TOL, err

@pytest.mark.parametrize("hq", [8, 16, 64], ids=["g1", "g2", "g8"])
@pytest.mark.parametrize("fp8", [False, True], ids=["fp16", "fp8"])
def test_decoder_full_size_gqa_groups(hq, fp8):
    """C2's batch and length (32 x 8192, 8 kv heads, 16-token scattered
    pages) with the other GQA groups (1, 2, 8 query heads per kv head; C2
    itself is 4), fp16 and FP8, against the oracle: the shapes timed beside
    C2 for the group sweep."""
    err, _ = decoder_case(32, [8192] * 32, fp8, hq=hq, hkv=8, threads=16)
    assert err < TOL, err

def test_decoder_full_size_config3():
    """Config C3 at full size: 64 x 8192, FP8 E4M3 (amax/448 scales,
    quantized by the append kernel), 16-token scattered pages."""
    err, _ = decoder_case(64, [8192] * 64, True, threads=16)
    assert err < TOL, err

def test_decoder_full_size_config4_all_rows():
    """Config C4 at full size (128 ragged rows, L ~ U[128, 16384],
    seed 4, about 4.3 GB of KV) decoded in one batch; every row against the
    oracle. Rows split across blocks go through the merge kernel."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=128)]
    err, dec = decoder_case(128, lens, False, threads=16)
    assert dec.num_segments >= 128 * 8
    assert err < TOL, err

def test_decoder_ragged_config4_subset():
    """Config C4's ragged lengths (U[128, 16384] from a seed), first 16 rows."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=16)]
    err, _ = decoder_case(len(lens), lens, False, threads=16)
    assert err < TOL, err

def test_decoder_long_context_config5_fp16():
    """Config C5 (1 x 131072), fp16 KV."""
    err, dec = decoder_case(1, [131072], False, threads=8)
    assert dec.num_segments > 8 * 64
    assert err < TOL, err

def test_decoder_long_context_config5_fp8():
    """Config C5 (1 x 131072), FP8 KV: hundreds of splits per row."""
    err, dec = decoder_case(1, [131072], True, threads=8)
    assert dec.num_segments > 8 * 64
    assert err < TOL, err

def test_full_size_output_invariant_under_page_placement():
    """At config 2's full size the output is bitwise the same for two
    different page permutations (the plan and tile order do not depend on
    placement), a size-independent check of block-table resolution."""
    import torch
    outs = []
    for seed in (0, 1):
        g = torch.Generator(device="cuda").manual_seed(123)
        n = 32 * 512
        k = torch.randn(n, 8, 16, D, device="cuda", dtype=torch.float16, generator=g)
        v = torch.randn(n, 8, 16, D, device="cuda", dtype=torch.float16, generator=g)
        q = torch.randn(32, 32, D, device="cuda", dtype=torch.float16, generator=g)
        logical = torch.arange(n, device="cuda", dtype=torch.int32).view(32, 512)
        perm = torch.randperm(n, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed))
        perm = perm.to(torch.int32)
        kp, vp = torch.empty_like(k), torch.empty_like(v)
        kp[perm.long()] = k                      # logical page i lives at physical page perm[i]
        vp[perm.long()] = v
        table = perm[logical.reshape(-1).long()].view(32, 512).contiguous()
        dec = pa_amd.Decoder(32, 8, D, 16, False)
        lens = torch.full((32,), 8192, dtype=torch.int32)
        dec.plan(lens, 0)
        outs.append(dec.run(q, kp, vp, table, lens.cuda(), 1.0, 1.0).view(torch.int16).cpu().numpy())
        del k, v, kp, vp
    assert np.array_equal(outs[0], outs[1])

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_alloc_kv_pools_decode_bitwise_equal(fp8):
    """Pools laid out by alloc_kv_pools (one allocation, V a gap after K) hold
    the same pages as separately allocated pools and decode bitwise equal."""
    import torch
    lens = [3000, 1, 777, 4096]
    q, k, v, table, ks, vs = paged_inputs(len(lens), lens, 32, 8, 16, fp8, seed=21)
    kp, vp = pa_amd.alloc_kv_pools(k.shape[0], 8, 16, D, fp8)
    assert vp.data_ptr() - kp.data_ptr() == k.numel() * k.element_size() + pa_amd.kv_pool_stagger()
    kp.copy_(k.view(kp.dtype))
    vp.copy_(v.view(vp.dtype))
    dec = pa_amd.Decoder(32, 8, D, 16, fp8)
    t = torch.tensor(lens, dtype=torch.int32)
    dec.plan(t, 0)
    a = dec.run(q, k, v, table, t.cuda(), ks, vs)
    b = dec.run(q, kp, vp, table, t.cuda(), ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_compiled_and_ctypes_decoders_agree(fp8):
    """pa_amd.Decoder is the compiled binding (csrc/pa_torch.cpp); the ctypes
    Decoder drives the same library: same plans, bitwise the same outputs,
    RuntimeError for the same bad inputs."""
    import torch
    from pa_amd import decoder as ctypes_decoder
    from pa_amd._pa_torch import Decoder as Compiled
    lens = [1024, 3, 5000, 77]
    q, k, v, table, ks, vs = paged_inputs(len(lens), lens, 32, 8, 16, fp8, seed=31)
    t = torch.tensor(lens, dtype=torch.int32)
    outs = []
    for cls in (Compiled, ctypes_decoder.Decoder):
        dec = cls(32, 8, D, 16, fp8)
        dec.plan(t, 0)
        outs.append((dec.run(q, k, v, table, t.cuda(), ks, vs), dec.num_ctas, dec.num_segments))
        with pytest.raises(RuntimeError):
            dec.run(q[:1].contiguous(), k, v, table, t.cuda(), ks, vs)
        with pytest.raises(RuntimeError):
            dec.plan(t.long())
    torch.cuda.synchronize()
    assert isinstance(pa_amd.Decoder(32, 8, D, 16, fp8), Compiled)
    assert outs[0][1:] == outs[1][1:]
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))


def test_decoder_rejects_inconsistent_inputs():
    """Decoder.run raises RuntimeError (the reference's TORCH_CHECK) for inputs
    whose shapes or types do not match the plan, before any launch."""
    import torch
    q, k, v, table, ks, vs = paged_inputs(2, [40, 17], 32, 8, 16, False, 0)
    dec = pa_amd.Decoder(32, 8, D, 16, False)
    lens = torch.tensor([40, 17], dtype=torch.int32)
    dec.plan(lens, 0)
    good = dict(q=q, k_cache=k, v_cache=v, block_table=table, seq_lens_dev=lens.cuda(), k_scale=1.0, v_scale=1.0)
    dec.run(**good)
    bad = [dict(q=q.float()), dict(q=q[:1].contiguous()), dict(q=q.view(2, 8, 4 * D)),
           dict(k_cache=k.view(-1, 8, 8, D)), dict(v_cache=v.view(torch.uint8)), dict(block_table=table[:, :2].contiguous()),
           dict(block_table=table.long()), dict(seq_lens_dev=lens), dict(k_cache=k.cpu())]
    for change in bad:
        with pytest.raises(RuntimeError):
            dec.run(**{**good, **change})
    torch.cuda.synchronize()


def _paged_layout(logical, page_size, perm):
    """[B][H][L][D] logical K or V -> (pool [B * L / P][H][P][D], table [B][L / P]):
    logical page i of the batch (row-major over rows, then pages) lives at
    physical page perm[i]."""
    import torch
    B, H, L, Dd = logical.shape
    npp = L // page_size
    pages = logical.view(B, H, npp, page_size, Dd).permute(0, 2, 1, 3, 4).reshape(B * npp, H, page_size, Dd)
    pool = torch.empty_like(pages)
    pool[perm.long()] = pages
    return pool, perm.view(B, npp).contiguous()


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_full_size_config2_page_size_sweep_bitwise(fp8):
    """Config 2's page-size sweep at full size (32 x 8192, results/h100_pagesize.csv:2-11,
    tests/test_paged_decode.cu:171-180): the same q/K/V laid out in pages of
    4, 8, 16, 32, 64 and 8192 tokens (8192 = one page per sequence, the
    contiguous point), each under its own seeded page permutation, decode to
    bitwise the same output (every load path: staged small pages, 16-token
    runs, whole-sequence pages); the contiguous layout is also checked against
    the oracle. FP8 uses random finite E4M3 codes at scale 4/448."""
    import torch
    B, L, hq, hkv = 32, 8192, 32, 8
    g = torch.Generator(device="cuda").manual_seed(71)
    if fp8:
        def codes():
            c = torch.randint(0, 0x7f, (B, hkv, L, D), device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
            return c | (torch.randint(0, 2, c.shape, device="cuda", generator=g, dtype=torch.int32).to(torch.uint8) << 7)
        klog, vlog = codes(), codes()
        ks = vs = 4.0 / 448.0
    else:
        klog = torch.randn((B, hkv, L, D), device="cuda", dtype=torch.float16, generator=g)
        vlog = torch.randn((B, hkv, L, D), device="cuda", dtype=torch.float16, generator=g)
        ks = vs = 1.0
    q = torch.randn((B, hq, D), device="cuda", dtype=torch.float16, generator=g)
    lens = torch.full((B,), L, dtype=torch.int32)
    outs = {}
    for P in (4, 8, 16, 32, 64, 8192):
        perm = torch.randperm(B * (L // P), device="cuda", generator=torch.Generator(device="cuda").manual_seed(P))
        perm = perm.to(torch.int32)
        kp, table = _paged_layout(klog, P, perm)
        vp, _ = _paged_layout(vlog, P, perm)
        dec = pa_amd.Decoder(hq, hkv, D, P, fp8)
        dec.plan(lens, 0)
        outs[P] = dec.run(q, kp, vp, table, lens.cuda(), ks, vs)
        torch.cuda.synchronize()
        if P == 8192:
            dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
            kb = kp.cpu().numpy() if fp8 else kp.view(torch.int16).cpu().numpy().view(np.uint16)
            vb = vp.cpu().numpy() if fp8 else vp.view(torch.int16).cpu().numpy().view(np.uint16)
            ref = oracle.paged_decode(dt, q.view(torch.int16).cpu().numpy().view(np.uint16), kb, vb,
                                      table.cpu().numpy(), lens.numpy(), hq, hkv, D, P, ks, vs, threads=16)
            err = float(np.max(np.abs(outs[P].float().cpu().numpy() - ref)))
            assert err < TOL, err
        del kp, vp
    base = outs[16].view(torch.int16)
    for P, o in outs.items():
        assert torch.equal(o.view(torch.int16), base), f"page size {P} differs from 16"


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_config1_page_size_sweep_bitwise(fp8):
    """Config 1 (4 x 1024), whose rows span 8 blocks each and are merged across
    blocks inside the split kernel: the same q/K/V in pages of 1, 4, 8, 16,
    64 and 1024 tokens, each under its own page permutation, decode to
    bitwise the same output (the block partials and their combine order do
    not depend on where or how the pages sit), within tolerance of the oracle."""
    import torch
    B, L, hq, hkv = 4, 1024, 32, 8
    g = torch.Generator(device="cuda").manual_seed(73)
    if fp8:
        def codes():
            c = torch.randint(0, 0x7f, (B, hkv, L, D), device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
            return c | (torch.randint(0, 2, c.shape, device="cuda", generator=g, dtype=torch.int32).to(torch.uint8) << 7)
        klog, vlog = codes(), codes()
        ks = vs = 4.0 / 448.0
    else:
        klog = torch.randn((B, hkv, L, D), device="cuda", dtype=torch.float16, generator=g)
        vlog = torch.randn((B, hkv, L, D), device="cuda", dtype=torch.float16, generator=g)
        ks = vs = 1.0
    q = torch.randn((B, hq, D), device="cuda", dtype=torch.float16, generator=g)
    lens = torch.full((B,), L, dtype=torch.int32)
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    assert pa_amd.make_plan(dt, [L] * B, hq, hkv, D, 0).merge_mode == 2
    outs = {}
    for P in (1, 4, 8, 16, 64, 1024):
        perm = torch.randperm(B * (L // P), device="cuda", generator=torch.Generator(device="cuda").manual_seed(P))
        perm = perm.to(torch.int32)
        kp, table = _paged_layout(klog, P, perm)
        vp, _ = _paged_layout(vlog, P, perm)
        dec = pa_amd.Decoder(hq, hkv, D, P, fp8)
        dec.plan(lens, 0)
        outs[P] = dec.run(q, kp, vp, table, lens.cuda(), ks, vs)
        torch.cuda.synchronize()
        if P == 16:
            kb = kp.cpu().numpy() if fp8 else kp.view(torch.int16).cpu().numpy().view(np.uint16)
            vb = vp.cpu().numpy() if fp8 else vp.view(torch.int16).cpu().numpy().view(np.uint16)
            ref = oracle.paged_decode(dt, q.view(torch.int16).cpu().numpy().view(np.uint16), kb, vb,
                                      table.cpu().numpy(), lens.numpy(), hq, hkv, D, P, ks, vs, threads=16)
            err = float(np.max(np.abs(outs[P].float().cpu().numpy() - ref)))
            assert err < TOL, err
    base = outs[16].view(torch.int16)
    for P, o in outs.items():
        assert torch.equal(o.view(torch.int16), base), f"page size {P} differs from 16"


def test_full_size_config3_stored_fp8_bytes():
    """Config 3 at full size (64 x 8192): every FP8 byte the append kernel
    stored, at the run's own per-tensor scales (amax / 448 over the seeded
    N(0,1) K and V), equals the oracle's E4M3 store of the same fp16 source
    (orc_append's encoder, as a 65536-entry table per scale), found through
    the run's scattered block table."""
    import torch
    B, L, hkv, P = 64, 8192, 8, 16
    q, kc, vc, table, ks, vs, srcs = paged_inputs(B, [L] * B, 32, hkv, P, True, seed=0, keep_sources=True)
    assert ks > 0 and vs > 0
    lut_k = oracle.e4m3_quantize_table(float(np.float32(1.0) / np.float32(ks)))
    lut_v = oracle.e4m3_quantize_table(float(np.float32(1.0) / np.float32(vs)))
    assert lut_k[0x3c00] != 0                                     # 1.0 quantizes to a nonzero code
    npp = L // P
    tab = table.cpu().numpy()
    pk, pv = kc.cpu().numpy(), vc.cpu().numpy()
    saturated = 0
    for b, (ksrc, vsrc) in enumerate(srcs):
        for src, pool, lut in ((ksrc, pk, lut_k), (vsrc, pv, lut_v)):
            bits = src.view(torch.int16).cpu().numpy().view(np.uint16)            # [L][Hkv][D]
            want = lut[bits].reshape(npp, P, hkv, D).transpose(0, 2, 1, 3)        # [page][Hkv][P][D]
            got = pool[tab[b, :npp]]
            assert np.array_equal(got, want), f"row {b}: stored FP8 bytes differ"
            saturated += int(np.count_nonzero((want & 0x7f) == 0x7e))
    assert saturated >= 2                                          # each tensor's amax lands on +-448


@pytest.mark.parametrize("compiled", [True, False], ids=["compiled", "ctypes"])
def test_decoder_empty_batch(compiled):
    """An empty batch (no sequences) plans to zero work units and segments and
    decodes to an empty output without a launch or an error, through both
    Decoder classes (the reference's make_plan and paged_decode do no work
    for it)."""
    import torch
    from pa_amd.decoder import Decoder as CtypesDecoder, decoder_class
    cls = decoder_class() if compiled else CtypesDecoder
    if compiled and cls is CtypesDecoder:
        pytest.skip("the compiled binding is not built")
    dec = cls(32, 8, 128, 16, False)
    dec.plan(torch.zeros(0, dtype=torch.int32))
    assert dec.num_ctas == 0 and dec.num_segments == 0
    q = torch.empty(0, 32, 128, dtype=torch.float16, device="cuda")
    kv = torch.zeros(1, 8, 16, 128, dtype=torch.float16, device="cuda")
    table = torch.zeros(0, 1, dtype=torch.int32, device="cuda")
    lens = torch.zeros(0, dtype=torch.int32, device="cuda")
    out = dec.run(q, kv, kv, table, lens, 1.0, 1.0)
    torch.cuda.synchronize()
    assert out.shape == (0, 32, 128) and out.dtype == torch.float16
