"""The BASELINE configurations through the torch `Decoder` binding
(bindings/torch_decode.cu:14-81): C1-C3 and C5 at full size against the
oracle, C4 at full size with sampled rows, a full-size placement-invariance
check, and the binding's argument checks.
"""

from __future__ import annotations

import numpy as np
import pytest

import pa_amd
from helpers import D, TOL, decoder_case, paged_inputs

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu_device")]

DTYPES = [False, True]   # fp8?
IDS = ["fp16", "fp8"]


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_decoder_binding_config1(fp8):
    """BASELINE config 1 shape (4 x 1024, P=16, scattered) via the torch_decode
    `Decoder` signature."""
    err, dec = decoder_case(4, [1024] * 4, fp8)
    assert dec.num_ctas > 0 and dec.num_segments >= 32
    assert err < TOL, err

def test_decoder_full_size_config2():
    """BASELINE config 2 at full size: 32 x 8192 fp16, 16-token scattered pages."""
    err, _ = decoder_case(32, [8192] * 32, False, threads=16)
    assert err < TOL, err

def test_decoder_full_size_config3():
    """BASELINE config 3 at full size: 64 x 8192, FP8 E4M3 (amax/448 scales,
    quantized by the append kernel), 16-token scattered pages."""
    err, _ = decoder_case(64, [8192] * 64, True, threads=16)
    assert err < TOL, err

def test_decoder_full_size_config4_sampled_rows():
    """BASELINE config 4 at full size (128 ragged rows, L ~ U[128, 16384],
    seed 4) decoded in one batch; 12 rows spread over the batch (first, last,
    longest, shortest, 8 seeded) checked against the oracle."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=128)]
    pick = {0, 127, int(np.argmax(lens)), int(np.argmin(lens))}
    pick |= set(int(x) for x in np.random.default_rng(9).choice(128, 8, replace=False))
    err, dec = decoder_case(128, lens, False, threads=16, rows=sorted(pick))
    assert dec.num_segments >= 128 * 8
    assert err < TOL, err

def test_decoder_ragged_config4_subset():
    """BASELINE config 4's ragged lengths (U[128, 16384] from a seed), first 16 rows."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=16)]
    err, _ = decoder_case(len(lens), lens, False, threads=16)
    assert err < TOL, err

def test_decoder_long_context_config5_fp16():
    """BASELINE config 5 (1 x 131072), fp16 KV."""
    err, dec = decoder_case(1, [131072], False, threads=8)
    assert dec.num_segments > 8 * 64
    assert err < TOL, err

def test_decoder_long_context_config5_fp8():
    """BASELINE config 5 (1 x 131072), FP8 KV: hundreds of splits per row."""
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
