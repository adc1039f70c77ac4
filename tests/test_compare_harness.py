"""The comparison harness's fp32 torch reference (compare_flashinfer.py:113-126
restated in pa_amd.compare.reference), pinned on the CPU against the C oracle's
paged attention over the same pools, fp16 and FP8, with a scattered block
table and a length that ends inside a page. Also its page gather."""

import numpy as np
import pytest
import torch

import oracle
import pa_amd
from pa_amd import compare

HQ, HKV, D, P = compare.HQ, compare.HKV, compare.DIM, compare.PAGE


def _pools(batch, seq_len, fp8, seed):
    g = torch.Generator().manual_seed(seed)
    n = -(-seq_len // P)
    k = torch.randn(batch * n, HKV, P, D, generator=g).to(torch.float16)
    v = torch.randn(batch * n, HKV, P, D, generator=g).to(torch.float16)
    ks = vs = 1.0
    if fp8:
        ks, vs = k.abs().max().item() / 448.0, v.abs().max().item() / 448.0
        k, v = (k / ks).to(torch.float8_e4m3fn), (v / vs).to(torch.float8_e4m3fn)
    bt = torch.randperm(batch * n, generator=g).to(torch.int32).view(batch, n).contiguous()
    q = torch.randn(batch, HQ, D, generator=g).to(torch.float16)
    return q, k, v, ks, vs, bt


@pytest.mark.parametrize("fp8", [False, True], ids=["fp16", "fp8"])
def test_reference_matches_oracle(fp8):
    batch, seq_len = 3, 77
    q, k, v, ks, vs, bt = _pools(batch, seq_len, fp8, seed=5)
    got = compare.reference(q, k, v, ks, vs, bt, seq_len).numpy()
    raw = (lambda t: t.view(torch.uint8).numpy()) if fp8 else (lambda t: t.view(torch.int16).numpy().view(np.uint16))
    exp = oracle.paged_decode(pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16, q.view(torch.int16).numpy().view(np.uint16),
                              raw(k), raw(v), bt.numpy(), np.full(batch, seq_len, np.int32), HQ, HKV, D, P,
                              ks, vs)
    assert np.max(np.abs(got - exp)) < 2e-6


def test_gather_follows_the_block_table():
    q, k, v, ks, vs, bt = _pools(2, 40, False, seed=9)
    g = compare.gather(k, bt, 40, 1.0)
    assert g.shape == (2, HKV, 40, D) and g.dtype == torch.float16
    for b in range(2):
        for t in (0, 15, 16, 39):
            assert torch.equal(g[b, :, t], k[bt[b, t // P], :, t % P])
