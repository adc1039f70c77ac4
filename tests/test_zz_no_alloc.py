"""pa_decode_static, the allocation-free variant of pa_decode (no counterpart
in the reference): the partial workspace of rows split across blocks lives in
the library's fixed device array instead of the caller's params.

GPU: two calls in a row through the C ABI, the second with a smaller input,
each bitwise equal to pa_decode on the same plan with the device plan's own
workspace (same kernels, same arithmetic), and within the tolerance of the
oracle. CPU: oversized plans and bad arguments are refused before any device
use.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
import pa_amd
from helpers import D, TOL, paged_inputs
from pa_amd import _lib

SCRATCH_BYTES = 32 << 20


def _params(q, k, v, table, lens, hq, hkv, ks, vs, dplan):
    import torch
    p = pa_amd.DecodeParams()
    p.q, p.k_cache, p.v_cache, p.block_table = q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr()
    out = torch.empty_like(q)
    p.out = out.data_ptr()
    p.block_table_stride = table.size(1)
    p.batch, p.num_q_heads, p.num_kv_heads, p.head_dim, p.page_size = len(lens), hq, hkv, D, 16
    p.sm_scale, p.k_scale, p.v_scale = pa_amd.sm_scale(D), ks, vs
    dplan.bind(p)
    return p, out


def test_decode_static_refuses_oversized_plans_without_a_device():
    """The workspace is sized from the bound plan's own segment count
    (params.num_segments, set by DevicePlan.bind). A plan whose partial
    workspace exceeds the 32 MiB array is refused with PA_ERR_LENGTH; null
    params, params not bound to a plan (num_segments 0 for a non-empty grid), a
    caller's count that differs from the bound one (under- or overstated), split
    rows with neither merge set, an unknown dtype or an unsupported head_dim
    with PA_ERR_INVALID_ARGUMENT; all before the library looks up the array or
    launches anything."""
    lib = _lib.load()
    p = pa_amd.DecodeParams()
    p.num_q_heads, p.num_kv_heads, p.head_dim, p.num_ctas, p.batch = 32, 8, D, 2048, 4
    per_seg = 4 * (D + 1) * 4                         # group 4: 4 rows of head_dim + 1 floats
    too_many = SCRATCH_BYTES // per_seg + 1
    p.num_segments, p.needs_merge = too_many, 1
    assert lib.pa_decode_static(0, ctypes.byref(p), too_many, None) == _lib.PA_ERR_LENGTH
    assert b"static scratch" in lib.pa_last_error()
    p.needs_merge, p.block_merge = 0, 2                 # merged across blocks: partials in the array too
    assert lib.pa_decode_static(0, ctypes.byref(p), too_many, None) == _lib.PA_ERR_LENGTH
    assert b"static scratch" in lib.pa_last_error()
    p.needs_merge, p.block_merge = 1, 0
    assert lib.pa_decode_static(0, None, 10, None) == _lib.PA_ERR_INVALID_ARGUMENT
    # An understated count: the kernels would write the bound plan's partials.
    p.num_segments = 2048
    for wrong in (2047, 1000, 32, 0, 4096):
        assert lib.pa_decode_static(0, ctypes.byref(p), wrong, None) == _lib.PA_ERR_INVALID_ARGUMENT, wrong
        assert b"differs from the bound plan" in lib.pa_last_error()
    p.num_segments = 0                                  # not bound
    assert lib.pa_decode_static(0, ctypes.byref(p), 0, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"not bound" in lib.pa_last_error()
    p.num_segments, p.needs_merge, p.block_merge = 2048, 0, 0   # split rows, no merge
    assert lib.pa_decode_static(0, ctypes.byref(p), 2048, None) == _lib.PA_ERR_INVALID_ARGUMENT
    p.needs_merge = 1
    assert lib.pa_decode_static(5, ctypes.byref(p), 2048, None) == _lib.PA_ERR_INVALID_ARGUMENT
    p.head_dim = 64
    assert lib.pa_decode_static(0, ctypes.byref(p), 2048, None) == _lib.PA_ERR_INVALID_ARGUMENT


def test_decode_static_sizes_no_workspace_for_unsplit_or_block_merged_plans():
    """Plans that write no partial to HBM need no workspace, however many
    segments they have: every segment whole (2048 rows x 8 kv heads = 16384
    whole segments, 33.8 MB at 4 x 129 floats each) or every split row merged
    in LDS. Neither is refused for size; without a device the call then stops
    at the device step (or, with one, at the null pointers of these params)."""
    lib = _lib.load()
    p = pa_amd.DecodeParams()
    p.num_q_heads, p.num_kv_heads, p.head_dim, p.num_ctas, p.batch = 32, 8, D, 2048, 2048
    assert 16384 * 4 * (D + 1) * 4 > SCRATCH_BYTES
    p.num_segments, p.needs_merge, p.block_merge = 16384, 0, 0
    st = lib.pa_decode_static(0, ctypes.byref(p), 16384, None)
    assert st not in (_lib.PA_OK, _lib.PA_ERR_LENGTH) and b"static scratch" not in lib.pa_last_error()
    p.batch = 4
    p.num_segments, p.needs_merge, p.block_merge = 16384, 0, 1
    st = lib.pa_decode_static(0, ctypes.byref(p), 16384, None)
    assert st not in (_lib.PA_OK, _lib.PA_ERR_LENGTH) and b"static scratch" not in lib.pa_last_error()


@pytest.mark.gpu
@pytest.mark.usefixtures("gpu_device")
@pytest.mark.parametrize("fp8", [False, True], ids=["fp16", "fp8"])
def test_decode_static_matches_decode_on_two_calls(fp8):
    import torch
    lib = _lib.load()
    hq, hkv = 32, 8
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    # Call 1: 4 x 1024 on the default grid (rows split across blocks, merged
    # by the split kernel through block partials in the array). Call 2,
    # smaller: a ragged batch on 100 units, forced through the merge kernel
    # (every segment's partial in the array). Call 3: 8 x 2048 on 512 units,
    # merged inside one block each (no workspace).
    cases = [([1024] * 4, 0, 2, False), ([700, 33, 2000], 100, 2, True), ([2048] * 8, 512, 1, False)]
    prev_segments = None
    for i, (lens, ctas, mode, force_kernel) in enumerate(cases):
        q, k, v, table, ks, vs = paged_inputs(len(lens), lens, hq, hkv, 16, fp8, seed=40 + i)
        plan = pa_amd.make_plan(dt, lens, hq, hkv, D, ctas)
        nseg = len(plan.segments)
        if prev_segments is not None and mode != 1:
            assert nseg < prev_segments                # the second call is the smaller input
        prev_segments = nseg
        dplan = pa_amd.DevicePlan()
        dplan.upload(plan, hq // hkv, D)
        p_ref, out_ref = _params(q, k, v, table, lens, hq, hkv, ks, vs, dplan)
        assert p_ref.block_merge == mode and p_ref.needs_merge == 0
        p_st, out_st = _params(q, k, v, table, lens, hq, hkv, ks, vs, dplan)
        if force_kernel:
            for p in (p_ref, p_st):
                p.block_merge, p.needs_merge = 0, 1
        p_st.partial_out = None                        # ignored by the static entry point
        p_st.partial_lse = None
        out_st.fill_(float("nan"))
        stream = torch.cuda.current_stream().cuda_stream
        assert p_st.num_segments == nseg                 # recorded by bind
        # A count that disagrees with the bound plan launches nothing.
        assert lib.pa_decode_static(dt, ctypes.byref(p_st), nseg - 1, stream) == _lib.PA_ERR_INVALID_ARGUMENT
        torch.cuda.synchronize()
        assert torch.isnan(out_st.float()).all()
        assert lib.pa_decode(dt, ctypes.byref(p_ref), stream) == _lib.PA_OK
        assert lib.pa_decode_static(dt, ctypes.byref(p_st), nseg, stream) == _lib.PA_OK, lib.pa_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_st.view(torch.int16), out_ref.view(torch.int16)), f"call {i + 1} differs"
        kb = k.view(torch.uint8).cpu().numpy() if fp8 else k.view(torch.int16).cpu().numpy().view(np.uint16)
        vb = v.view(torch.uint8).cpu().numpy() if fp8 else v.view(torch.int16).cpu().numpy().view(np.uint16)
        ref = oracle.paged_decode(dt, q.view(torch.int16).cpu().numpy().view(np.uint16), kb, vb, table.cpu().numpy(),
                                  np.asarray(lens, np.int32), hq, hkv, D, 16, ks, vs, threads=16)
        err = float(np.max(np.abs(out_st.float().cpu().numpy() - ref)))
        assert err < TOL, (i, err)


@pytest.mark.gpu
@pytest.mark.usefixtures("gpu_device")
@pytest.mark.parametrize("force_kernel", [False, True], ids=["split_kernel_merge", "merge_kernel"])
def test_decode_static_graph_replays_match_eager(force_kernel):
    """The callers the entry point is for: pa_decode_static captured into a HIP
    graph, on a plan whose rows span blocks (block partials in the library's
    array, merged by the split kernel; or, forced, every partial there for the
    merge kernel). Every replay, with q rewritten before it and an eager
    pa_decode_static of other inputs after it (the same array, the same
    stream), equals an eager pa_decode of the same q with the plan's own
    workspace, bitwise."""
    import torch
    lib = _lib.load()
    hq, hkv = 32, 8
    lens = [1024] * 4
    q, k, v, table, ks, vs = paged_inputs(len(lens), lens, hq, hkv, 16, False, seed=77)
    plan = pa_amd.make_plan(pa_amd.FP16, lens, hq, hkv, D, 0)
    nseg = len(plan.segments)
    dplan = pa_amd.DevicePlan()
    dplan.upload(plan, hq // hkv, D)
    p_ref, out_ref = _params(q, k, v, table, lens, hq, hkv, ks, vs, dplan)
    assert p_ref.needs_merge == 0 and p_ref.block_merge == 2
    p_st, out_st = _params(q, k, v, table, lens, hq, hkv, ks, vs, dplan)
    g = torch.Generator(device="cuda").manual_seed(5)
    other_q = torch.randn(q.shape, device="cuda", dtype=q.dtype, generator=g)
    p_other, _ = _params(other_q, k, v, table, lens, hq, hkv, ks, vs, dplan)
    if force_kernel:
        for p in (p_ref, p_st, p_other):
            p.block_merge, p.needs_merge = 0, 1
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        h = st.cuda_stream
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            status = lib.pa_decode_static(0, ctypes.byref(p_st), nseg, torch.cuda.current_stream().cuda_stream)
        assert status == _lib.PA_OK, lib.pa_last_error()
        torch.cuda.synchronize()
        for rep in range(4):
            q.normal_(generator=g)
            assert lib.pa_decode(0, ctypes.byref(p_ref), h) == _lib.PA_OK
            torch.cuda.synchronize()
            out_st.zero_()
            graph.replay()
            assert lib.pa_decode_static(0, ctypes.byref(p_other), nseg, h) == _lib.PA_OK
            torch.cuda.synchronize()
            assert torch.equal(out_st.view(torch.int16), out_ref.view(torch.int16)), f"replay {rep} differs"


_FIRST_CALL_IN_CAPTURE = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1], sys.argv[2], sys.argv[3]]
import torch
import pa_amd
from pa_amd import _lib
from helpers import D, paged_inputs
torch.cuda.set_device(0)
lib = _lib.load()
hq, hkv, lens = 32, 8, [1024] * 4
q, k, v, table, ks, vs = paged_inputs(len(lens), lens, hq, hkv, 16, False, seed=78)
plan = pa_amd.make_plan(pa_amd.FP16, lens, hq, hkv, D, 0)
dplan = pa_amd.DevicePlan()
dplan.upload(plan, hq // hkv, D)          # set-up: looks up the array's address
def params(out):
    p = pa_amd.DecodeParams()
    p.q, p.k_cache, p.v_cache, p.block_table = q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr()
    p.out = out.data_ptr()
    p.block_table_stride = table.size(1)
    p.batch, p.num_q_heads, p.num_kv_heads, p.head_dim, p.page_size = len(lens), hq, hkv, D, 16
    p.sm_scale, p.k_scale, p.v_scale = pa_amd.sm_scale(D), ks, vs
    dplan.bind(p)
    return p
out_ref, out_st = torch.empty_like(q), torch.zeros_like(q)
p_ref, p_st = params(out_ref), params(out_st)
assert p_ref.block_merge == 2
st = torch.cuda.Stream()
with torch.cuda.stream(st):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        status = lib.pa_decode_static(0, ctypes.byref(p_st), len(plan.segments),
                                      torch.cuda.current_stream().cuda_stream)
    assert status == _lib.PA_OK, lib.pa_last_error()
    assert lib.pa_decode(0, ctypes.byref(p_ref), st.cuda_stream) == _lib.PA_OK
    torch.cuda.synchronize()
    for rep in range(3):
        out_st.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_st.view(torch.int16), out_ref.view(torch.int16)), rep
print("first call in capture: ok", flush=True)
"""


@pytest.mark.gpu
@pytest.mark.usefixtures("gpu_device")
def test_decode_static_first_call_inside_a_capture():
    """In a fresh process, the entry point's first call is made inside a HIP
    graph capture: the plan upload before it has already looked up the array,
    so the capture needs no lookup, and every replay equals eager pa_decode."""
    import pathlib
    import subprocess
    import sys
    root = pathlib.Path(__file__).resolve().parent.parent
    print("# child: first pa_decode_static call inside a graph capture (4 x 1024 fp16)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, str(root), str(root / "paged-attention_amd"),
                        str(root / "tests")], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    assert "first call in capture: ok" in r.stdout
