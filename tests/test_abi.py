"""The C ABI library (include/pa_decode.h): loads, exports every declared
symbol, and maps errors to status codes without touching a device."""

import ctypes
import subprocess

import pytest

import pa_amd
from pa_amd import _lib


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    declared = _lib.header_functions()
    assert len(declared) >= 50
    assert declared == sorted(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T pa_" in line}
    assert exported == set(declared)


def test_library_has_gfx950_code_object():
    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data


def test_dtype_helpers():
    assert pa_amd.kv_dtype_bytes(pa_amd.FP16) == 2 and pa_amd.kv_dtype_bytes(pa_amd.FP8_E4M3) == 1
    assert pa_amd.kv_dtype_name(pa_amd.FP16) == "fp16"
    assert pa_amd.kv_dtype_name(pa_amd.FP8_E4M3) == "fp8_e4m3"


def test_tile_tokens_and_shape_errors():
    for g in (1, 2, 4, 8):
        assert pa_amd.tile_tokens(pa_amd.FP16, 128, g) == 16
    out = ctypes.c_int()
    lib = _lib.load()
    assert lib.pa_tile_tokens(0, 64, 4, ctypes.byref(out)) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"head_dim" in lib.pa_last_error()
    assert lib.pa_tile_tokens(0, 128, 3, ctypes.byref(out)) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_tile_tokens(7, 128, 4, ctypes.byref(out)) == _lib.PA_ERR_INVALID_ARGUMENT


def test_decode_rejects_bad_shapes_before_any_launch():
    p = _lib.DecodeParams()
    p.num_q_heads, p.num_kv_heads, p.head_dim, p.num_ctas = 32, 8, 64, 4
    with pytest.raises(pa_amd.InvalidArgument, match="head_dim"):
        pa_amd.paged_decode(pa_amd.FP16, p, 0)
    p.head_dim, p.num_q_heads = 128, 24
    with pytest.raises(pa_amd.InvalidArgument, match="group"):
        pa_amd.decode_split(pa_amd.FP16, p, 0)
    p.num_q_heads = 32
    with pytest.raises(pa_amd.InvalidArgument):
        pa_amd.decode_split(pa_amd.FP16, p, 0)          # null pointers, page_size 0
    # Split rows merged by the merge kernel and inside the split kernel at
    # once: refused by both launches (the merge kernel would read partial
    # slots the split kernel does not write).
    p.needs_merge, p.block_merge = 1, 2
    for launch in (pa_amd.decode_split, pa_amd.decode_merge, pa_amd.paged_decode):
        with pytest.raises(pa_amd.InvalidArgument, match="exclude"):
            launch(pa_amd.FP16, p, 0)
    lib = _lib.load()
    assert lib.pa_decode(0, None, None) == _lib.PA_ERR_INVALID_ARGUMENT


def test_null_handles_are_rejected():
    lib = _lib.load()
    assert lib.pa_plan_copy(None, None, None, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_pool_release(None, 0) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_cache_run(None, None, None, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_pool_admit(None) == -1
    assert lib.pa_append_quantize(0, None, None, None, None, None, 0, 4, 8, 128, 16, 1.0, 1.0, None) \
        == _lib.PA_ERR_INVALID_ARGUMENT


def test_device_queries_report_errors_not_crashes():
    import torch
    if torch.cuda.is_available():
        assert pa_amd.wave_ctas(pa_amd.FP16, 128, 4) > 0
    else:
        with pytest.raises(pa_amd.DeviceError):
            pa_amd.wave_ctas(pa_amd.FP16, 128, 4)


def test_kv_pool_stagger_and_alloc_kv_pools():
    """The library's K/V pool gap is a positive multiple of 4 KiB, and
    alloc_kv_pools lays caller-owned pools out the same way: two views of one
    allocation, V starting that many bytes after the end of K."""
    import torch
    gap = pa_amd.kv_pool_stagger()
    assert gap > 0 and gap % 4096 == 0
    for fp8, elem in ((False, 2), (True, 1)):
        k, v = pa_amd.alloc_kv_pools(3, 2, 16, 128, fp8, device="cpu")
        assert k.shape == v.shape == (3, 2, 16, 128)
        assert k.dtype == (torch.uint8 if fp8 else torch.float16) == v.dtype
        assert k.is_contiguous() and v.is_contiguous()
        assert v.data_ptr() - k.data_ptr() == 3 * 2 * 16 * 128 * elem + gap
        assert k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()


def test_append_rejects_thread_counts_past_int32():
    """The append kernel indexes (token, kv head, 8-dim chunk) in 32 bits: a
    single append of n tokens with n * num_kv_heads * 16 > INT_MAX is refused
    with PA_ERR_LENGTH (std::length_error) before any pointer is used or any
    kernel is launched; one token fewer than the limit passes the size check
    and stops at the null-pointer check."""
    lib = _lib.load()
    hkv = 8
    limit = (2**31 - 1) // (hkv * 16)
    assert lib.pa_append_quantize(1, None, None, None, None, None, 0, limit + 1, hkv, 128, 16, 1.0, 1.0, None) \
        == _lib.PA_ERR_LENGTH
    assert b"INT_MAX" in lib.pa_last_error()
    assert lib.pa_append_quantize(1, None, None, None, None, None, 0, limit, hkv, 128, 16, 1.0, 1.0, None) \
        == _lib.PA_ERR_INVALID_ARGUMENT


def test_compiled_torch_binding_loads_without_a_device():
    """The compiled binding (pa_amd/_pa_torch*.so, built with the library) is
    in tree, imports, exposes the reference binding's Decoder surface and
    raises RuntimeError for a bad seq_lens tensor before any device use."""
    import torch
    from pa_amd.decoder import decoder_class
    from pa_amd import _pa_torch
    assert decoder_class() is _pa_torch.Decoder
    dec = _pa_torch.Decoder(32, 8, 128, 16, False)
    for name in ("plan", "run", "num_ctas", "num_segments"):
        assert hasattr(dec, name)
    assert dec.num_ctas == 0 and dec.num_segments == 0
    with pytest.raises(RuntimeError, match="CPU int32"):
        dec.plan(torch.tensor([10], dtype=torch.int64))


_BAD_ORDER = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1]]
ctypes.CDLL(sys.argv[2])                  # the library first: the system's HIP runtime
import torch                              # then torch: its own copy beside it
from pa_amd import _lib
assert len(_lib.hip_runtimes()) == 2, _lib.hip_runtimes()
try:
    _lib.load()
except RuntimeError as e:
    assert "two HIP runtimes" in str(e), e
    print("refused")
"""

_GOOD_ORDER = r"""
import sys
sys.path[:0] = [sys.argv[1]]
import torch
from pa_amd import _lib
_lib.load()
assert len(_lib.hip_runtimes()) == 1, _lib.hip_runtimes()
print("one runtime")
"""


def test_loader_refuses_a_second_hip_runtime():
    """torch links its own copy of the HIP runtime and asks for it as
    libamdhip64.so; the library asks for libamdhip64.so.7. Loaded after
    torch, the library shares torch's copy; loaded before it, the process
    ends up with two runtimes (the second sees no GPU), and pa_amd's loader
    says so instead of failing later with hipErrorNoDevice. No GPU needed."""
    import pathlib
    import subprocess
    import sys
    pkg = pathlib.Path(pa_amd.__file__).resolve().parent.parent
    lib = str(pkg / "lib" / "libpa_decode.so")
    bad = subprocess.run([sys.executable, "-c", _BAD_ORDER, str(pkg), lib], capture_output=True, text=True,
                         timeout=120)
    assert bad.returncode == 0 and "refused" in bad.stdout, bad.stdout + bad.stderr[-2000:]
    good = subprocess.run([sys.executable, "-c", _GOOD_ORDER, str(pkg)], capture_output=True, text=True,
                          timeout=120)
    assert good.returncode == 0 and "one runtime" in good.stdout, good.stdout + good.stderr[-2000:]
