"""Builds libpa_decode.so (the C ABI in include/pa_decode.h) for gfx950.

    python paged-attention_amd/build.py          # compile + link in-tree

The library is written to paged-attention_amd/lib/ so that it travels with the
source tree; nothing is installed. Every call recompiles (a few seconds per
file), so the result always matches the sources.
"""

from __future__ import annotations

import os
import pathlib
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
OBJ_DIR = PKG / "_build"
LIB = LIB_DIR / "libpa_decode.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled on purpose (they have produced silent wrong
# results on this hardware pool); the host pass warns that it does not know the
# feature, which is harmless.
COMMON = [
    "-O3",
    "-std=c++20",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]

SOURCES = ["pa_decode.hip", "pa_cache.hip", "pa_scratch.hip", "pa_plan.cpp", "pa_pool.cpp", "pa_kvcache.cpp"]

# Device code only: the first kernel arguments (up to the first struct passed by
# value) arrive preloaded in SGPRs when the wave starts, so a kernel's first
# loads do not wait for a read of the kernel-argument segment. The code object
# keeps an entry sequence that loads them for firmware without preloading.
KERNARG_PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=8"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")


def build(verbose: bool = False, defines: list[str] | None = None, lib: pathlib.Path | None = None,
          obj_dir: pathlib.Path | None = None) -> pathlib.Path:
    """Compiles SOURCES and links `lib` (default lib/libpa_decode.so). `defines`
    are extra -D options (the kernels' compile-time tuning knobs)."""
    lib = lib or LIB
    obj_dir = obj_dir or OBJ_DIR
    obj_dir.mkdir(parents=True, exist_ok=True)
    lib.parent.mkdir(parents=True, exist_ok=True)
    extra = [f"-D{d}" for d in (defines or [])]
    jobs = []
    objs = []
    for src in SOURCES:
        obj = obj_dir / (src + ".o")
        lang = ["-x", "hip", *KERNARG_PRELOAD] if src.endswith(".hip") else []
        jobs.append([HIPCC, *COMMON, *extra, *lang, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    if verbose:
        for cmd in jobs:
            print(" ".join(cmd), flush=True)
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        list(ex.map(_run, jobs))
    tmp = lib.with_suffix(".so.tmp")
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(tmp, lib)
    return lib


BENCH_SRC = PKG / "bench" / "bench_decode.cpp"
BENCH_BIN = PKG / "bench" / "_build" / "bench_decode"


def build_bench(verbose: bool = False) -> pathlib.Path:
    """The native bench CLI (bench/bench_decode.cpp) against lib/libpa_decode.so."""
    BENCH_BIN.parent.mkdir(parents=True, exist_ok=True)
    cmd = [HIPCC, *COMMON, "-x", "hip", str(BENCH_SRC), f"-I{PKG / 'cpp'}", "-o", str(BENCH_BIN),
           f"-L{LIB_DIR}", "-lpa_decode", f"-Wl,-rpath,$ORIGIN/../../lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    return BENCH_BIN


TORCH_EXT_SRC = CSRC / "pa_torch.cpp"
TORCH_EXT_NAME = "_pa_torch"


def torch_ext_path() -> pathlib.Path:
    """Where the compiled torch binding goes: inside the pa_amd package."""
    import sysconfig
    return PKG / "pa_amd" / (TORCH_EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_torch_ext(verbose: bool = False) -> pathlib.Path:
    """The compiled torch binding (csrc/pa_torch.cpp: Decoder, the reference's
    bindings/torch_decode.cu signature) against lib/libpa_decode.so and the
    installed torch (host code only; its headers need the HIP platform macro)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce

    out = torch_ext_path()
    incs = ce.include_paths(device_type="cuda") + [sysconfig.get_paths()["include"], str(ROOT / "include")]
    libs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = out.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           f"-DTORCH_EXTENSION_NAME={TORCH_EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in incs], str(TORCH_EXT_SRC), "-o", str(tmp),
           *[f"-L{p}" for p in libs], f"-L{LIB_DIR}",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", "-lpa_decode",
           f"-Wl,-rpath,$ORIGIN/../lib", f"-Wl,-rpath,{libs[0]}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description="Builds libpa_decode.so for gfx950. With -D, a comparison build of the "
                                             "kernels' compile-time knobs (e.g. -D PA_STAGE_SWIZZLE=0) into --lib; "
                                             "load it with PA_DECODE_LIB=<path>.")
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("-D", dest="defines", action="append", default=[], metavar="NAME=VALUE")
    ap.add_argument("--lib", type=pathlib.Path, default=None, help="output library (default lib/libpa_decode.so)")
    a = ap.parse_args()
    if a.defines and a.lib is None:
        ap.error("a build with -D needs its own --lib path (lib/libpa_decode.so stays the product build)")
    obj = None if a.lib is None else OBJ_DIR / ("variant_" + a.lib.stem)
    print(build(verbose=a.verbose, defines=a.defines, lib=a.lib, obj_dir=obj))
