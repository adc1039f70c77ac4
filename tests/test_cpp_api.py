"""The C++ surface (paged-attention_amd/cpp) through tests/cpp/test_cpp_api.cpp
(decode:: API) and tests/cpp/test_legacy_api.cpp (KVPool / AttentionBackend
implementations, host fp16 codec): host-only checks on the CPU, device decode
against the oracle on the GPU."""

import pathlib
import subprocess

import pytest

HERE = pathlib.Path(__file__).resolve().parent
BUILD = HERE / "cpp" / "_build"


def _binary(name: str) -> pathlib.Path:
    if not (BUILD / name).exists():
        subprocess.run(["make", "-s", "-C", str(HERE / "cpp")], check=True)
    return BUILD / name


def _run(mode: str, name: str = "test_cpp_api") -> None:
    proc = subprocess.run([str(_binary(name)), mode], capture_output=True, text=True, timeout=600)
    print(proc.stdout, proc.stderr, flush=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_cpp_api_host():
    _run("cpu")


@pytest.mark.gpu
def test_cpp_api_device():
    _run("gpu")


def test_legacy_api_host():
    _run("cpu", "test_legacy_api")


@pytest.mark.gpu
def test_legacy_api_device():
    _run("gpu", "test_legacy_api")
