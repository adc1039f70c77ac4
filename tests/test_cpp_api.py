"""The C++ surface (paged-attention_amd/cpp) through tests/cpp/test_cpp_api.cpp:
host-only checks on the CPU, device decode against the oracle on the GPU."""

import pathlib
import subprocess

import pytest

HERE = pathlib.Path(__file__).resolve().parent
BIN = HERE / "cpp" / "_build" / "test_cpp_api"


def _binary() -> pathlib.Path:
    if not BIN.exists():
        subprocess.run(["make", "-s", "-C", str(HERE / "cpp")], check=True)
    return BIN


def _run(mode: str) -> None:
    proc = subprocess.run([str(_binary()), mode], capture_output=True, text=True, timeout=600)
    print(proc.stdout, proc.stderr, flush=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_cpp_api_host():
    _run("cpu")


@pytest.mark.gpu
def test_cpp_api_device():
    _run("gpu")
