"""The C ABI driven from C: tests/c/abi_ring.c binds include/longctx100m_attn.h
as a non-Python caller would (plain pointers, the reference's host-pointer
ring signatures) and checks validation texts (CPU), BASELINE config 1's
forward and backward of both ranks against the C oracle at 1e-5 (GPU), and
the call sequence of the candle CustomOp3 in longctx100m_amd/rust/amd_attn.rs
(one rank, GQA, bf16 host buffers, the forward's saved m and l handed to the
backward) against the C oracle at 2e-2 (GPU)."""

import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
BIN = HERE / "c" / "bin" / "abi_ring"


@pytest.fixture(scope="module")
def abi_ring():
    srcs = [HERE / "c" / "abi_ring.c", HERE.parent / "include" / "longctx100m_attn.h"]
    if not BIN.exists() or any(s.stat().st_mtime > BIN.stat().st_mtime for s in srcs):
        subprocess.run(["make", "-s", "-C", str(HERE / "c")], check=True)
    return BIN


def _run(binary, mode, timeout):
    res = subprocess.run([str(binary), mode], capture_output=True, text=True, timeout=timeout)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("abi_ring: ok")
    return res.stdout


def test_c_caller_validation(abi_ring):
    out = _run(abi_ring, "validate", 60)
    assert "FAIL" not in out


@pytest.mark.gpu
def test_c_caller_config1_against_c_oracle(abi_ring):
    out = _run(abi_ring, "config1", 120)
    assert out.count("pass: config 1 rank") == 6 and "FAIL" not in out


@pytest.mark.gpu
def test_c_caller_customop3_sequence_against_c_oracle(abi_ring):
    out = _run(abi_ring, "customop3", 120)
    assert out.count("pass: customop3") == 2 and "FAIL" not in out
