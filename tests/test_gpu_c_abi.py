"""The C ABI from plain C: tests/c_abi/consumer.c, built by __graft_entry__.build()
against include/ingot_rocm.h and the in-tree library, runs the reference's own
Gemm+ReLU case (f32), an exact MatMulInteger and an error path on device 0,
each checked inside the C program (double-precision / exact integer references)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "consumer")


def test_c_consumer():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: run __graft_entry__.build()")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"consumer failed ({r.returncode}):\n{r.stdout}\n{r.stderr}"
    assert "c-abi consumer ok" in r.stdout
