"""The C ABI from a plain C host (tests/c_abi/q4rdna_c_check.c): sidecar
image in memory, lookup by ggml name and shape, mul_mat / _add / _glu and a
plan against a double-precision CPU dot product, and the not-applicable
paths.  Built by __graft_entry__.build()."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "c_abi", "q4rdna_c_check")


@pytest.mark.gpu
def test_c_host_uses_the_abi(cuda):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: run __graft_entry__.build()")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c abi ok" in r.stdout
