"""The header-only sytorch-style backend (include/mpcx_backend.hpp), driven
from C++ (tests/cpp/backend_check.cpp): a dealer pass writes the keys of a
small network (reveal, matmul with public weights + bias, truncation, ReLU,
local linear ops, Beaver product, masked max-pool, output), an evaluator pass
consumes them, and the outputs are compared with exact host integer arithmetic."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "backend_check")


def test_backend_check_built():
    assert os.path.exists(BIN), "tests/cpp/backend_check not built (run __graft_entry__.build())"


@pytest.mark.gpu
@pytest.mark.parametrize("bw", [32, 64])
def test_backend_dealer_then_evaluator(bw):
    r = subprocess.run([BIN, str(bw)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bit-exact" in r.stdout


@pytest.mark.gpu
def test_backend_local_truncation():
    """set_truncation(MPCX_LOCALARS) on the dealer and the evaluator (the reference
    batched backend's default): keyless truncations, outputs within 1 of exact."""
    r = subprocess.run([BIN, "64", "local"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "within 1" in r.stdout
