"""Runs the C++ drop-in driver (tests/cpp/test_backend.cpp): the reference's
C++ interface (KVCache, AttentionBackend, factory) over the C ABI, checked
against the oracle inside the driver."""
import subprocess
from pathlib import Path

import pytest

from gpu_util import step

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "bin" / "test_backend"


def test_cpp_backend_driver():
    assert EXE.exists(), "build first: __graft_entry__.build()"
    step("cpp driver")
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=300)
    print(res.stdout[-4000:], res.stderr[-2000:])
    assert res.returncode == 0
    assert "ALL OK" in res.stdout
