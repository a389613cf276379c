"""The C ABI from C++ with no Python in the loop (GPU): tests/kat_c_abi.cpp,
built next to the library by ez-ops_amd/build.py, runs known-answer cases
whose results are exact (GEMV of small integers, decode attention with a
uniform softmax over the live rows of a larger cache, causal prefill
attention with a uniform softmax over each token's prefix, RMSNorm of +-2
rows)
and the EZOPS_EINVAL error path, as a child process."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
KAT = Path(__file__).resolve().parents[1] / "ez-ops_amd" / "ezops" / "_lib" / "ezops_kat_c_abi"


def test_c_abi_known_answers():
    assert KAT.exists(), "build first: python ez-ops_amd/build.py --all"
    r = subprocess.run([str(KAT)], capture_output=True, text=True, timeout=90)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "KAT OK" in r.stdout, r.stdout
