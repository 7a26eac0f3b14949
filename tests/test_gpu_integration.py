"""The reference-side adapters on the GPU: tests/_build/seam_check (built by
tests/seam_check.mk against the reference's headers) creates a model through
hip_gen::HipEngine (cuda_gen::Engine) and the C ABI and compares both with the
oracle model, runs Session::generate's MTP loop through the adapter, and launches
every hip_gen::HipDevice kernel name with the reference's parameter structs
against the oracle's ops."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "_build", "seam_check")


def test_reference_side_adapters(gpu):
    if not os.path.exists(BIN):
        pytest.skip("seam_check not built (make -f tests/seam_check.mk, needs the RapidLLM headers)")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "seam_check ok" in r.stdout
