"""The reference-side adapters (rapidllm_amd/integration: HipEngine for
cuda_gen::Engine, include/rapidllm/runtime/cuda_engine.h:13-83, and HipDevice for
rapidllm::Device, include/rapidllm/backend/device.h:49-60) compile against the
reference's own headers with the reference's compiler settings (g++, C++20).
Skipped where no RapidLLM tree is present; tests/test_gpu_integration.py runs
them on the GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = os.environ.get("RAPIDLLM_INCLUDE", "/root/reference/include")


@pytest.mark.parametrize("src", ["hip_engine.cpp", "hip_device.cpp"])
def test_adapter_compiles_against_reference_headers(src, tmp_path):
    if not os.path.isfile(os.path.join(REF_INC, "rapidllm", "runtime", "cuda_engine.h")):
        pytest.skip("no RapidLLM include tree here")
    cmd = ["g++", "-std=c++20", "-Wall", "-Werror=return-type", "-c",
           os.path.join(ROOT, "rapidllm_amd", "integration", src), "-I", REF_INC, "-I", os.path.join(ROOT, "include"),
           "-o", str(tmp_path / (src + ".o"))]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
