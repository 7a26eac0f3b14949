"""The allocation-free K-quant entry point (rl_hip_gemm_kquant_noalloc) against
the workspace entry point (rl_hip_gemm_kquant) through the C ABI: bit-identical
results on two calls in a row, the second with a smaller input (the shared
scratch keeps the first call's contents, and its split-K tickets must be back at
zero), and a clear RL_ERR_RANGE for a shape whose scratch need exceeds the fixed
array."""
import ctypes as C

import numpy as np
import pytest

from rapidllm_amd import hip, ops, synth
from rapidllm_amd.hip import DeviceBuffer, call

pytestmark = pytest.mark.gpu


def run_both(qt, m, n, T, seed, accumulate=False):
    r = synth.rng(seed)
    blocks = synth.q4k_blocks(r, m, n) if qt == ops.Q4_K else synth.q6k_blocks(r, m, n)
    lin = ops.KQuantLinear(qt, blocks, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    Y0 = r.standard_normal((T, m)).astype(np.float32)
    xd = DeviceBuffer.from_numpy(X)
    ya = DeviceBuffer.from_numpy(Y0)
    yb = DeviceBuffer.from_numpy(Y0)
    ws = ops.kquant_workspace(m, n, T)
    call("rl_hip_gemm_kquant", qt, lin.w.ptr, xd.ptr, ya.ptr, ws.ptr, ws.nbytes, m, n, T, int(accumulate), None)
    call("rl_hip_gemm_kquant_noalloc", qt, lin.w.ptr, xd.ptr, yb.ptr, m, n, T, int(accumulate), None)
    call("rl_hip_stream_synchronize", None)
    return ya.numpy(np.float32, (T, m)), yb.numpy(np.float32, (T, m)), ws.nbytes


def test_noalloc_equals_workspace_entry_point_twice(gpu):
    L = hip.lib()
    assert L.rl_hip_gemm_kquant_noalloc_max_scratch() == 4 << 20
    # first call: the C2 shape at T=4 (split-K: tickets and partials in scratch)
    want, got, need = run_both(ops.Q4_K, 5120, 17408, 4, seed=1)
    assert need > 256  # this shape does use split-K partials
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # second call, smaller input, other type, accumulate mode
    want, got, _ = run_both(ops.Q6_K, 1000, 4096, 2, seed=2, accumulate=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_rejects_shapes_beyond_scratch(gpu):
    L = hip.lib()
    m, n, T = 4096, 256 * 4096, 4
    assert L.rl_hip_kquant_workspace_bytes(m, n, T) > L.rl_hip_gemm_kquant_noalloc_max_scratch()
    rc = L.rl_hip_gemm_kquant_noalloc(ops.Q4_K, None, None, None, m, n, T, 0, None)
    assert rc == 6  # RL_ERR_RANGE
    assert b"scratch" in L.rl_hip_last_error()
