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


FIRST_USE = r"""
import sys
sys.path.insert(0, {root!r})
import numpy as np
from rapidllm_amd import hip, ops, synth
from rapidllm_amd.hip import DeviceBuffer, call
import ctypes as C
hip.require_gpu()
L = hip.lib()
m, n, T = 5120, 17408, 4
r = synth.rng(9)
lin = ops.KQuantLinear(ops.Q4_K, synth.q4k_blocks(r, m, n), m, n)
X = r.standard_normal((T, n)).astype(np.float32)
xd = DeviceBuffer.from_numpy(X)
ys = [DeviceBuffer.from_numpy(np.zeros((T, m), np.float32)) for _ in range(3)]
ws = ops.kquant_workspace(m, n, T)
call("rl_hip_gemm_kquant", ops.Q4_K, lin.w.ptr, xd.ptr, ys[0].ptr, ws.ptr, ws.nbytes, m, n, T, 0, None)
call("rl_hip_stream_synchronize", None)
streams = []
for _ in range(2):
    h = C.c_void_p()
    call("rl_hip_stream_create", C.byref(h))
    streams.append(h)
# the process's first two allocation-free calls, on two streams, no host sync between
call("rl_hip_gemm_kquant_noalloc", ops.Q4_K, lin.w.ptr, xd.ptr, ys[1].ptr, m, n, T, 0, streams[0])
call("rl_hip_gemm_kquant_noalloc", ops.Q4_K, lin.w.ptr, xd.ptr, ys[2].ptr, m, n, T, 0, streams[1])
for h in streams:
    call("rl_hip_stream_synchronize", h)
want = ys[0].numpy(np.float32, (T, m)).view(np.uint32)
for y in ys[1:]:
    assert np.array_equal(y.numpy(np.float32, (T, m)).view(np.uint32), want)
for h in streams:
    call("rl_hip_stream_destroy", h)
print("FIRST_USE_OK")
"""


def test_noalloc_first_use_on_two_streams(gpu):
    # a fresh process, so these are the library's first allocation-free calls
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p = subprocess.run([sys.executable, "-c", FIRST_USE.format(root=root)], capture_output=True, text=True,
                       timeout=110)
    assert p.returncode == 0 and "FIRST_USE_OK" in p.stdout, p.stdout[-2000:] + p.stderr[-2000:]
