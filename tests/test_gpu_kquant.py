"""GPU parity: GGUF Q4_K / Q6_K dequant (bit-exact) and dequant-dot GEMV
(<= 1e-3 relative L2) against the CPU oracle."""
import numpy as np
import pytest

from rapidllm_amd import ops, synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _blocks(kind, r, m, n):
    return (synth.q4k_blocks if kind == "q4k" else synth.q6k_blocks)(r, m, n)


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_dequant_bitexact(gpu, orc, kind):
    r = synth.rng(31)
    m, n = 37, 4096
    blocks = _blocks(kind, r, m, n)
    # edge blocks: zero scale, maximal 6-bit scales/mins, fp16 subnormal d
    flat = blocks.reshape(-1, 144 if kind == "q4k" else 210)
    flat[0, :] = 0
    flat[1, :] = 0xFF
    if kind == "q4k":
        flat[1, 0:4] = np.frombuffer(np.array([6.0e-8, 3.0e-5], np.float16).tobytes(), np.uint8)
    else:
        flat[1, 208:210] = np.frombuffer(np.array([6.0e-8], np.float16).tobytes(), np.uint8)
    packed = np.ascontiguousarray(flat.reshape(-1))
    fn_gpu = ops.dequant_q4_k if kind == "q4k" else ops.dequant_q6_k
    fn_orc = orc.dequant_q4_k if kind == "q4k" else orc.dequant_q6_k
    got = fn_gpu(packed, m * n)
    want = fn_orc(packed, m * n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
@pytest.mark.parametrize("m,n", [(64, 256), (100, 1024), (1000, 2048), (5120, 17408)])
@pytest.mark.parametrize("T", [1, 2, 4, 8, 16])
def test_gemm_kquant_vs_oracle(gpu, orc, kind, m, n, T):
    if (m, n) == (5120, 17408) and T == 2:
        pytest.skip("full shape covered at T=1, 4, 8 and 16")
    r = synth.rng(41 + m + T)
    blocks = _blocks(kind, r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.KQuantLinear(ops.Q4_K if kind == "q4k" else ops.Q6_K, blocks, m, n)
    Y = ops.kquant_linear_T(lin, X)
    fo = orc.gemv_q4_k if kind == "q4k" else orc.gemv_q6_k
    for t in range(T):
        want = fo(blocks, X[t], m, n, 8)
        assert rel_l2(Y[t], want) <= 1e-3, (kind, m, n, T, t, rel_l2(Y[t], want))


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_gemm_kquant_tokens_independent_of_T(gpu, kind):
    """Every row of a T = 4, 6, 8, 13 or 16 launch equals the T = 1 launch of that row
    bit for bit (one weight pass over token groups of four changes no sum order)."""
    r = synth.rng(5)
    m, n = 512, 4096
    blocks = _blocks(kind, r, m, n)
    X = r.standard_normal((16, n)).astype(np.float32)
    lin = ops.KQuantLinear(ops.Q4_K if kind == "q4k" else ops.Q6_K, blocks, m, n)
    Y1 = [ops.kquant_linear_T(lin, X[t:t + 1])[0] for t in range(16)]
    for T in (4, 6, 8, 13, 16):
        YT = ops.kquant_linear_T(lin, X[:T])
        for t in range(T):
            assert np.array_equal(Y1[t].view(np.uint32), YT[t].view(np.uint32)), (T, t)


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
@pytest.mark.parametrize("m,n,T", [(17, 256, 3), (200, 4096, 3), (300, 3072, 1), (17, 256, 5), (200, 4096, 7),
                                   (300, 3072, 6)])
def test_gemm_kquant_ragged_and_odd_T(gpu, orc, kind, m, n, T):
    """Row counts that leave a partial 16-row tile and a partial 4-tile workgroup,
    one super-block per row, three tokens (the second token set half empty)."""
    r = synth.rng(7 + m + n + T)
    blocks = _blocks(kind, r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.KQuantLinear(ops.Q4_K if kind == "q4k" else ops.Q6_K, blocks, m, n)
    Y = ops.kquant_linear_T(lin, X)
    fo = orc.gemv_q4_k if kind == "q4k" else orc.gemv_q6_k
    for t in range(T):
        assert rel_l2(Y[t], fo(blocks, X[t], m, n, 8)) <= 1e-3, (kind, m, n, T, t)


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_gemm_kquant_extreme_blocks(gpu, orc, kind):
    """Maximal 6-bit scales / mins and quants (all-ones bytes), zero scales and an
    fp16 subnormal d, mixed into random blocks."""
    r = synth.rng(77)
    m, n = 128, 2048
    blocks = _blocks(kind, r, m, n)
    bb = 144 if kind == "q4k" else 210
    flat = blocks.reshape(-1, bb)
    flat[::7] = 0xFF
    if kind == "q4k":
        flat[::7, 0:4] = np.frombuffer(np.array([1e-3, 2e-3], np.float16).tobytes(), np.uint8)
        flat[3::11, 0:2] = 0
        flat[5::13, 0:2] = np.frombuffer(np.array([6.0e-8], np.float16).tobytes(), np.uint8)
    else:
        flat[::7, 208:210] = np.frombuffer(np.array([1e-3], np.float16).tobytes(), np.uint8)
        flat[3::11, 192:208] = 0
        flat[5::13, 208:210] = np.frombuffer(np.array([6.0e-8], np.float16).tobytes(), np.uint8)
    X = r.standard_normal((2, n)).astype(np.float32)
    lin = ops.KQuantLinear(ops.Q4_K if kind == "q4k" else ops.Q6_K, blocks, m, n)
    Y = ops.kquant_linear_T(lin, X)
    fo = orc.gemv_q4_k if kind == "q4k" else orc.gemv_q6_k
    for t in range(2):
        assert rel_l2(Y[t], fo(blocks, X[t], m, n, 8)) <= 1e-3, (kind, t)


def test_gemm_kquant_repeat_and_accumulate(gpu):
    """Split-K launches share ticket counters that the last workgroup of each row
    group resets: back-to-back launches must give bit-identical results, and the
    accumulate mode adds the product to Y."""
    from rapidllm_amd.hip import DeviceBuffer
    r = synth.rng(12)
    m, n, T = 5120, 17408, 2
    blocks = synth.q4k_blocks(r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.KQuantLinear(ops.Q4_K, blocks, m, n)
    ws = ops.kquant_workspace(m, n, T)
    xd = DeviceBuffer.from_numpy(X)
    outs = []
    for _ in range(3):
        yd = DeviceBuffer(4 * T * m)
        lin.forward(xd.ptr, yd.ptr, T, ws)
        outs.append(yd.numpy(np.float32, (T, m)))
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    Y0 = r.standard_normal((T, m)).astype(np.float32)
    yd = DeviceBuffer.from_numpy(Y0)
    lin.forward(xd.ptr, yd.ptr, T, ws, accumulate=True)
    got = yd.numpy(np.float32, (T, m))
    assert rel_l2(got, Y0 + outs[0]) <= 1e-6


def test_gemm_kquant_two_streams_own_workspaces(gpu):
    """Split-K tickets live in the caller's workspace: two streams, each with its
    own workspace, running interleaved K-quant GEMVs (launched without waiting for
    each other) give the serial results bit for bit."""
    import ctypes as C

    from rapidllm_amd.hip import DeviceBuffer, call
    r = synth.rng(13)
    m, n, T = 5120, 17408, 4
    lin = ops.KQuantLinear(ops.Q6_K, synth.q6k_blocks(r, m, n), m, n)
    X = [r.standard_normal((T, n)).astype(np.float32) for _ in range(2)]
    want = [ops.kquant_linear_T(lin, x) for x in X]
    streams = [C.c_void_p(), C.c_void_p()]
    for s in streams:
        call("rl_hip_stream_create", C.byref(s))
    try:
        ws = [ops.kquant_workspace(m, n, T) for _ in range(2)]
        xd = [DeviceBuffer.from_numpy(x) for x in X]
        yd = [[DeviceBuffer(4 * T * m) for _ in range(8)] for _ in range(2)]
        for i in range(8):
            for k in range(2):
                lin.forward(xd[k].ptr, yd[k][i].ptr, T, ws[k], stream=streams[k].value)
        for s in streams:
            call("rl_hip_stream_synchronize", s.value)
        for k in range(2):
            for i in range(8):
                got = yd[k][i].numpy(np.float32, (T, m))
                assert np.array_equal(got.view(np.uint32), want[k].view(np.uint32)), (k, i)
    finally:
        for s in streams:
            call("rl_hip_stream_destroy", s.value)


def test_synthetic_q4_k_engine_spec_invariant(gpu, monkeypatch):
    """The benchmark's device-generated K-quant model (RL_SYNTH_LINEAR=q4_k: Q4_K
    layer linears, Q6_K lm_head): T=4 verify with MTP drafts gives the tokens of
    plain T=1 decoding (the greedy invariant, tests/test_spec.cpp:46-79)."""
    from rapidllm_amd import model as M
    from rapidllm_amd.engine import Engine

    spec = M.ModelSpec(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4,
                       n_kv=2, layer_kinds=[0, 0, 0, 1])
    monkeypatch.setenv("RL_SYNTH_LINEAR", "q4_k")
    eng = Engine(spec, None, ctx=512, seed=5)
    off, _, _ = eng.generate([1, 2, 3], 12, spec_n=0)
    on, _, _ = eng.generate([1, 2, 3], 12, spec_n=3)
    assert on == off
    eng.close()


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
@pytest.mark.parametrize("I,n,T", [(8, 256, 1), (200, 1024, 3), (1024, 2048, 4), (200, 1024, 7), (17408, 5120, 1),
                                   (17408, 5120, 4), (17408, 5120, 8)])
def test_gemm_kquant_swiglu(gpu, orc, kind, I, n, T):
    """Gate / up half tiles with the SwiGLU write: against the oracle's two GEMVs
    and swiglu (<= 1e-3 relative L2), and against the same rows as one plain
    2I-row launch (gate rows then up rows: the same split and per-row sums)
    followed by silu(g) * u on the host (<= 1e-6; only exp's rounding differs)."""
    r = synth.rng(3 + I + n + T)
    qt = ops.Q4_K if kind == "q4k" else ops.Q6_K
    g = _blocks(kind, r, I, n)
    u = _blocks(kind, r, I, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    H = ops.KQuantGateUp(qt, g, u, I, n)(X)
    assert np.isfinite(H).all()
    cat = ops.KQuantLinear(qt, np.concatenate([g.reshape(-1), u.reshape(-1)]), 2 * I, n)
    GU = ops.kquant_linear_T(cat, X).astype(np.float64)
    with np.errstate(over="ignore"):  # exp(-g) overflows to inf for very negative g: silu -> 0
        host = GU[:, :I] / (1.0 + np.exp(-GU[:, :I])) * GU[:, I:]
    assert rel_l2(H, host) <= 1e-6, rel_l2(H, host)
    fo = orc.gemv_q4_k if kind == "q4k" else orc.gemv_q6_k
    for t in range(min(T, 2) if I > 4096 else T):
        want = orc.swiglu(fo(g, X[t], I, n, 8), fo(u, X[t], I, n, 8))
        assert rel_l2(H[t], want) <= 1e-3, (t, rel_l2(H[t], want))
