"""GPU parity: block-FP8 / BF16 skinny GEMM and e4m3 decode vs the CPU oracle.

Tolerances: decode bit-exact; fp32 outputs within 1e-3
relative L2 of the reference CPU result.
"""
import numpy as np
import pytest

from rapidllm_amd import hip, ops, synth

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def test_e4m3_decode_bitexact(gpu, orc):
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    got = ops.e4m3_to_f32(codes)
    want = np.array([orc.lib().orc_e4m3_to_f32(int(c)) for c in codes], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m,n", [(64, 512), (300, 1000), (17, 130), (1024, 5120)])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16])
def test_gemm_fp8_vs_oracle(gpu, orc, m, n, T):
    r = synth.rng(100 + m + n + T)
    W = synth.fp8_weight(r, m, n)
    s = synth.fp8_scales(r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.Fp8Linear(W, s)
    Y = ops.linear_T(lin, X)
    Yo = orc.gemm_fp8(W, s, X)
    for t in range(T):
        assert rel_l2(Y[t], Yo[t]) <= REL_L2, (m, n, T, t, rel_l2(Y[t], Yo[t]))


@pytest.mark.parametrize("T", [4, 8, 13, 16])
def test_gemm_fp8_tokens_independent_of_T(gpu, T):
    """Token t's output is bit-identical whether it runs alone (T=1) or inside a
    T=4 verify or a batch of 8 rows: the greedy invariant needs T=4 == 4 x T=1
    exactly, and a batch slot's token equals the single-sequence step's."""
    r = synth.rng(7)
    m, n = 2048, 5120
    W = synth.fp8_weight(r, m, n)
    s = synth.fp8_scales(r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.Fp8Linear(W, s)
    YT = ops.linear_T(lin, X)
    for t in range(T):
        Y1 = ops.linear_T(lin, X[t:t + 1])[0]
        assert np.array_equal(Y1.view(np.uint32), YT[t].view(np.uint32)), t


def test_gemm_fp8_config1_full_shape(gpu, orc):
    """W[17408x5120] e4m3, log-uniform scales, x ~ N(0,1)."""
    r = synth.rng(0xC1)
    m, n = 17408, 5120
    W = synth.fp8_weight(r, m, n)
    s = synth.fp8_scales(r, m, n)
    x = r.standard_normal(n).astype(np.float32)
    y = ops.gemv_fp8(W, s, x)
    yo = orc.gemv_fp8(W, s, x)
    assert rel_l2(y, yo) <= REL_L2, rel_l2(y, yo)


@pytest.mark.parametrize("m,T", [(16480, 1), (16480, 4), (16400, 2)])
def test_gemm_fp8_overflow_row_tiles(gpu, orc, m, T):
    """Launches with a few row tiles past two workgroups per CU (the DeltaNet in_proj:
    16480 rows = 1030 tiles) give the overflow tiles single-tile workgroups; every
    row, including the last ones, matches the oracle."""
    r = synth.rng(900 + m + T)
    n = 512
    W, s = synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    Y = ops.linear_T(ops.Fp8Linear(W, s), X)
    Yo = orc.gemm_fp8(W, s, X)
    for t in range(T):
        assert rel_l2(Y[t], Yo[t]) <= REL_L2
        tail = slice(m - 6 * 16, m)
        assert rel_l2(Y[t][tail], Yo[t][tail]) <= REL_L2


def test_gemm_fp8_large_activations(gpu, orc):
    """Activations far outside fp16 range (the split keeps fp32's exponent range)."""
    r = synth.rng(8)
    m, n = 256, 1024
    W = synth.fp8_weight(r, m, n)
    s = synth.fp8_scales(r, m, n)
    X = (r.standard_normal((2, n)) * np.float32(1e6)).astype(np.float32)
    X[1] *= np.float32(1e-12)
    Y = ops.linear_T(ops.Fp8Linear(W, s), X)
    Yo = orc.gemm_fp8(W, s, X)
    for t in range(2):
        assert rel_l2(Y[t], Yo[t]) <= REL_L2


@pytest.mark.parametrize("m,n,T", [(96, 512, 1), (1000, 384, 4), (5120, 5120, 3), (700, 640, 8), (2048, 1024, 6), (1500, 768, 16),
                                   (300, 256, 11)])
def test_gemm_bf16_vs_oracle(gpu, orc, m, n, T):
    r = synth.rng(200 + m)
    Wf = r.standard_normal((m, n)).astype(np.float32)
    Wb = synth.bf16_bits(Wf)
    X = r.standard_normal((T, n)).astype(np.float32)
    Y = ops.linear_T(ops.Bf16Linear(Wb), X)
    for t in range(T):
        yo = orc.gemv_bf16(Wb, X[t])
        assert rel_l2(Y[t], yo) <= REL_L2


def _time_gemm(lin, X, epi, split=4, frag_out=None, ss_in=None):
    """One launch through rl_hip_time_gemm_fp8 (iters=1): exposes the split-K and
    SwiGLU epilogues the engine uses on the real GEMM kernel."""
    import ctypes as C

    from rapidllm_amd.hip import DeviceBuffer, call

    T, n = X.shape
    m = lin.m
    xd = DeviceBuffer.from_numpy(np.ascontiguousarray(X, np.float32))
    frag = ops.act_frag_buffer(n, T)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, n, T, None)
    rows = split * T * m if epi == 3 else T * (m // 2 if epi in (2, 5) else m)
    yd = DeviceBuffer(4 * rows)
    yd.zero()
    ptrs = (C.c_void_p * 1)(lin.w.ptr)
    ms = C.c_float()
    ssd = DeviceBuffer.from_numpy(np.ascontiguousarray(ss_in, np.float32)) if ss_in is not None else None
    call("rl_hip_time_gemm_fp8", ptrs, 1, lin.ts.ptr, frag.ptr, yd.ptr, frag_out, None, None, None,
         ssd.ptr if ssd else None, m, n, T, epi,
         split, 1, None, C.byref(ms))
    return yd.numpy(np.float32, (rows,))


@pytest.mark.parametrize("T", [1, 4])
def test_gemm_fp8_split_k_partials(gpu, orc, T):
    """Split-K epilogue (residual GEMMs: out_proj, o_proj, down): 4 partial slices
    whose sum is the product, as the next RMSNorm kernel consumes them."""
    r = synth.rng(300 + T)
    m, n = 5120, 6144
    W, s = synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.Fp8Linear(W, s)
    P = _time_gemm(lin, X, 3).reshape(4, T, m)
    Yo = orc.gemm_fp8(W, s, X)
    Y = P.astype(np.float64).sum(0)
    for t in range(T):
        assert rel_l2(Y[t], Yo[t]) <= REL_L2, (t, rel_l2(Y[t], Yo[t]))
    assert np.any(P[1] != 0) and np.any(P[3] != 0)  # every slice did work


@pytest.mark.parametrize("T", [1, 3, 7, 12])
def test_gemm_fp8_swiglu_epilogue(gpu, orc, T):
    """Gate/up interleaved by 16-row tile, SwiGLU in the epilogue:
    h = silu(gate . x) * (up . x) (ops_fused.cpp:66-82, ops.cpp:607-609)."""
    r = synth.rng(400 + T)
    I, n = 512, 1024
    Wg, Wu = synth.fp8_weight(r, I, n), synth.fp8_weight(r, I, n)
    # one scale per column block for every row, so row interleaving keeps the
    # 128x128 scale blocks valid for both source matrices
    col_s = synth.fp8_scales(r, 128, n)[0]
    sg = np.tile(col_s, (I // 128, 1))
    Wi = np.empty((2 * I, n), np.uint8)
    for k in range(I // 16):
        Wi[32 * k:32 * k + 16] = Wg[16 * k:16 * k + 16]
        Wi[32 * k + 16:32 * k + 32] = Wu[16 * k:16 * k + 16]
    lin = ops.Fp8Linear(Wi, np.tile(col_s, (2 * I // 128, 1)))
    X = r.standard_normal((T, n)).astype(np.float32)
    H = _time_gemm(lin, X, 2).reshape(T, I)
    g = orc.gemm_fp8(Wg, sg, X).astype(np.float64)
    u = orc.gemm_fp8(Wu, sg, X).astype(np.float64)
    with np.errstate(over="ignore"):
        want = g / (1 + np.exp(-g)) * u
    for t in range(T):
        assert rel_l2(H[t], want[t]) <= REL_L2, (t, rel_l2(H[t], want[t]))


def _unpack_frag(raw, n, T):
    """GEMM input fragments [kb][i][g][2T][8 bf16] -> fp32 [T][n] (hi + mid)."""
    u16 = raw.view(np.uint16).reshape(n // 128, 4, 4, 2 * T, 8)
    f = (u16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    val = f[:, :, :, :T, :] + f[:, :, :, T:, :]          # [kb][i][g][t][e]
    # column = kb*128 + 32g + 8i + e
    return val.transpose(3, 0, 2, 1, 4).reshape(T, n)


@pytest.mark.parametrize("T,block_scale,n", [(1, False, 1024), (4, False, 1024), (1, True, 1024), (4, True, 1024),
                                               (2, True, 10240), (8, False, 1024), (6, True, 1024), (16, False, 1024),
                                               (11, True, 1024), (16, True, 10240)])
def test_gemm_fp8_add_norm_epilogue(gpu, orc, T, block_scale, n):
    """Residual GEMM fused with the next RMSNorm's data: x += W.a in place,
    fragments of x * (1 + gamma) for the next linear, and sum of x^2 per row group.
    block_scale: the input's 128-column blocks are scaled per token by
    1/sqrt(sum/128 + 1e-6) of four given partial sums (the DeltaNet out_proj's
    folded gated RMSNorm; n = 10240: 80 heads, 10 blocks per wave)."""
    import ctypes as C

    from rapidllm_amd.hip import DeviceBuffer, call

    r = synth.rng(500 + T + n)
    m = 512
    W, s = synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n, 1e-3, 1e-2)
    lin = ops.Fp8Linear(W, s)
    X = r.standard_normal((T, n)).astype(np.float32)
    x0 = r.standard_normal((T, m)).astype(np.float32)
    gamma = (0.1 * r.standard_normal(m)).astype(np.float32)
    xd = DeviceBuffer.from_numpy(X)
    frag = ops.act_frag_buffer(n, T)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, n, T, None)
    yd = DeviceBuffer.from_numpy(x0)
    fo = ops.act_frag_buffer(m, T)
    gd = DeviceBuffer.from_numpy(gamma)
    G = hip.lib().rl_hip_norm_group_rows()
    ssd = DeviceBuffer(4 * T * (m // G))
    Xin = X
    bsd = None
    if block_scale:
        bsum = (r.random((n // 128, T, 4)) * 64 + 1).astype(np.float32)
        bsd = DeviceBuffer.from_numpy(bsum)
        sc = 1.0 / np.sqrt(bsum.astype(np.float64).sum(2) / 128 + 1e-6)  # [kb][t]
        Xin = (X.astype(np.float64) * np.repeat(sc.T, 128, axis=1)).astype(np.float32)
    ptrs = (C.c_void_p * 1)(lin.w.ptr)
    ms = C.c_float()
    call("rl_hip_time_gemm_fp8", ptrs, 1, lin.ts.ptr, frag.ptr, yd.ptr, fo.ptr, gd.ptr, ssd.ptr,
         bsd.ptr if bsd else None, None, m, n, T, 4, 1, 1, None, C.byref(ms))
    x = yd.numpy(np.float32, (T, m)).astype(np.float64)
    want = x0.astype(np.float64) + orc.gemm_fp8(W, s, Xin)
    for t in range(T):
        assert rel_l2(x[t], want[t]) <= REL_L2
    ss = ssd.numpy(np.float32, (m // G, T)).astype(np.float64)
    assert np.allclose(ss, (x ** 2).reshape(T, m // G, G).sum(2).T, rtol=1e-5)
    fr = _unpack_frag(fo.numpy(np.uint8, (fo.nbytes,)), m, T)
    xg = x * (1.0 + gamma.astype(np.float64))
    assert np.all(np.abs(fr - xg) <= 2.0 ** -15 * np.abs(xg) + 1e-30)


@pytest.mark.parametrize("T,I", [(1, 512), (3, 520), (4, 256), (6, 136), (8, 264), (16, 512), (10, 136)])
def test_gemm_fp8_swiglu_half_tiles(gpu, orc, T, I):
    """The engine's gate/up packing (rl_hip_pack_fp8_gate_up: tile k = gate rows
    8k..8k+7 then up rows 8k..8k+7, a block scale per half) with the SwiGLU epilogue
    5: h = silu(gate . x) * (up . x) against the oracle, gate and up with independent
    block scales.  I = 520 and 136 end in a partial 128-row scale block and give an
    odd tile count; T = 6 takes the runtime-T kernel."""
    r = synth.rng(700 + T + I)
    n = 1024
    Wg, Wu = synth.fp8_weight(r, I, n), synth.fp8_weight(r, I, n)
    sg, su = synth.fp8_scales(r, I, n), synth.fp8_scales(r, I, n)
    lin = ops.Fp8GateUp(Wg, sg, Wu, su)
    X = r.standard_normal((T, n)).astype(np.float32)
    Hh = _time_gemm(lin, X, 5).reshape(T, I)
    for t in range(T):
        g = orc.gemv_fp8(Wg, sg, X[t]).astype(np.float64)
        u = orc.gemv_fp8(Wu, su, X[t]).astype(np.float64)
        with np.errstate(over="ignore"):
            want = g / (1.0 + np.exp(-g)) * u
        assert rel_l2(Hh[t], want) <= REL_L2, (t, rel_l2(Hh[t], want))


@pytest.mark.parametrize("T", [1, 2, 4, 5, 8, 10, 16])
@pytest.mark.parametrize("epi", [0, 5])
def test_gemm_fp8_folded_norm_input(gpu, orc, T, epi):
    """Store and half-tile SwiGLU launches that read the residual stream's sums of
    squares (as the previous add-norm launch writes them: [ceil(n/32)][T]) and scale
    each token's products by 1/sqrt(sum / n + 1e-6): the RMSNorm folded into the
    consuming GEMM, its gamma already in the weights (ops.cpp:389-402 rmsnorm, then
    ops::linear)."""
    r = synth.rng(900 + 10 * T + epi)
    n = 1536
    X = r.standard_normal((T, n)).astype(np.float32)
    G = hip.lib().rl_hip_norm_group_rows()
    ss = (r.random(((n + G - 1) // G, T)) * 40 + 1).astype(np.float32)
    sc = 1.0 / np.sqrt(ss.astype(np.float64).sum(0) / n + 1e-6)  # [t]
    if epi == 0:
        m = 384
        W, s = synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n)
        Y = _time_gemm(ops.Fp8Linear(W, s), X, 0, ss_in=ss).reshape(T, m)
        want = orc.gemm_fp8(W, s, X).astype(np.float64) * sc[:, None]
    else:
        I = 264
        Wg, Wu = synth.fp8_weight(r, I, n), synth.fp8_weight(r, I, n)
        sg, su = synth.fp8_scales(r, I, n), synth.fp8_scales(r, I, n)
        Y = _time_gemm(ops.Fp8GateUp(Wg, sg, Wu, su), X, 5, ss_in=ss).reshape(T, I)
        g = orc.gemm_fp8(Wg, sg, X).astype(np.float64) * sc[:, None]
        u = orc.gemm_fp8(Wu, su, X).astype(np.float64) * sc[:, None]
        with np.errstate(over="ignore"):
            want = g / (1.0 + np.exp(-g)) * u
    for t in range(T):
        assert rel_l2(Y[t], want[t]) <= REL_L2, (t, rel_l2(Y[t], want[t]))


@pytest.mark.parametrize("m,n", [(100, 1024), (16480, 5120)])
def test_valu_gemv_comparison_kernel(gpu, orc, m, n):
    """The VALU T=1 GEMV that the bench times against the matrix-core kernel computes
    the same product (<= 1e-3 relative L2 against the oracle), so the comparison is
    between equal work."""
    import ctypes as C

    from rapidllm_amd.hip import DeviceBuffer, call

    r = synth.rng(900 + m)
    W, s = synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n, 1e-3, 1e-2)
    lin = ops.Fp8Linear(W, s)
    X = r.standard_normal((1, n)).astype(np.float32)
    xd = DeviceBuffer.from_numpy(X)
    yd = DeviceBuffer(4 * m)
    ptrs = (C.c_void_p * 1)(lin.w.ptr)
    ms = C.c_float()
    call("rl_hip_time_gemv_fp8_valu", ptrs, 1, lin.ts.ptr, xd.ptr, yd.ptr, m, n, 1, None, C.byref(ms))
    y = yd.numpy(np.float32, (m,))
    want = orc.gemm_fp8(W, s, X)[0] if m * n <= 1 << 20 else None
    if want is None:
        # large shape: against the matrix-core kernel (itself checked against the oracle)
        want = _time_gemm(lin, X, 0)[:m]
    assert rel_l2(y, want) <= REL_L2
