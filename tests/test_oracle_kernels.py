"""Pins the CPU oracle (oracle/oracle.cpp) before anything is checked against it.

Each oracle function is checked against (a) the reference's own compiled CPU
kernels (oracle/_ref, built from /root/reference where present) and (b) something
the mathematics fixes independently: exhaustive closed forms, exact rational
arithmetic, inverse encoders, or special cases with known answers.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from rapidllm_amd import synth


def _ulp32(x):
    return np.spacing(np.float32(abs(x)))


# ---------------------------------------------------------------- conversions


def e4m3_closed_form(c):
    """OCP e4m3fn from the spec: sign, 4-bit exponent (bias 7), 3-bit mantissa."""
    s = -1.0 if c & 0x80 else 1.0
    e = (c >> 3) & 0xF
    m = c & 7
    if e == 15 and m == 7:
        return math.nan
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8) * 2.0 ** (e - 7)


def test_e4m3_exhaustive_closed_form(orc):
    L = orc.lib()
    for c in range(256):
        want = e4m3_closed_form(c)
        got = L.orc_e4m3_to_f32(c)
        if math.isnan(want):
            assert math.isnan(got)
        else:
            assert got == want and math.copysign(1, got) == math.copysign(1, want), c
    # known anchor values of the format
    assert L.orc_e4m3_to_f32(0x7E) == 448.0
    assert L.orc_e4m3_to_f32(0x01) == 2.0 ** -9
    assert L.orc_e4m3_to_f32(0x38) == 1.0


def test_e4m3_matches_reference(orc, ref_lib):
    for c in range(256):
        a, b = orc.lib().orc_e4m3_to_f32(c), ref_lib.ref_e4m3_to_f32(c)
        assert (math.isnan(a) and math.isnan(b)) or np.float32(a).tobytes() == np.float32(b).tobytes()


def test_fp16_decode_exhaustive(orc):
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    L = orc.lib()
    got = np.array([L.orc_fp16_to_f32(int(c)) for c in codes], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp16_decode_matches_reference(orc, ref_lib):
    L = orc.lib()
    for c in range(0, 65536, 7):
        a, b = L.orc_fp16_to_f32(c), ref_lib.ref_fp16_to_f32(c)
        assert (math.isnan(a) and math.isnan(b)) or np.float32(a).tobytes() == np.float32(b).tobytes()


def test_f32_to_fp16_rne_matches_numpy(orc):
    r = synth.rng(11)
    L = orc.lib()
    vals = np.concatenate([
        r.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** r.integers(-8, 6, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    # halfway cases between fp16 neighbours (ties to even)
    h = np.arange(0, 0x7bff, 97, dtype=np.uint16).view(np.float16).astype(np.float32)
    h2 = (np.arange(1, 0x7c00, 97, dtype=np.uint16)).view(np.float16).astype(np.float32)
    n = min(len(h), len(h2))
    vals = np.concatenate([vals, ((h[:n].astype(np.float64) + h2[:n]) / 2).astype(np.float32)])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f32_to_fp16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- FP8 GEMV


def test_gemv_fp8_exact_rational(orc):
    """Tiny shapes with scale blocks that straddle rows/cols: compare with the exact
    rational sum (the reference accumulates in double, so within 1 fp32 ulp)."""
    r = synth.rng(1)
    for m, n in [(3, 5), (130, 257), (129, 131)]:
        W = synth.fp8_weight(r, m, n)
        s = synth.fp8_scales(r, m, n)
        x = r.standard_normal(n).astype(np.float32)
        y = orc.gemv_fp8(W, s, x)
        dec = [Fraction(e4m3_closed_form(c)) if c not in (0x7F, 0xFF) else None for c in range(256)]
        for i in range(0, m, max(1, m // 7)):
            acc = Fraction(0)
            for j in range(n):
                acc += dec[W[i, j]] * Fraction(float(s[i // 128, j // 128])) * Fraction(float(x[j]))
            exact = float(acc)
            assert abs(y[i] - exact) <= _ulp32(exact) + 1e-30, (m, n, i)


def test_gemv_fp8_matches_reference_bitexact(orc, ref_lib):
    r = synth.rng(2)
    m, n = 300, 1000
    W = synth.fp8_weight(r, m, n)
    s = synth.fp8_scales(r, m, n)
    x = r.standard_normal(n).astype(np.float32)
    y = orc.gemv_fp8(W, s, x)
    yr = np.empty(m, np.float32)
    ref_lib.ref_gemv_fp8(orc.P(W, orc._u8), orc.P(s), orc.P(x), orc.P(yr), m, n)
    assert np.array_equal(y.view(np.uint32), yr.view(np.uint32))


# ---------------------------------------------------------------- K-quants


def encode_q4k_scales(sc, mn):
    """Pack eight 6-bit scales and mins into 12 bytes (inverse of the decoder:
    GGUF Q4_K layout, j<4 low 6 bits of bytes j / j+4; j>=4 low nibble in byte j+4
    (scale) / high nibble (min), top 2 bits in bytes j-4 (scale) / j (min))."""
    b = [0] * 12
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(b)


def test_q4k_hand_built_block(orc):
    d, dmin = 0.5, 0.25
    sc = [1, 2, 3, 4, 33, 47, 60, 63]
    mn = [0, 5, 10, 15, 20, 41, 52, 63]
    q = np.array([(i * 7 + 3) & 0xFF for i in range(128)], np.uint8)
    blk = (np.float16(d).tobytes() + np.float16(dmin).tobytes() + encode_q4k_scales(sc, mn) + q.tobytes())
    out = orc.dequant_q4_k(np.frombuffer(blk, np.uint8).copy(), 256)
    for j in range(8):
        g, hi = divmod(j, 2)
        nib = (q[32 * g: 32 * g + 32] >> 4) if hi else (q[32 * g: 32 * g + 32] & 15)
        want = np.float32(d) * sc[j] * nib.astype(np.float32) - np.float32(dmin) * mn[j]
        # d, dmin, sc are small powers-of-two multiples: every value is exact
        assert np.array_equal(out[32 * j: 32 * j + 32], want), j


def test_q6k_hand_built_block(orc):
    d = 0.125
    vals = np.array([((i * 37) % 64) for i in range(256)], np.int64)  # 6-bit codes
    sc = np.array([-128, -7, -1, 0, 1, 2, 5, 9, 17, 33, 65, 127, -64, -33, 3, 100], np.int8)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for half in range(2):
        for l in range(32):
            v = [vals[128 * half + l + 32 * k] for k in range(4)]
            ql[64 * half + l] = (v[0] & 15) | ((v[2] & 15) << 4)
            ql[64 * half + l + 32] = (v[1] & 15) | ((v[3] & 15) << 4)
            qh[32 * half + l] = (v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6)
    blk = ql.tobytes() + qh.tobytes() + sc.tobytes() + np.float16(d).tobytes()
    out = orc.dequant_q6_k(np.frombuffer(blk, np.uint8).copy(), 256)
    for idx in range(256):
        half, rem = divmod(idx, 128)
        s = sc[8 * half + (rem % 32) // 16 + 2 * (rem // 32)]
        assert out[idx] == np.float32(d) * np.float32(s) * np.float32(vals[idx] - 32), idx


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_kquant_dequant_matches_reference_bitexact(orc, ref_lib, kind):
    r = synth.rng(3)
    m, n = 4, 2048
    blocks = (synth.q4k_blocks if kind == "q4k" else synth.q6k_blocks)(r, m, n)
    flat = np.ascontiguousarray(blocks.reshape(-1))
    ours = (orc.dequant_q4_k if kind == "q4k" else orc.dequant_q6_k)(flat, m * n)
    theirs = np.empty(m * n, np.float32)
    fn = ref_lib.ref_dequant_q4_k if kind == "q4k" else ref_lib.ref_dequant_q6_k
    fn(orc.P(flat, orc._u8), orc.P(theirs), m * n)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_kquant_gemv_matches_reference_bitexact(orc, ref_lib, kind):
    r = synth.rng(4)
    m, n = 96, 2048
    blocks = (synth.q4k_blocks if kind == "q4k" else synth.q6k_blocks)(r, m, n)
    x = r.standard_normal(n).astype(np.float32)
    ours = (orc.gemv_q4_k if kind == "q4k" else orc.gemv_q6_k)(blocks, x, m, n)
    theirs = np.empty(m, np.float32)
    fn = ref_lib.ref_gemv_q4_k if kind == "q4k" else ref_lib.ref_gemv_q6_k
    fn(orc.P(blocks, orc._u8), orc.P(x), orc.P(theirs), m, n)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_kquant_gemv_is_dequant_dot(orc):
    """gemv == dot(dequant(row), x) per super-block (structure, not formula)."""
    r = synth.rng(5)
    m, n = 8, 1024
    blocks = synth.q6k_blocks(r, m, n)
    x = r.standard_normal(n).astype(np.float32)
    y = orc.gemv_q6_k(blocks, x, m, n)
    for i in range(m):
        w = orc.dequant_q6_k(np.ascontiguousarray(blocks[i]), n).astype(np.float64)
        assert abs(y[i] - w @ x) <= 1e-4 * (np.abs(w) @ np.abs(x))


# ---------------------------------------------------------------- norms / conv / delta


def test_rmsnorm_constant_vector(orc):
    n = 256
    x = np.full(n, 3.0, np.float32)
    g = np.linspace(-0.5, 0.5, n).astype(np.float32)
    y = orc.qwen3_rmsnorm(x, g, 1e-6)
    want = 3.0 / math.sqrt(9.0 + 1e-6) * (1 + g.astype(np.float64))
    assert np.allclose(y, want, rtol=1e-6)


def test_norms_match_reference(orc, ref_lib):
    r = synth.rng(6)
    x = r.standard_normal(6144).astype(np.float32)
    z = r.standard_normal(6144).astype(np.float32)
    g = r.standard_normal(128).astype(np.float32)
    y = orc.gated_rmsnorm(x, z, g, 1e-6, 128)
    yr = np.empty_like(y)
    ref_lib.ref_gated_rmsnorm(orc.P(x), orc.P(z), orc.P(g), orc.P(yr), 6144, 1e-6, 128)
    assert np.array_equal(y, yr)
    gg = r.standard_normal(5120).astype(np.float32)
    xx = r.standard_normal(5120).astype(np.float32)
    a = orc.qwen3_rmsnorm(xx, gg)
    b = np.empty_like(a)
    ref_lib.ref_qwen3_rmsnorm(orc.P(xx), orc.P(gg), orc.P(b), 5120, 1e-6)
    # the reference takes its AVX path for n >= 64 (float partial sums)
    assert np.allclose(a, b, rtol=2e-6, atol=1e-7)


def test_conv1d_identity_tap_and_shift(orc):
    dim, k = 16, 4
    w = np.zeros((dim, k), np.float32)
    w[:, k - 1] = 1.0
    st = np.arange(dim * k, dtype=np.float32).reshape(dim, k)
    old = st.copy()
    x = np.linspace(-2, 2, dim).astype(np.float32)
    y = orc.conv1d_update(x, w, st)
    assert np.array_equal(st[:, :k - 1], old[:, 1:]) and np.array_equal(st[:, k - 1], x)
    assert np.allclose(y, x / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6)


def test_conv1d_matches_reference(orc, ref_lib):
    r = synth.rng(7)
    dim, k = 10240, 4
    w = r.standard_normal((dim, k)).astype(np.float32)
    st = r.standard_normal((dim, k)).astype(np.float32)
    st2 = st.copy()
    x = r.standard_normal(dim).astype(np.float32)
    y = orc.conv1d_update(x, w, st)
    yr = np.empty(dim, np.float32)
    ref_lib.ref_conv1d_update(orc.P(x), orc.P(w), orc.P(st2), orc.P(yr), dim, k)
    assert np.array_equal(y, yr) and np.array_equal(st, st2)


def test_delta_step_closed_forms(orc):
    nv, dk, dv = 3, 8, 8
    r = synth.rng(8)
    q = r.standard_normal((nv, dk)).astype(np.float32)
    k = r.standard_normal((nv, dk)).astype(np.float32)
    v = r.standard_normal((nv, dv)).astype(np.float32)
    qn = q / np.sqrt((q.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6) / math.sqrt(dk)
    kn = k / np.sqrt((k.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6)
    # zero state, beta = 1, no decay: S' = k v^T, o = v (k.q)
    S = np.zeros((nv, dk, dv), np.float32)
    o = orc.delta_step(S, q, k, v, np.ones(nv, np.float32), np.zeros(nv, np.float32))
    assert np.allclose(S, kn[:, :, None] * v[:, None, :], rtol=1e-5, atol=1e-6)
    assert np.allclose(o, v * (kn * qn).sum(1, keepdims=True), rtol=1e-4, atol=1e-6)
    # beta = 0: only decay; o = exp(g) S^T q
    S0 = r.standard_normal((nv, dk, dv)).astype(np.float32)
    S = S0.copy()
    gl = np.array([-0.5, -1.0, -2.0], np.float32)
    o = orc.delta_step(S, q, k, v, np.zeros(nv, np.float32), gl)
    dec = np.exp(gl)[:, None, None]
    assert np.allclose(S, S0 * dec, rtol=1e-6)
    assert np.allclose(o, np.einsum("hij,hi->hj", S0 * dec, qn), rtol=1e-4, atol=1e-6)


def test_delta_step_matches_reference(orc, ref_lib):
    r = synth.rng(9)
    nv, dk, dv = 48, 128, 128
    S = (r.standard_normal((nv, dk, dv)) * 0.02).astype(np.float32)
    S2 = S.copy()
    q = r.standard_normal((nv, dk)).astype(np.float32)
    k = r.standard_normal((nv, dk)).astype(np.float32)
    v = r.standard_normal((nv, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-r.standard_normal(nv)))).astype(np.float32)
    gl = (-np.log1p(np.exp(r.standard_normal(nv)))).astype(np.float32)
    o = orc.delta_step(S, q, k, v, beta, gl)
    o2 = np.empty_like(o)
    ref_lib.ref_delta_step_scalar(orc.P(S2), orc.P(q), orc.P(k), orc.P(v), orc.P(beta), orc.P(gl), orc.P(o2),
                                  nv, dk, dv, 1e-6)
    assert np.array_equal(o, o2) and np.array_equal(S, S2)


def test_gates_closed_form(orc):
    a = np.array([-30.0, -1.0, 0.0, 2.0, 40.0], np.float32)
    b = np.array([-3.0, 0.0, 1.0, 5.0, -40.0], np.float32)
    A = np.array([0.0, 0.5, -1.0, 1.0, 0.0], np.float32)
    dt = np.array([0.0, 1.0, 0.5, -2.0, 0.0], np.float32)
    beta, gl = orc.gdn_gates(a, b, A, dt)
    x = a.astype(np.float64) + dt
    assert np.allclose(beta, 1 / (1 + np.exp(-b.astype(np.float64))), rtol=1e-6)
    assert np.allclose(gl, -np.exp(A.astype(np.float64)) * np.logaddexp(0, x), rtol=1e-6, atol=1e-30)


# ---------------------------------------------------------------- attention / rope / argmax


def test_rope_rotation_properties(orc):
    nq, nkv, hd, rot = 2, 1, 256, 64
    r = synth.rng(10)
    q = r.standard_normal(nq * hd).astype(np.float32)
    k = r.standard_normal(nkv * hd).astype(np.float32)
    q0, k0 = orc.rope_partial(q, k, nq, nkv, hd, rot, 0, 1e7)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q5, k5 = orc.rope_partial(q, k, nq, nkv, hd, rot, 5, 1e7)
    # dims beyond rotary untouched; pair norms preserved; dim 0 pair rotates by pos*1 rad
    assert np.array_equal(q5.reshape(nq, hd)[:, rot:], q.reshape(nq, hd)[:, rot:])
    qq, q5r = q.reshape(nq, hd), q5.reshape(nq, hd)
    assert np.allclose(qq[:, :32] ** 2 + qq[:, 32:64] ** 2, q5r[:, :32] ** 2 + q5r[:, 32:64] ** 2, rtol=1e-5)
    c, s = math.cos(5.0), math.sin(5.0)
    assert np.allclose(q5r[:, 0], qq[:, 0] * c - qq[:, 32] * s, rtol=1e-5)


def test_rope_matches_reference(orc, ref_lib):
    r = synth.rng(12)
    q = r.standard_normal(24 * 256).astype(np.float32)
    k = r.standard_normal(4 * 256).astype(np.float32)
    for pos in (0, 1, 777, 32767):
        a, b = orc.rope_partial(q, k, 24, 4, 256, 64, pos, 1e7)
        q2, k2 = q.copy(), k.copy()
        ref_lib.ref_rope_partial(orc.P(q2), orc.P(k2), 24, 4, 256, 64, pos, 1e7)
        assert np.array_equal(a, q2) and np.array_equal(b, k2)


def test_attn_decode_closed_forms(orc):
    nq, nkv, hd, L = 4, 2, 16, 9
    r = synth.rng(13)
    q = r.standard_normal(nq * hd).astype(np.float32)
    kc = np.tile(r.standard_normal(nkv * hd).astype(np.float32), (L, 1))  # identical keys
    vc = r.standard_normal((L, nkv * hd)).astype(np.float32)
    o = orc.attn_decode(q, kc, vc, L - 1, nq, nkv, hd).reshape(nq, hd)
    mean_v = vc.reshape(L, nkv, hd).mean(0)
    for h in range(nq):
        assert np.allclose(o[h], mean_v[h // (nq // nkv)], rtol=1e-5, atol=1e-6)
    # one dominant key per kv head -> output equals that value row
    kc2 = np.zeros((L, nkv * hd), np.float32)
    qd = np.zeros(nq * hd, np.float32)
    qd[::hd] = 1.0
    kc2[3, ::hd] = 4000.0
    o2 = orc.attn_decode(qd, kc2, vc, L - 1, nq, nkv, hd).reshape(nq, hd)
    for h in range(nq):
        assert np.allclose(o2[h], vc[3].reshape(nkv, hd)[h // 2], rtol=1e-6)


def test_attn_decode_matches_reference(orc, ref_lib):
    r = synth.rng(14)
    nq, nkv, hd, L = 24, 4, 256, 300
    q = r.standard_normal(nq * hd).astype(np.float32)
    kc = r.standard_normal((L, nkv * hd)).astype(np.float32)
    vc = r.standard_normal((L, nkv * hd)).astype(np.float32)
    o = orc.attn_decode(q, kc, vc, L - 1, nq, nkv, hd)
    o2 = np.empty_like(o)
    ref_lib.ref_attn_decode(orc.P(q), orc.P(kc), orc.P(vc), orc.P(o2), L - 1, nq, nkv, hd)
    assert np.array_equal(o, o2)


def test_greedy_ties_lowest_index(orc, ref_lib):
    x = np.array([1, 5, 5, -1, 5], np.float32)
    assert orc.greedy(x) == 1 == int(np.argmax(x))
    r = synth.rng(15)
    for _ in range(20):
        v = r.integers(-3, 3, 1000).astype(np.float32)
        assert orc.greedy(v) == int(np.argmax(v)) == ref_lib.ref_greedy(orc.P(v), v.size)


def test_accept_prefix(orc):
    import ctypes as C

    def acc(toks, preds):
        t = np.array(toks, np.int32)
        p = np.array(preds, np.int32)
        return orc.lib().orc_accept_prefix(t.ctypes.data_as(C.POINTER(C.c_int)), p.ctypes.data_as(C.POINTER(C.c_int)),
                                           len(toks))

    assert acc([7, 1, 2, 3], [1, 2, 3, 9]) == 4
    assert acc([7, 1, 2, 3], [1, 5, 3, 9]) == 2
    assert acc([7, 1, 2, 3], [0, 2, 3, 9]) == 1
    assert acc([7], [4]) == 1


def test_oracle_model_tiny_hybrid_golden(orc):
    """Whole-model pin: the oracle model reproduces the reference golden script's
    greedy tokens (forward(), tiny_hybrid.py:221-354) and MTP stem drafts
    (mtp_draft_py(), tiny_hybrid.py:357-430) on its 8-layer hybrid fixture."""
    from oracle.oracle import OracleModel
    from tests.tiny_hybrid import load

    spec, W, meta = load()
    m = OracleModel(spec, W, ctx=64, kv_fp16=False, threads=1)
    got, _, _ = m.generate(meta["prompt_ids"], len(meta["greedy_ids"]))
    assert got == meta["greedy_ids"]
    m.reset()
    for t in meta["prompt_ids"]:
        g, _, _ = m.decode(t)
    assert g == meta["greedy_ids"][0]
    drafts = m.mtp_draft(g, 3).tolist()
    assert drafts == meta["mtp_draft_ids"]


def test_gemm_fp8_rows_are_gemv(orc):
    """The T-row oracle GEMM is T independent GEMVs (the reference's CUDA T=4 verify
    runs four T=1 GEMVs, cuda_engine.cu:11997-12005), bit for bit."""
    r = synth.rng(21)
    m, n = 48, 384
    W, s = synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n)
    X = r.standard_normal((4, n)).astype(np.float32)
    Y = orc.gemm_fp8(W, s, X)
    for t in range(4):
        assert np.array_equal(Y[t], orc.gemv_fp8(W, s, X[t]))


def test_dense_gemv_f16_f32_error_bound(orc):
    """F16 / F32 linears (float accumulator, ops.cpp:165-172 restated for f32 in
    double): against an exact float64 product within fp32 summation error."""
    r = synth.rng(22)
    m, n = 16, 300
    W = r.standard_normal((m, n)).astype(np.float16)
    x = r.standard_normal(n).astype(np.float32)
    exact = W.astype(np.float64) @ x.astype(np.float64)
    bound = 1.2e-7 * n * (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(orc.gemv_f16(W.view(np.uint16), x) - exact) <= bound)
    W32 = W.astype(np.float32)
    assert np.all(np.abs(orc.gemv_f32(W32, x) - exact) <= bound)


def test_argmax_rows_matches_numpy(orc):
    r = synth.rng(23)
    L = r.integers(-5, 5, (6, 1000)).astype(np.float32)
    assert np.array_equal(orc.argmax_rows(L), np.argmax(L, axis=1))


def test_oracle_mtp_layer_draft_equals_reference_composition(orc, ref_lib):
    """The oracle's MTP decoder-layer draft against Session::mtp_layer_step composed
    from the reference's own kernels (session.cpp:561-617 after the stem of
    :650-680): per draft i, h' = gemv_fp8(fc, [norm_e(embed tok); norm_h(h)]), then
    ops::fused_attn_decode with the mtp.layers[0] weights at position i of a cache
    zeroed per call, ops::fused_mlp_decode, qwen3_rmsnorm(mtp.norm), gemv_bf16
    (lm_head) and greedy_sample.  Drafts equal; the last hidden within 1e-6
    relative L2 (the reference's SIMD RMSNorm / SwiGLU inside the fused decode
    functions round a few last bits differently from the scalar restatement)."""
    from oracle.oracle import OracleModel, P, _u8, _u16
    from rapidllm_amd import model as M

    spec = M.ModelSpec(vocab=300, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4,
                       n_kv=2, head_dim=64, rotary_dim=16, layer_kinds=[0, 0, 0, 1], mtp_layer=True)
    W = M.random_weights(spec, seed=21, w_scale=(1e-3, 1e-2))
    t = {n: (q, d, r, c, s) for n, (q, r, c, d, s) in W.t.items()}
    om = OracleModel(spec, W, ctx=64, kv_fp16=False, threads=1)
    hid = []
    for tok in [5, 17, 42, 99]:
        g, _, h = om.decode(tok)
        hid.append(h)
    H, V, hd, nq, nkv = spec.hidden, spec.vocab, spec.head_dim, spec.n_q, spec.n_kv
    R = ref_lib

    def f32(n):
        return np.ascontiguousarray(t[n][1], np.float32)

    def fp8(n):
        return np.ascontiguousarray(t[n][1], np.uint8), np.ascontiguousarray(t[n][4], np.float32)

    def rms(x, n):
        y = np.empty_like(x)
        R.ref_qwen3_rmsnorm(P(x), P(f32(n)), P(y), H, spec.rms_eps)
        return y

    emb = t["embed"][1].reshape(V, H)
    n = 4
    kc = np.zeros(n * nkv * hd, np.float32)
    vc = np.zeros_like(kc)
    tok, drafts = g, []
    for i in range(n):
        href = hid[-1] if i == 0 else hid[-2]
        er = synth.bf16_to_f32(emb[tok]).astype(np.float32)
        cat = np.concatenate([rms(er, "mtp.pre_fc_norm_embedding"), rms(href, "mtp.pre_fc_norm_hidden")])
        hp = np.empty(H, np.float32)
        w, s = fp8("mtp.fc")
        R.ref_gemv_fp8(P(w, _u8), P(s), P(cat), P(hp), H, 2 * H)
        p = "mtp.layers[0]."
        q, k, v, o = fp8(p + "attn.wq"), fp8(p + "attn.wk"), fp8(p + "attn.wv"), fp8(p + "attn.wo")
        R.ref_fused_attn(P(f32(p + "attn_norm")), P(q[0], _u8), P(q[1]), P(k[0], _u8), P(k[1]), P(v[0], _u8),
                         P(v[1]), P(o[0], _u8), P(o[1]), P(f32(p + "attn.q_norm")), P(f32(p + "attn.k_norm")),
                         P(kc), P(vc), P(hp), H, nq, nkv, hd, spec.rotary_dim, i, spec.rope_theta, spec.rms_eps)
        gt, up, dn = fp8(p + "mlp.gate"), fp8(p + "mlp.up"), fp8(p + "mlp.down")
        R.ref_fused_mlp(P(f32(p + "ffn_norm")), P(gt[0], _u8), P(gt[1]), P(up[0], _u8), P(up[1]), P(dn[0], _u8),
                        P(dn[1]), P(hp), H, spec.intermediate, spec.rms_eps)
        lg = np.empty(V, np.float32)
        R.ref_gemv_bf16(P(np.ascontiguousarray(t["lm_head"][1], np.uint16), _u16), P(rms(hp, "mtp.norm")), P(lg), V, H)
        tok = R.ref_greedy(P(lg), V)
        drafts.append(tok)
    om.set_mtp_mode(1)
    got = om.mtp_draft(g, n).tolist()
    assert got == drafts
    got_h = om.mtp_hidden().astype(np.float64)
    assert np.linalg.norm(got_h - hp) / np.linalg.norm(hp) < 1e-6
    # the stem alone drafts from a different hidden (the layer is not a no-op)
    om.set_mtp_mode(0)
    om.mtp_draft(g, n)
    assert not np.allclose(om.mtp_hidden(), hp)
