"""GPU parity of the prefill path (many prompt tokens per launch) against the CPU
oracle: block-FP8 linears on the matrix cores, 1e-3 relative L2 per token."""
import numpy as np
import pytest

from rapidllm_amd import ops, synth

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("m,n,T", [(64, 512, 1), (300, 1000, 17), (1000, 1536, 64), (129, 640, 100),
                                   (2048, 5120, 256)])
def test_gemm_prefill_vs_oracle(gpu, orc, m, n, T):
    r = synth.rng(300 + m + n + T)
    W = synth.fp8_weight(r, m, n)
    s = synth.fp8_scales(r, m, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    lin = ops.Fp8Linear(W, s)
    Y = ops.linear_prefill(lin, X)
    Yo = orc.gemm_fp8(W, s, X)
    for t in range(T):
        assert rel_l2(Y[t], Yo[t]) <= REL_L2, (m, n, T, t, rel_l2(Y[t], Yo[t]))


@pytest.mark.parametrize("T,I", [(70, 256), (200, 520)])
def test_gemm_prefill_swiglu_half_tiles(gpu, orc, T, I):
    """Prefill SwiGLU (epilogue 5) over the engine's half-tile gate/up packing,
    gate and up with independent block scales; I = 520 ends in a partial 128-row
    scale block."""
    r = synth.rng(43 + I)
    n = 768
    Wg, Wu = synth.fp8_weight(r, I, n), synth.fp8_weight(r, I, n)
    sg, su = synth.fp8_scales(r, I, n), synth.fp8_scales(r, I, n)
    X = r.standard_normal((T, n)).astype(np.float32)
    g = orc.gemm_fp8(Wg, sg, X).astype(np.float64)
    u = orc.gemm_fp8(Wu, su, X).astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    got = ops.linear_prefill(ops.Fp8GateUp(Wg, sg, Wu, su), X, epilogue=5)
    for t in range(T):
        assert rel_l2(got[t], want[t]) <= REL_L2, (t, rel_l2(got[t], want[t]))


@pytest.mark.parametrize("T,I", [(70, 256), (131, 384)])
def test_gemm_prefill_swiglu_to_fragments(gpu, T, I):
    """Epilogue 6 (SwiGLU half tiles written as the next GEMM's bf16 hi + mid
    fragments) is byte-identical to epilogue 5 followed by rl_hip_pack_act."""
    from rapidllm_amd.hip import DeviceBuffer, call
    r = synth.rng(47 + I)
    n = 512
    lin = ops.Fp8GateUp(synth.fp8_weight(r, I, n), synth.fp8_scales(r, I, n), synth.fp8_weight(r, I, n),
                        synth.fp8_scales(r, I, n))
    X = r.standard_normal((T, n)).astype(np.float32)
    xd = DeviceBuffer.from_numpy(X)
    frag = ops.act_frag_buffer(n, T)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, n, T, None)
    yd = DeviceBuffer(4 * T * I)
    call("rl_hip_gemm_fp8_prefill", lin.w.ptr, lin.ts.ptr, frag.ptr, yd.ptr, 2 * I, n, T, 5, I, None)
    want = ops.act_frag_buffer(I, T)
    call("rl_hip_pack_act", yd.ptr, want.ptr, I, T, None)
    got = ops.act_frag_buffer(I, T)
    call("rl_hip_gemm_fp8_prefill", lin.w.ptr, lin.ts.ptr, frag.ptr, got.ptr, 2 * I, n, T, 6, I, None)
    nb = (I // 128) * 16 * 2 * T * 16  # fragment units (block, i, g) x (hi, mid) x T x 16 B
    a = got.numpy(np.uint8, (got.nbytes,))[:nb]
    b = want.numpy(np.uint8, (want.nbytes,))[:nb]
    assert np.array_equal(a, b)


def test_gemm_prefill_add_and_swiglu(gpu, orc):
    r = synth.rng(41)
    T, n, I = 70, 768, 256
    # gate/up interleaved per 16-row tile, as the engine packs them
    Wg, Wu = synth.fp8_weight(r, I, n), synth.fp8_weight(r, I, n)
    sg, su = synth.fp8_scales(r, I, n), synth.fp8_scales(r, I, n)
    W = np.empty((2 * I, n), np.uint8)
    S = np.empty((2 * I // 128, (n + 127) // 128), np.float32)
    for b in range(I // 16):
        W[32 * b:32 * b + 16] = Wg[16 * b:16 * b + 16]
        W[32 * b + 16:32 * b + 32] = Wu[16 * b:16 * b + 16]
    X = r.standard_normal((T, n)).astype(np.float32)
    g = orc.gemm_fp8(Wg, sg, X)
    u = orc.gemm_fp8(Wu, su, X)
    want = g / (1.0 + np.exp(-g.astype(np.float64))) * u
    # the interleaved matrix's 128-row scale blocks mix gate and up rows, so pack
    # it with per-row-tile scales by building the tiles from the two halves
    lin_g, lin_u = ops.Fp8Linear(Wg, sg), ops.Fp8Linear(Wu, su)
    from rapidllm_amd.hip import DeviceBuffer, call
    L = __import__("rapidllm_amd.hip", fromlist=["lib"]).lib()
    w = DeviceBuffer(L.rl_hip_fp8_packed_bytes(2 * I, n))
    ts = DeviceBuffer(4 * L.rl_hip_fp8_tile_scales(2 * I, n))
    tile = 2048 * ((n + 127) // 128)
    nt = (n + 127) // 128
    for b in range(I // 16):
        call("rl_hip_memcpy_d2d", w.ptr + (2 * b) * tile, lin_g.w.ptr + b * tile, tile, None)
        call("rl_hip_memcpy_d2d", w.ptr + (2 * b + 1) * tile, lin_u.w.ptr + b * tile, tile, None)
        call("rl_hip_memcpy_d2d", ts.ptr + 4 * (2 * b) * nt, lin_g.ts.ptr + 4 * b * nt, 4 * nt, None)
        call("rl_hip_memcpy_d2d", ts.ptr + 4 * (2 * b + 1) * nt, lin_u.ts.ptr + 4 * b * nt, 4 * nt, None)
    xd = DeviceBuffer.from_numpy(X)
    frag = ops.act_frag_buffer(n, T)
    yd = DeviceBuffer(4 * T * I)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, n, T, None)
    call("rl_hip_gemm_fp8_prefill", w.ptr, ts.ptr, frag.ptr, yd.ptr, 2 * I, n, T, 2, I, None)
    got = yd.numpy(np.float32, (T, I))
    for t in range(T):
        assert rel_l2(got[t], want[t]) <= REL_L2, t
    # add epilogue: Y0 + W . X
    Y0 = r.standard_normal((T, I)).astype(np.float32)
    got = ops.linear_prefill(lin_g, X, epilogue=1, Y0=Y0)
    for t in range(T):
        assert rel_l2(got[t], Y0[t] + g[t]) <= REL_L2, t


def test_gemm_prefill_matches_decode_gemm(gpu):
    """The prefill kernel and the decode kernel compute the same products; results
    agree to fp32 reassociation (different K-split orders)."""
    r = synth.rng(9)
    m, n, T = 512, 2048, 8
    lin = ops.Fp8Linear(synth.fp8_weight(r, m, n), synth.fp8_scales(r, m, n))
    X = r.standard_normal((T, n)).astype(np.float32)
    a = ops.linear_prefill(lin, X)
    b = ops.linear_T(lin, X)
    assert rel_l2(a, b) <= 1e-5


@pytest.mark.parametrize("T,pos,nq,nkv", [(1, 0, 24, 4), (16, 0, 24, 4), (37, 300, 24, 4), (100, 1000, 24, 4),
                                          (70, 250, 4, 2), (33, 17, 2, 2)])
def test_attn_prefill_vs_oracle(gpu, orc, T, pos, nq, nkv):
    """Causal prefill attention: every token over the cache and the earlier prompt
    tokens, against the per-token oracle (fp16 K/V as the device cache holds them)."""
    from tests.test_gpu_layers import _attn_oracle
    r = synth.rng(60 + pos + T + nq)
    hd = 256
    ctx = ((pos + T + 255) // 256) * 256 + 256
    Y = r.standard_normal((T, 2 * nq * hd + 2 * nkv * hd)).astype(np.float32)
    qn = (r.standard_normal(hd) * 0.1).astype(np.float32)
    kn = (r.standard_normal(hd) * 0.1).astype(np.float32)
    K = r.standard_normal((pos, nkv, hd)).astype(np.float16).astype(np.float32)
    V = r.standard_normal((pos, nkv, hd)).astype(np.float16).astype(np.float32)
    cache = ops.AttnCache(nkv, ctx, hd)
    if pos:
        cache.fill(K, V)
    out = ops.attn_prefill_layer(Y, cache, pos, qn, kn, nq, nkv)
    want = _attn_oracle(orc, Y, K, V, pos, qn, kn, nq, nkv)
    for t in range(T):
        assert rel_l2(out[t], want[t]) < 1e-3, (t, rel_l2(out[t], want[t]))


def test_attn_prefill_then_decode(gpu, orc):
    """K/V written by the prefill serve a following decode step: decode at the next
    position after a prefill equals the oracle over the whole sequence."""
    from tests.test_gpu_layers import _attn_oracle
    r = synth.rng(99)
    nq, nkv, hd, pos, T = 24, 4, 256, 200, 40
    ctx = 512
    Y = r.standard_normal((T + 1, 2 * nq * hd + 2 * nkv * hd)).astype(np.float32)
    qn = (r.standard_normal(hd) * 0.1).astype(np.float32)
    kn = (r.standard_normal(hd) * 0.1).astype(np.float32)
    K = r.standard_normal((pos, nkv, hd)).astype(np.float16).astype(np.float32)
    V = r.standard_normal((pos, nkv, hd)).astype(np.float16).astype(np.float32)
    cache = ops.AttnCache(nkv, ctx, hd)
    cache.fill(K, V)
    ops.attn_prefill_layer(Y[:T], cache, pos, qn, kn, nq, nkv)
    got = ops.attn_decode_layer(Y[T:], cache, pos + T, qn, kn, nq, nkv)
    want = _attn_oracle(orc, Y, K, V, pos, qn, kn, nq, nkv)
    assert rel_l2(got[0], want[T]) < 1e-3


@pytest.mark.parametrize("chunk", ["512", "2048"])
def test_engine_chunked_prefill_matches_oracle(gpu, orc, monkeypatch, chunk):
    """A 600-token prompt: two prefill chunks (512 + 84, RL_PREFILL_CHUNK=512) or one
    (the default chunk of 2048) through the chunked path,
    the last max_T tokens as a decode step; logits equal the oracle's, decoding and
    speculative generation continue exactly as from a token-by-token prefill."""
    from oracle.oracle import OracleModel
    from rapidllm_amd import model as M
    from rapidllm_amd.engine import Engine
    from tests.test_gpu_engine import margin_ok, mini_spec
    spec = mini_spec()
    W = M.random_weights(spec, seed=3, w_scale=(1e-3, 1e-2))
    monkeypatch.setenv("RL_PREFILL_CHUNK", chunk)
    eng = Engine(spec, W, ctx=1024)
    orc_m = OracleModel(spec, W, ctx=1024)
    rng = np.random.default_rng(5)
    prompt = [int(t) for t in rng.integers(0, spec.vocab, 600)]
    eng.prefill(prompt)
    orc_m.reset()
    for t in prompt:
        g, lg, hd = orc_m.decode(t)
    assert rel_l2(eng.copy_logits(), lg) < 1e-3
    assert rel_l2(eng.copy_last_hidden(), hd) < 1e-3
    if margin_ok(lg):
        assert eng.greedy() == g
    tok = g
    for _ in range(4):
        eng.decode_token(tok)
        g, lg, _ = orc_m.decode(tok)
        assert rel_l2(eng.copy_logits(), lg) < 1e-3
        tok = g
    want, _, _ = orc_m.generate(prompt, 8)
    got, _, _ = eng.generate(prompt, 8, spec_n=3)
    assert got == want


@pytest.mark.parametrize("T,nk,nv,v_tiled", [(1, 16, 48, False), (37, 16, 48, False), (200, 2, 6, True),
                                             (64, 4, 4, False)])
def test_gdn_prefill_vs_oracle(gpu, orc, T, nk, nv, v_tiled):
    """DeltaNet prefill (conv over all tokens, then the recurrence with the state in
    registers) against per-token oracle steps: outputs, final state, final window."""
    from tests.test_gpu_layers import _gdn_case, _gdn_oracle
    r = synth.rng(400 + T + nv)
    case = _gdn_case(r, T, nk, nv, v_tiled)
    o, S, conv = ops.gdn_prefill(*case, nk, nv, v_tiled)
    o_ref, S_ref, conv_ref = _gdn_oracle(orc, *case, nk, nv, v_tiled)
    for t in range(T):
        assert rel_l2(o[t], o_ref[t]) < 1e-3, (t, rel_l2(o[t], o_ref[t]))
    assert rel_l2(S, S_ref) < 1e-4
    assert np.array_equal(conv, conv_ref)


@pytest.mark.parametrize("T,decay", [(700, 0.5), (130, 6.0), (64, -3.0)])
def test_gdn_prefill_chunked_vs_per_token(gpu, orc, monkeypatch, T, decay):
    """The chunked scan (chunks of 64 tokens in WY form) and the per-token scan
    (RL_PF_GDN_CHUNK=0) against the per-token oracle over several chunks and a
    ragged last one: decay 6 makes A_log large enough that g underflows to 0 in
    fp32 on some tokens (the chunk's log-decay sums must not turn into inf - inf),
    decay -3 keeps g near 1 (little forgetting, the state carries over chunks)."""
    from tests.test_gpu_layers import _gdn_case, _gdn_oracle
    nk, nv = 2, 4
    r = synth.rng(900 + T)
    case = list(_gdn_case(r, T, nk, nv, False))
    case[3] = (case[3] + decay).astype(np.float32)  # A_log
    o_ref, S_ref, conv_ref = _gdn_oracle(orc, *case, nk, nv, False)
    for mode in ("1", "0"):
        monkeypatch.setenv("RL_PF_GDN_CHUNK", mode)
        o, S, conv = ops.gdn_prefill(*case, nk, nv, False)
        assert np.isfinite(o).all() and np.isfinite(S).all()
        for t in range(T):
            assert rel_l2(o[t], o_ref[t]) < 1e-3, (mode, t, rel_l2(o[t], o_ref[t]))
        assert rel_l2(S, S_ref) < 1e-4, mode
        assert np.array_equal(conv, conv_ref)


def test_gdn_prefill_chunked_full_shape(gpu, monkeypatch):
    """At the 27B DeltaNet shape (16 k-heads, 48 v-heads) over a full 2048-token
    prefill chunk, the chunked scan and the per-token scan (each pinned to the
    per-token oracle at smaller sizes above) agree on every output row and on the
    final state."""
    from tests.test_gpu_layers import _gdn_case
    T, nk, nv = 2048, 16, 48
    case = _gdn_case(synth.rng(950), T, nk, nv, False)
    monkeypatch.setenv("RL_PF_GDN_CHUNK", "1")
    o1, S1, c1 = ops.gdn_prefill(*case, nk, nv, False)
    monkeypatch.setenv("RL_PF_GDN_CHUNK", "0")
    o0, S0, c0 = ops.gdn_prefill(*case, nk, nv, False)
    assert np.isfinite(o1).all() and np.isfinite(S1).all()
    err = np.linalg.norm(o1 - o0, axis=1) / np.maximum(np.linalg.norm(o0, axis=1), 1e-30)
    assert err.max() < 1e-4, (int(err.argmax()), float(err.max()))
    assert rel_l2(S1, S0) < 1e-5
    assert np.array_equal(c1, c0)


@pytest.mark.parametrize("qt,m,n,T", [(ops.Q4_K, 256, 1024, 70), (ops.Q6_K, 160, 768, 130),
                                      (ops.Q4_K, 5120, 4096, 300)])
def test_kquant_prefill_gemm_vs_oracle(gpu, orc, qt, m, n, T):
    """The K-quant prefill linear: rl_hip_kquant_to_bf16x2 turns the tiled blocks
    into BF16 hi + lo tiles (hi + lo equal the reference's dequantised weight to 16
    significant bits; checked against ops::dequant_q4_k / dequant_q6_k), and the
    BF16 x2 prefill GEMM over them matches the oracle's K-quant GEMV per token."""
    from rapidllm_amd.hip import DeviceBuffer, call
    r = synth.rng(700 + m + T)
    blocks = synth.q4k_blocks(r, m, n) if qt == ops.Q4_K else synth.q6k_blocks(r, m, n)
    lin = ops.KQuantLinear(qt, blocks, m, n)
    mt = (m + 15) // 16
    hi, lo = DeviceBuffer(mt * 16 * n * 2), DeviceBuffer(mt * 16 * n * 2)
    call("rl_hip_kquant_to_bf16x2", qt, lin.w.ptr, hi.ptr, lo.ptr, m, n, None)
    # the split against the exact dequantisation, element by element (first row tile)
    deq = orc.dequant_q4_k if qt == ops.Q4_K else orc.dequant_q6_k
    Wd = deq(np.ascontiguousarray(blocks.reshape(-1)), m * n).reshape(m, n)
    h = hi.numpy(np.uint16, (mt * 16 * n,))
    l = lo.numpy(np.uint16, (mt * 16 * n,))
    nkb = n // 128
    for row in (0, 5, 15):
        for c in (0, 37, 128, n - 1):
            kb, j = c // 128, c % 128
            g, q, e = j // 32, (j % 32) // 8, j % 8
            i = (0 * nkb + kb) * 2048 + q * 512 + 8 * (row + 16 * g) + e
            w = synth.bf16_to_f32(h[i:i + 1])[0] + synth.bf16_to_f32(l[i:i + 1])[0]
            assert abs(w - Wd[row, c]) <= abs(Wd[row, c]) * 2.0 ** -15, (row, c, w, Wd[row, c])
    X = r.standard_normal((T, n)).astype(np.float32)
    xd = DeviceBuffer.from_numpy(X)
    frag = ops.act_frag_buffer(n, T)
    yd = DeviceBuffer(4 * T * m)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, n, T, None)
    call("rl_hip_gemm_bf16_prefill", hi.ptr, lo.ptr, frag.ptr, yd.ptr, m, n, T, 0, m, None)
    got = yd.numpy(np.float32, (T, m))
    gemv = orc.gemv_q4_k if qt == ops.Q4_K else orc.gemv_q6_k
    for t in range(0, T, max(1, T // 7)):
        want = gemv(np.ascontiguousarray(blocks.reshape(-1)), X[t], m, n, 8)
        assert rel_l2(got[t], want) <= REL_L2, (t, rel_l2(got[t], want))


def _f16_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


@pytest.mark.parametrize("qt,m,n,T,epi", [(ops.Q4_K, 256, 1024, 70, 0), (ops.Q6_K, 160, 768, 130, 1),
                                          (ops.Q4_K, 5120, 4096, 300, 0), (ops.Q6_K, 512, 1280, 64, 5)])
def test_kquant_f16_prefill_gemm_vs_oracle(gpu, orc, qt, m, n, T, epi):
    """The K-quant prefill linears' fp16 form: rl_hip_kquant_to_f16 stores each
    weight of a (16-row tile, 128-column block) as rn16(w / s) with a power-of-two s
    per block (checked against ops::dequant_q4_k / dequant_q6_k to fp16 rounding);
    rl_hip_act_frag_to_f16 turns the bf16 hi + mid fragments into fp16 hi + lo of
    x / xscale without losing a bit; the fp16 prefill GEMM (store, add, and SwiGLU
    over half tiles) matches the oracle's K-quant GEMV per token."""
    from rapidllm_amd.hip import DeviceBuffer, call
    r = synth.rng(800 + m + T)
    blocks = synth.q4k_blocks(r, m, n) if qt == ops.Q4_K else synth.q6k_blocks(r, m, n)
    lin = ops.KQuantLinear(qt, blocks, m, n)
    mt, nkb = (m + 15) // 16, n // 128
    w16 = DeviceBuffer(mt * 16 * n * 2)
    ts = DeviceBuffer(4 * mt * nkb)
    call("rl_hip_kquant_to_f16", qt, lin.w.ptr, w16.ptr, ts.ptr, m, n, None)
    deq = orc.dequant_q4_k if qt == ops.Q4_K else orc.dequant_q6_k
    Wd = deq(np.ascontiguousarray(blocks.reshape(-1)), m * n).reshape(m, n)
    h = _f16_to_f32(w16.numpy(np.uint16, (mt * 16 * n,)))
    sc = ts.numpy(np.float32, (mt, nkb))
    for rt in (0, mt - 1):
        for kb in (0, nkb - 1):
            blk = np.abs(Wd[16 * rt:16 * rt + 16, 128 * kb:128 * kb + 128])
            s = sc[rt, kb]
            mx = blk.max()
            assert s > 0 and (mx == 0 or 2.0 ** 14 <= mx / s < 2.0 ** 15), (rt, kb, s, mx)
            assert s == 2.0 ** np.round(np.log2(s))  # a power of two
    for row in (0, 5, 15, 16 * (mt - 1) + 3):
        for c in (0, 37, 128, n - 1):
            rt, kb, j = row // 16, c // 128, c % 128
            g, q, e = j // 32, (j % 32) // 8, j % 8
            i = (rt * nkb + kb) * 2048 + q * 512 + 8 * (row % 16 + 16 * g) + e
            w = np.float32(h[i]) * sc[rt, kb]
            want = np.float32(Wd[row, c] / sc[rt, kb]).astype(np.float16).astype(np.float32) * sc[rt, kb]
            assert w == want, (row, c, w, Wd[row, c])
    X = (r.standard_normal((T, n)) * np.exp(r.uniform(-6, 6, (T, 1)))).astype(np.float32)
    xd = DeviceBuffer.from_numpy(X)
    frag = ops.act_frag_buffer(n, T)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, n, T, None)
    frag16 = ops.act_frag_buffer(n, T)
    xs = DeviceBuffer(4 * nkb * T)
    call("rl_hip_act_frag_to_f16", frag.ptr, frag16.ptr, xs.ptr, n, T, None)
    # hi + lo (fp16) times the scale equals hi + mid (bf16) exactly, unit by unit
    fb = frag.numpy(np.uint16, (frag.nbytes // 2,)).reshape(nkb * 16, 2 * T, 8)
    f16 = frag16.numpy(np.uint16, (frag16.nbytes // 2,)).reshape(nkb * 16, 2 * T, 8)
    xsv = xs.numpy(np.float32, (nkb, T))
    for t in (0, T - 1):
        bf = synth.bf16_to_f32(fb[:, t]) + synth.bf16_to_f32(fb[:, T + t])
        hl = (_f16_to_f32(f16[:, t]).astype(np.float64) + _f16_to_f32(f16[:, T + t])) * \
            np.repeat(xsv[:, t], 16)[:, None]
        assert np.array_equal(bf.astype(np.float64), hl), t
    mo = m // 2 if epi == 5 else m
    Y0 = r.standard_normal((T, mo)).astype(np.float32)
    yd = DeviceBuffer.from_numpy(Y0)
    call("rl_hip_gemm_f16_prefill", w16.ptr, ts.ptr, frag16.ptr, xs.ptr, yd.ptr, m, n, T, epi, mo, None)
    got = yd.numpy(np.float32, (T, mo))
    gemv = orc.gemv_q4_k if qt == ops.Q4_K else orc.gemv_q6_k
    for t in range(0, T, max(1, T // 7)):
        y = gemv(np.ascontiguousarray(blocks.reshape(-1)), X[t], m, n, 8).astype(np.float64)
        if epi == 5:  # half tiles: rows 16k .. 16k+7 gate, 16k+8 .. 16k+15 up of outputs 8k .. 8k+7
            yt = y.reshape(-1, 2, 8)
            with np.errstate(over="ignore"):
                want = (yt[:, 0] / (1.0 + np.exp(-yt[:, 0])) * yt[:, 1]).reshape(-1)
        else:
            want = y + (Y0[t] if epi == 1 else 0.0)
        assert rel_l2(got[t], want) <= REL_L2, (t, rel_l2(got[t], want))


@pytest.mark.parametrize("quant", ["q4_k", "q6_k", "bf16"])
def test_engine_kquant_chunked_prefill_matches_oracle(gpu, orc, monkeypatch, quant):
    """A GGUF-style model (K-quant layer linears, BF16 a / b rows, Q6_K lm_head), or
    a model with BF16 layer linears, prefills a 300-token prompt through the chunked
    path (two chunks of 256 + the decode-step tail): logits and decoding continue as
    the oracle's."""
    from oracle.oracle import OracleModel
    from rapidllm_amd import model as M
    from rapidllm_amd.engine import Engine
    from tests.test_gpu_engine import margin_ok, mini_spec
    spec = mini_spec()
    lq = {"q4_k": M.Q_Q4_K, "q6_k": M.Q_Q6_K, "bf16": M.Q_BF16}[quant]
    W = M.random_weights(spec, seed=13, linear_quant=lq, head_quant=M.Q_BF16 if quant == "bf16" else M.Q_Q6_K)
    monkeypatch.setenv("RL_PREFILL_CHUNK", "256")
    eng = Engine(spec, W, ctx=1024)
    orc_m = OracleModel(spec, W, ctx=1024)
    rng = np.random.default_rng(15)
    prompt = [int(t) for t in rng.integers(0, spec.vocab, 300)]
    eng.prefill(prompt)
    orc_m.reset()
    for t in prompt:
        g, lg, hd = orc_m.decode(t)
    assert rel_l2(eng.copy_logits(), lg) < 1e-3
    if margin_ok(lg):
        assert eng.greedy() == g
    tok = g
    for _ in range(3):
        eng.decode_token(tok)
        g, lg, _ = orc_m.decode(tok)
        assert rel_l2(eng.copy_logits(), lg) < 1e-3
        tok = g
    eng.close()
