"""GPU parity for the DeltaNet decode, gated attention decode, norms and greedy
sampling kernels against the CPU oracle (1e-3 relative L2 on fp32 outputs;
exact for integer results)."""
import numpy as np
import pytest

from rapidllm_amd import ops, synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def test_rmsnorm(gpu, orc):
    r = synth.rng(1)
    x = r.standard_normal((3, 5120)).astype(np.float32) * 7
    g = r.standard_normal(5120).astype(np.float32) * 0.1
    y = ops.qwen3_rmsnorm(x, g)
    for t in range(3):
        assert rel_l2(y[t], orc.qwen3_rmsnorm(x[t], g)) < 1e-6


@pytest.mark.parametrize("n,gn", [(6144, 128), (48, 8), (256, 256)])
def test_gated_rmsnorm(gpu, orc, n, gn):
    r = synth.rng(2 + n)
    o = r.standard_normal((2, n)).astype(np.float32)
    z = r.standard_normal((2, n)).astype(np.float32)
    g = r.standard_normal(gn).astype(np.float32)
    y = ops.gated_rmsnorm(o, z, g, 1e-6, gn)
    for t in range(2):
        assert rel_l2(y[t], orc.gated_rmsnorm(o[t], z[t], g, 1e-6, gn)) < 1e-5


def _gdn_case(r, T, nk, nv, v_tiled):
    dk = dv = 128
    conv_dim = 2 * nk * dk + nv * dv
    qkv = r.standard_normal((T, conv_dim)).astype(np.float32)
    a = r.standard_normal((T, nv)).astype(np.float32)
    b = r.standard_normal((T, nv)).astype(np.float32)
    A_log = (r.standard_normal(nv) * 0.5).astype(np.float32)
    dt = (r.standard_normal(nv) * 0.5).astype(np.float32)
    conv_w = (r.standard_normal((conv_dim, 4)) * 0.5).astype(np.float32)
    conv = r.standard_normal((conv_dim, 4)).astype(np.float32)
    S = (r.standard_normal((nv, dk, dv)) * 0.02).astype(np.float32)
    return qkv, a, b, A_log, dt, conv_w, conv, S


def _gdn_oracle(orc, qkv, a, b, A_log, dt, conv_w, conv, S, nk, nv, v_tiled):
    T = qkv.shape[0]
    dk = S.shape[1]
    qd = nk * dk
    S = S.copy()
    conv = conv.copy()
    outs = []
    rep = nv // nk
    for t in range(T):
        mix = orc.conv1d_update(qkv[t], conv_w, conv)
        src = [(h % nk) if v_tiled else (h // rep) for h in range(nv)]
        q = np.stack([mix[s * dk:(s + 1) * dk] for s in src])
        k = np.stack([mix[qd + s * dk: qd + (s + 1) * dk] for s in src])
        v = mix[2 * qd:].reshape(nv, -1)
        beta, gl = orc.gdn_gates(a[t], b[t], A_log, dt)
        outs.append(orc.delta_step(S, q, k, v, beta, gl).reshape(-1))
    return np.stack(outs), S, conv


@pytest.mark.parametrize("T,nk,nv,v_tiled", [(1, 16, 48, False), (4, 16, 48, False), (3, 2, 6, True), (8, 4, 4, False)])
def test_gdn_decode_vs_oracle(gpu, orc, T, nk, nv, v_tiled):
    r = synth.rng(10 + T + nv)
    case = _gdn_case(r, T, nk, nv, v_tiled)
    o, S, conv = ops.gdn_decode(*case, nk, nv, v_tiled)
    o_ref, S_ref, conv_ref = _gdn_oracle(orc, *case, nk, nv, v_tiled)
    for t in range(T):
        assert rel_l2(o[t], o_ref[t]) < 1e-3, (t, rel_l2(o[t], o_ref[t]))
    assert rel_l2(S, S_ref) < 1e-4
    assert np.array_equal(conv, conv_ref)  # window shift is pure data movement


def _attn_oracle(orc, Y, K, V, pos, qn, kn, nq, nkv, hd=256, rot=64, theta=1e7):
    T = Y.shape[0]
    K = list(K)
    V = list(V)
    outs = []
    for t in range(T):
        row = Y[t]
        qg = row[:2 * nq * hd].reshape(nq, 2, hd)
        q = qg[:, 0, :].reshape(-1)
        gate = qg[:, 1, :].reshape(-1)
        k = row[2 * nq * hd: 2 * nq * hd + nkv * hd]
        v = row[2 * nq * hd + nkv * hd:]
        q = np.concatenate([orc.qwen3_rmsnorm(q[h * hd:(h + 1) * hd], qn) for h in range(nq)])
        k = np.concatenate([orc.qwen3_rmsnorm(k[h * hd:(h + 1) * hd], kn) for h in range(nkv)])
        q, k = orc.rope_partial(q, k, nq, nkv, hd, rot, pos + t, theta)
        K.append(k.reshape(nkv, hd).astype(np.float16).astype(np.float32))
        V.append(v.reshape(nkv, hd).astype(np.float16).astype(np.float32))
        kc = np.ascontiguousarray(np.stack(K).reshape(len(K), -1))
        vc = np.ascontiguousarray(np.stack(V).reshape(len(V), -1))
        o = orc.attn_decode(q, kc, vc, pos + t, nq, nkv, hd)
        outs.append(o / (1 + np.exp(-gate.astype(np.float64))))
    return np.stack(outs)


@pytest.mark.parametrize("T,pos,nq,nkv", [(1, 0, 24, 4), (1, 700, 24, 4), (4, 300, 24, 4), (4, 255, 6, 1),
                                          (2, 1000, 12, 2), (3, 511, 24, 4)])
def test_attn_decode_vs_oracle(gpu, orc, T, pos, nq, nkv):
    r = synth.rng(20 + pos + T)
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
    out = ops.attn_decode_layer(Y, cache, pos, qn, kn, nq, nkv)
    want = _attn_oracle(orc, Y, K, V, pos, qn, kn, nq, nkv)
    for t in range(T):
        assert rel_l2(out[t], want[t]) < 1e-3, (t, rel_l2(out[t], want[t]))


def test_argmax_rows_ties_and_chunks(gpu):
    r = synth.rng(3)
    V = 248320
    L = r.standard_normal((4, V)).astype(np.float32)
    L[1, 100000] = 50.0
    L[1, 200000] = 50.0  # tie: lowest index wins
    L[2, :] = 1.0        # all equal
    L[3, V - 1] = 99.0   # last element
    idx, val = ops.argmax_rows(L)
    assert idx.tolist() == [int(np.argmax(L[0])), 100000, 0, V - 1]
    assert np.array_equal(val, L[np.arange(4), idx])


def test_accept_prefix(gpu):
    assert ops.accept_prefix([7, 1, 2, 3], [1, 2, 3, 9], 10) == (4, 14, 9)
    assert ops.accept_prefix([7, 1, 2, 3], [1, 5, 3, 9], 10) == (2, 12, 5)
    assert ops.accept_prefix([7, 1, 2, 3], [4, 2, 3, 9], 0) == (1, 1, 4)
    assert ops.accept_prefix([7], [4], 5) == (1, 6, 4)
