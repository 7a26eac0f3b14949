"""The single ops behind the kernel-name device seam (Device::launch names
conv1d_update, delta_recurrent, attn_decode; include/rapidllm/backend/device.h:
49-60) against the oracle's ops::conv1d_update / delta_recurrent_step /
attn_decode on the reference CPU layouts.  Bars: the conv window shift exact,
fp32 outputs within 1e-3 relative L2 (the reference's own table,
docs/architecture.md:829-842, allows 2e-3 for attention)."""
import numpy as np
import pytest

from rapidllm_amd import ops, synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("dim,k", [(10240, 4), (37, 3)])
def test_conv1d_update_vs_oracle(gpu, orc, dim, k):
    r = synth.rng(dim + k)
    x = r.standard_normal(dim).astype(np.float32)
    w = (r.standard_normal((dim, k)) * 0.5).astype(np.float32)
    st = r.standard_normal((dim, k)).astype(np.float32)
    y, st_new = ops.conv1d_update(x, w, st)
    st_ref = st.copy()
    y_ref = orc.conv1d_update(x, w, st_ref)
    assert np.array_equal(st_new, st_ref)
    assert rel_l2(y, y_ref) < 1e-6


@pytest.mark.parametrize("nv,dk,dv", [(48, 128, 128), (4, 64, 96), (3, 256, 300)])
def test_delta_recurrent_vs_oracle(gpu, orc, nv, dk, dv):
    r = synth.rng(nv * dk + dv)
    S = (r.standard_normal((nv, dk, dv)) * 0.02).astype(np.float32)
    q = r.standard_normal((nv, dk)).astype(np.float32)
    k = r.standard_normal((nv, dk)).astype(np.float32)
    v = r.standard_normal((nv, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-r.standard_normal(nv)))).astype(np.float32)
    g = (-np.log1p(np.exp(r.standard_normal(nv)))).astype(np.float32)
    S_dev = S.copy()
    for step in range(3):  # three tokens: the state carries over
        o, S_dev = ops.delta_recurrent_step(S_dev, q, k, v, beta, g)
        o_ref = orc.delta_step(S, q, k, v, beta, g)
        assert rel_l2(o, o_ref) < 1e-3, step
        assert rel_l2(S_dev, S) < 1e-4, step
        q, k, v = np.roll(q, 1, 1), np.roll(k, 3, 1), np.roll(v, 2, 1)


@pytest.mark.parametrize("pos,nq,nkv,hd", [(0, 24, 4, 256), (2, 24, 4, 256), (1000, 24, 4, 256), (77, 8, 8, 128)])
def test_attn_decode_f32_vs_oracle(gpu, orc, pos, nq, nkv, hd):
    r = synth.rng(pos + nq + hd)
    q = r.standard_normal(nq * hd).astype(np.float32)
    kc = r.standard_normal((pos + 1, nkv * hd)).astype(np.float32)
    vc = r.standard_normal((pos + 1, nkv * hd)).astype(np.float32)
    o = ops.attn_decode(q, kc, vc, pos, nq, nkv, hd)
    assert rel_l2(o, orc.attn_decode(q, kc, vc, pos, nq, nkv, hd)) < 1e-3
