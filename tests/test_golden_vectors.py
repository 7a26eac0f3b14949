"""The oracle against golden vectors committed under tests/golden/ (no reference
sources needed): ref_vectors.npz comes from the reference's own CPU kernels
(tests/golden/make_ref_vectors.py); every comparison is bit-exact, as the
oracle restates those kernels operation for operation."""
import os

import numpy as np
import pytest

from oracle import oracle as O

V = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz"))


def eq(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                          b.view(np.uint32) if b.dtype == np.float32 else b, equal_nan=False)


def test_e4m3_table():
    got = np.array([O.lib().orc_e4m3_to_f32(c) for c in range(256)], np.float32)
    exp = V["e4m3.out"]
    fin = ~np.isnan(exp)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    eq(got[fin], exp[fin])


def test_fp16_decode():
    got = np.array([O.lib().orc_fp16_to_f32(int(c)) for c in V["fp16.in"]], np.float32)
    exp = V["fp16.out"]
    fin = ~np.isnan(exp)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    eq(got[fin], exp[fin])


@pytest.mark.parametrize("tag", ["fp8a", "fp8b"])
def test_gemv_fp8(tag):
    eq(O.gemv_fp8(V[f"{tag}.W"], V[f"{tag}.s"], V[f"{tag}.x"]), V[f"{tag}.y"])


@pytest.mark.parametrize("tag", ["q4k", "q6k"])
def test_kquant(tag):
    blk, x, y = V[f"{tag}.blocks"], V[f"{tag}.x"], V[f"{tag}.y"]
    m, n = y.size, x.size
    deq = O.dequant_q4_k if tag == "q4k" else O.dequant_q6_k
    gemv = O.gemv_q4_k if tag == "q4k" else O.gemv_q6_k
    eq(deq(blk, m * n), V[f"{tag}.deq"])
    eq(gemv(blk, x, m, n), y)


def test_gemv_bf16():
    # The reference's gemv_bf16 dispatches on the host ISA (cpu_caps.cpp:171-198:
    # AVX-512 / AVX2 lanes, else the scalar loop the oracle restates), so its
    # summation order is machine-dependent: equal to within fp32 reassociation.
    W = (V["bf16.W"].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = V["bf16.x"].astype(np.float64)
    bound = 1.2e-7 * W.shape[1] * (np.abs(W) @ np.abs(x))
    assert np.all(np.abs(O.gemv_bf16(V["bf16.W"], V["bf16.x"]) - V["bf16.y"]) <= bound)


def test_norms():
    eq(O.qwen3_rmsnorm(V["rms.x"], V["rms.g"]), V["rms.y"])
    for tag in ("gnorm_head", "gnorm_whole"):
        g = V[f"{tag}.g"]
        eq(O.gated_rmsnorm(V[f"{tag}.x"], V[f"{tag}.z"], g, 1e-6, g.size), V[f"{tag}.y"])
    eq(O.l2norm(V["l2.x"]), V["l2.y"])


def test_conv1d_three_tokens():
    st = V["conv.st0"].copy()
    for t in range(3):
        eq(O.conv1d_update(V["conv.x"][t], V["conv.w"], st), V["conv.y"][t])
    eq(st, V["conv.st"])


def test_delta_step():
    S = V["delta.S0"].copy()
    o = O.delta_step(S, V["delta.q"], V["delta.k"], V["delta.v"], V["delta.beta"], V["delta.gl"])
    eq(o, V["delta.o"])
    eq(S, V["delta.S"])


@pytest.mark.parametrize("pos", [1, 777, 32767])
def test_rope(pos):
    q, k = O.rope_partial(V["rope.q"], V["rope.k"], 4, 2, 256, 64, pos, 1e7)
    eq(q, V[f"rope.q{pos}"])
    eq(k, V[f"rope.k{pos}"])


def test_attn_decode():
    kc = V["attn.kc"]
    eq(O.attn_decode(V["attn.q"], kc, V["attn.vc"], kc.shape[0] - 1, 4, 2, 256), V["attn.o"])


def test_greedy():
    assert O.greedy(V["greedy.x"]) == int(V["greedy.i"][0])


def test_swiglu():
    eq(O.swiglu(V["swiglu.g"], V["swiglu.u"]), V["swiglu.y"])
