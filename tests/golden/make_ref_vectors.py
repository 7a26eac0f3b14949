"""Generate kernel golden vectors from the reference's own CPU kernels.

The reference's src/kernels/cpu ops (compiled from /root/reference by
oracle/Makefile's `ref` target into oracle/_ref/libref.so; exported through
oracle/ref_shim.cpp) are run on seeded inputs, and inputs plus outputs are
written to ref_vectors.npz.  tests/test_golden_vectors.py checks the oracle
against this file, so the oracle stays pinned where /root/reference and
oracle/_ref are absent.  Usage (build container):
    make -C oracle ref && python tests/golden/make_ref_vectors.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from rapidllm_amd import synth  # noqa: E402

P, u8, u16 = O.P, O._u8, O._u16


def main():
    R = O.ref()
    if R is None:
        sys.exit("oracle/_ref/libref.so not built (make -C oracle ref)")
    r = synth.rng(2024)
    v = {}
    # e4m3 and fp16 decode tables (ops.h e4m3_to_f32 / fp16_to_f32)
    v["e4m3.out"] = np.array([R.ref_e4m3_to_f32(c) for c in range(256)], np.float32)
    codes = np.concatenate([np.arange(0, 65536, 97), [0x0000, 0x0001, 0x03ff, 0x0400, 0x7bff, 0x7c00, 0x7e00,
                                                      0x8000, 0x8001, 0xfc00, 0xffff]]).astype(np.uint16)
    v["fp16.in"] = codes
    v["fp16.out"] = np.array([R.ref_fp16_to_f32(int(c)) for c in codes], np.float32)
    # block-FP8 GEMV (128x128 scale blocks), a ragged column count included
    for tag, m, n in (("fp8a", 64, 512), ("fp8b", 40, 320)):
        W = synth.fp8_weight(r, m, n)
        s = synth.fp8_scales(r, m, n)
        x = r.standard_normal(n).astype(np.float32)
        y = np.empty(m, np.float32)
        R.ref_gemv_fp8(P(W, u8), P(s), P(x), P(y), m, n)
        v.update({f"{tag}.W": W, f"{tag}.s": s, f"{tag}.x": x, f"{tag}.y": y})
    # K-quant dequant and GEMV
    for tag, gen, deq, gemv in (("q4k", synth.q4k_blocks, R.ref_dequant_q4_k, R.ref_gemv_q4_k),
                                ("q6k", synth.q6k_blocks, R.ref_dequant_q6_k, R.ref_gemv_q6_k)):
        m, n = 16, 512
        blk = gen(r, m, n)
        d = np.empty(m * n, np.float32)
        deq(P(blk, u8), P(d), m * n)
        x = r.standard_normal(n).astype(np.float32)
        y = np.empty(m, np.float32)
        gemv(P(blk, u8), P(x), P(y), m, n)
        v.update({f"{tag}.blocks": blk, f"{tag}.deq": d, f"{tag}.x": x, f"{tag}.y": y})
    # bf16 GEMV
    Wb = synth.bf16_bits(r.standard_normal((24, 256)).astype(np.float32))
    xb = r.standard_normal(256).astype(np.float32)
    yb = np.empty(24, np.float32)
    R.ref_gemv_bf16(P(Wb, u16), P(xb), P(yb), 24, 256)
    v.update({"bf16.W": Wb, "bf16.x": xb, "bf16.y": yb})
    # norms: (1+w) rmsnorm, gated rmsnorm per head and whole-vector, l2norm
    x = (r.standard_normal(1024) * 3).astype(np.float32)
    g = (r.standard_normal(1024) * 0.1).astype(np.float32)
    y = np.empty_like(x)
    R.ref_qwen3_rmsnorm(P(x), P(g), P(y), 1024, 1e-6)
    v.update({"rms.x": x, "rms.g": g, "rms.y": y})
    for tag, n, gn in (("gnorm_head", 512, 128), ("gnorm_whole", 48, 48)):
        x = r.standard_normal(n).astype(np.float32)
        z = r.standard_normal(n).astype(np.float32)
        g = (1 + 0.1 * r.standard_normal(gn)).astype(np.float32)
        y = np.empty_like(x)
        R.ref_gated_rmsnorm(P(x), P(z), P(g), P(y), n, 1e-6, gn)
        v.update({f"{tag}.x": x, f"{tag}.z": z, f"{tag}.g": g, f"{tag}.y": y})
    x = r.standard_normal(128).astype(np.float32)
    y = np.empty_like(x)
    R.ref_l2norm(P(x), P(y), 128, 1e-6)
    v.update({"l2.x": x, "l2.y": y})
    # causal conv1d update, three consecutive tokens
    dim, k = 256, 4
    w = (r.standard_normal((dim, k)) * 0.5).astype(np.float32)
    st = r.standard_normal((dim, k)).astype(np.float32)
    v.update({"conv.w": w, "conv.st0": st.copy()})
    xs = r.standard_normal((3, dim)).astype(np.float32)
    ys = np.empty((3, dim), np.float32)
    for t in range(3):
        R.ref_conv1d_update(P(xs[t]), P(w), P(st), P(ys[t]), dim, k)
    v.update({"conv.x": xs, "conv.y": ys, "conv.st": st})
    # gated delta-rule recurrent step (scalar path)
    nv, dk, dv = 2, 128, 64
    S = (r.standard_normal((nv, dk, dv)) * 0.02).astype(np.float32)
    q = r.standard_normal((nv, dk)).astype(np.float32)
    kk = r.standard_normal((nv, dk)).astype(np.float32)
    vv = r.standard_normal((nv, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-r.standard_normal(nv)))).astype(np.float32)
    gl = (-np.log1p(np.exp(r.standard_normal(nv)))).astype(np.float32)
    v.update({"delta.S0": S.copy(), "delta.q": q, "delta.k": kk, "delta.v": vv, "delta.beta": beta,
              "delta.gl": gl})
    o = np.empty((nv, dv), np.float32)
    R.ref_delta_step_scalar(P(S), P(q), P(kk), P(vv), P(beta), P(gl), P(o), nv, dk, dv, 1e-6)
    v.update({"delta.S": S, "delta.o": o})
    # partial rope (27B: hd 256, rot 64, theta 1e7) at several positions
    q = r.standard_normal(4 * 256).astype(np.float32)
    kk = r.standard_normal(2 * 256).astype(np.float32)
    v.update({"rope.q": q, "rope.k": kk})
    for pos in (1, 777, 32767):
        q2, k2 = q.copy(), kk.copy()
        R.ref_rope_partial(P(q2), P(k2), 4, 2, 256, 64, pos, 1e7)
        v.update({f"rope.q{pos}": q2, f"rope.k{pos}": k2})
    # GQA attention decode over a short cache
    nq, nkv, hd, L = 4, 2, 256, 37
    q = r.standard_normal(nq * hd).astype(np.float32)
    kc = r.standard_normal((L, nkv * hd)).astype(np.float32)
    vc = r.standard_normal((L, nkv * hd)).astype(np.float32)
    o = np.empty(nq * hd, np.float32)
    R.ref_attn_decode(P(q), P(kc), P(vc), P(o), L - 1, nq, nkv, hd)
    v.update({"attn.q": q, "attn.kc": kc, "attn.vc": vc, "attn.o": o})
    # SwiGLU silu(g) * u (ops.cpp:607-609)
    g = (r.standard_normal(512) * 4).astype(np.float32)
    u = r.standard_normal(512).astype(np.float32)
    y = np.empty_like(g)
    R.ref_swiglu(P(g), P(u), P(y), 512)
    v.update({"swiglu.g": g, "swiglu.u": u, "swiglu.y": y})
    # greedy argmax with ties
    lg = r.integers(-4, 4, 3000).astype(np.float32)
    v.update({"greedy.x": lg, "greedy.i": np.array([R.ref_greedy(P(lg), lg.size)], np.int32)})
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **v)
    print(f"wrote {len(v)} arrays")


if __name__ == "__main__":
    main()
