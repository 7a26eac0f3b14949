"""TEST INFRASTRUCTURE ONLY -- ctypes bindings to the CPU oracle (oracle.cpp) and,
where it was built, to the reference's own CPU kernels (oracle/_ref/libref.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module.  The product package (rapidllm_amd) never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_u16 = C.POINTER(C.c_uint16)
_i32 = C.POINTER(C.c_int)


def build(ref: bool | None = None) -> None:
    """make the oracle; also the reference objects when /root/reference exists."""
    subprocess.check_call(["make", "-s", "-C", HERE, "all"])
    if ref is None:
        ref = os.path.isdir("/root/reference/src/kernels")
    if ref:
        subprocess.check_call(["make", "-s", "-C", HERE, "ref"])


def P(a: np.ndarray, t=_f):
    return a.ctypes.data_as(t)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = C.CDLL(LIB_PATH)
        L.orc_fp16_to_f32.restype = C.c_float
        L.orc_fp16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_fp16.restype = C.c_uint16
        L.orc_f32_to_fp16.argtypes = [C.c_float]
        L.orc_e4m3_to_f32.restype = C.c_float
        L.orc_e4m3_to_f32.argtypes = [C.c_uint8]
        L.orc_gemv_fp8.argtypes = [_u8, _f, _f, _f, C.c_int, C.c_int, C.c_int]
        L.orc_gemm_fp8.argtypes = [_u8, _f, _f, _f, C.c_int, C.c_int, C.c_int]
        L.orc_dequant_q4_k.argtypes = [_u8, _f, C.c_int]
        L.orc_dequant_q6_k.argtypes = [_u8, _f, C.c_int]
        L.orc_gemv_q4_k.argtypes = [_u8, _f, _f, C.c_int, C.c_int, C.c_int]
        L.orc_gemv_q6_k.argtypes = [_u8, _f, _f, C.c_int, C.c_int, C.c_int]
        L.orc_gemv_bf16.argtypes = [_u16, _f, _f, C.c_int, C.c_int, C.c_int]
        L.orc_gemv_f16.argtypes = [_u16, _f, _f, C.c_int, C.c_int]
        L.orc_gemv_f32.argtypes = [_f, _f, _f, C.c_int, C.c_int]
        L.orc_qwen3_rmsnorm.argtypes = [_f, _f, _f, C.c_int, C.c_float]
        L.orc_gated_rmsnorm.argtypes = [_f, _f, _f, _f, C.c_int, C.c_float, C.c_int]
        L.orc_l2norm.argtypes = [_f, _f, C.c_int, C.c_float]
        L.orc_conv1d_update.argtypes = [_f, _f, _f, _f, C.c_int, C.c_int]
        L.orc_gdn_gates.argtypes = [_f, _f, _f, _f, _f, _f, C.c_int]
        L.orc_delta_step.argtypes = [_f, _f, _f, _f, _f, _f, _f, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orc_rope_partial.argtypes = [_f, _f, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orc_attn_decode.argtypes = [_f, _f, _f, _f, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_swiglu.argtypes = [_f, _f, _f, C.c_int]
        L.orc_greedy.restype = C.c_int
        L.orc_greedy.argtypes = [_f, C.c_int]
        L.orc_argmax_rows.argtypes = [_f, C.c_int, C.c_int, _i32]
        L.orc_accept_prefix.restype = C.c_int
        L.orc_accept_prefix.argtypes = [_i32, _i32, C.c_int]
        L.orc_model_create.restype = C.c_void_p
        L.orc_model_create.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_model_reset.argtypes = [C.c_void_p]
        L.orc_model_pos.restype = C.c_int
        L.orc_model_pos.argtypes = [C.c_void_p]
        L.orc_model_decode.restype = C.c_int
        L.orc_model_decode.argtypes = [C.c_void_p, C.c_int, _f, _f]
        L.orc_model_mtp_draft.restype = C.c_int
        L.orc_model_mtp_draft.argtypes = [C.c_void_p, C.c_int, C.c_int, _i32]
        L.orc_model_set_mtp_mode.argtypes = [C.c_void_p, C.c_int]
        L.orc_model_mtp_hidden.restype = C.c_int
        L.orc_model_mtp_hidden.argtypes = [C.c_void_p, _f]
        L.orc_model_generate.restype = C.c_int
        L.orc_model_generate.argtypes = [C.c_void_p, _i32, C.c_int, C.c_int, C.c_int, _i32, _i32, _i32]
        L.orc_model_layer.restype = C.c_int
        L.orc_model_layer.argtypes = [C.c_void_p, C.c_int, _f, C.c_int]
        for nm in ("orc_model_state", "orc_model_conv", "orc_model_kcache", "orc_model_vcache"):
            getattr(L, nm).restype = _f
            getattr(L, nm).argtypes = [C.c_void_p, C.c_int]
        L.orc_model_set_pos.argtypes = [C.c_void_p, C.c_int]
        _lib = L
    return _lib


def ref():
    """The reference's compiled CPU kernels, or None where they were not built."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            return None
        R = C.CDLL(REF_PATH)
        R.ref_e4m3_to_f32.restype = C.c_float
        R.ref_e4m3_to_f32.argtypes = [C.c_uint8]
        R.ref_fp16_to_f32.restype = C.c_float
        R.ref_fp16_to_f32.argtypes = [C.c_uint16]
        R.ref_gemv_fp8.argtypes = [_u8, _f, _f, _f, C.c_int, C.c_int]
        R.ref_dequant_q4_k.argtypes = [_u8, _f, C.c_int]
        R.ref_dequant_q6_k.argtypes = [_u8, _f, C.c_int]
        R.ref_gemv_q4_k.argtypes = [_u8, _f, _f, C.c_int, C.c_int]
        R.ref_gemv_q6_k.argtypes = [_u8, _f, _f, C.c_int, C.c_int]
        R.ref_gemv_bf16.argtypes = [_u16, _f, _f, C.c_int, C.c_int]
        R.ref_qwen3_rmsnorm.argtypes = [_f, _f, _f, C.c_int, C.c_float]
        R.ref_gated_rmsnorm.argtypes = [_f, _f, _f, _f, C.c_int, C.c_float, C.c_int]
        R.ref_l2norm.argtypes = [_f, _f, C.c_int, C.c_float]
        R.ref_conv1d_update.argtypes = [_f, _f, _f, _f, C.c_int, C.c_int]
        R.ref_delta_step_scalar.argtypes = [_f, _f, _f, _f, _f, _f, _f, C.c_int, C.c_int, C.c_int, C.c_float]
        R.ref_delta_step_simd.argtypes = [_f, _f, _f, _f, _f, _f, _f, C.c_int, C.c_int, C.c_int, C.c_float]
        R.ref_rope_partial.argtypes = [_f, _f, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        R.ref_attn_decode.argtypes = [_f, _f, _f, _f, C.c_int, C.c_int, C.c_int, C.c_int]
        R.ref_swiglu.argtypes = [_f, _f, _f, C.c_int]
        R.ref_greedy.restype = C.c_int
        R.ref_greedy.argtypes = [_f, C.c_int]
        R.ref_num_threads.restype = C.c_int
        R.ref_simd_name.restype = C.c_char_p
        R.ref_fused_mlp.argtypes = [_f, _u8, _f, _u8, _f, _u8, _f, _f, C.c_int, C.c_int, C.c_float]
        R.ref_fused_delta.argtypes = [_f, _u8, _f, _u8, _f, _u8, _f, _u8, _f, _u8, _f, _f, _f, _f, _f, _f, _f, _f,
                                      C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        R.ref_fused_attn.argtypes = [_f, _u8, _f, _u8, _f, _u8, _f, _u8, _f, _f, _f, _f, _f, _f, C.c_int, C.c_int,
                                     C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float]
        vp = C.c_void_p
        R.ref_weights_open.restype = vp
        R.ref_weights_open.argtypes = [C.c_char_p, C.c_char_p, C.c_int]
        R.ref_weights_close.argtypes = [vp]
        R.ref_weights_count.argtypes = [vp]
        for fn in ("ref_weights_name", "ref_weights_src"):
            getattr(R, fn).restype = C.c_char_p
            getattr(R, fn).argtypes = [vp, C.c_int]
        R.ref_weights_quant.argtypes = [vp, C.c_int]
        R.ref_weights_shape.argtypes = [vp, C.c_int, C.POINTER(C.c_int64)]
        R.ref_weights_nbytes.restype = C.c_uint64
        R.ref_weights_nbytes.argtypes = [vp, C.c_int]
        R.ref_weights_data.restype = vp
        R.ref_weights_data.argtypes = [vp, C.c_int]
        R.ref_weights_nscale.argtypes = [vp, C.c_int]
        R.ref_weights_scale.restype = vp
        R.ref_weights_scale.argtypes = [vp, C.c_int]
        R.ref_weights_model.argtypes = [vp, C.POINTER(C.c_int), C.POINTER(C.c_ubyte)]
        R.ref_map_name.argtypes = [C.c_int, C.c_char_p, C.c_char_p, C.c_int]
        _ref = R
    return _ref


# ----------------------------------------------------------------- numpy wrappers


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def gemv_fp8(W, scale, x):
    m, n = W.shape
    y = np.empty(m, np.float32)
    lib().orc_gemv_fp8(P(W, _u8), P(f32(scale)), P(f32(x)), P(y), m, n, 128)
    return y


def gemm_fp8(W, scale, X):
    m, n = W.shape
    X = f32(X).reshape(-1, n)
    Y = np.empty((X.shape[0], m), np.float32)
    lib().orc_gemm_fp8(P(W, _u8), P(f32(scale)), P(X), P(Y), m, n, X.shape[0])
    return Y


def dequant_q4_k(packed, n):
    out = np.empty(n, np.float32)
    lib().orc_dequant_q4_k(P(packed, _u8), P(out), n)
    return out


def dequant_q6_k(packed, n):
    out = np.empty(n, np.float32)
    lib().orc_dequant_q6_k(P(packed, _u8), P(out), n)
    return out


def gemv_q4_k(packed, x, m, n, threads=1):
    y = np.empty(m, np.float32)
    lib().orc_gemv_q4_k(P(packed, _u8), P(f32(x)), P(y), m, n, threads)
    return y


def gemv_q6_k(packed, x, m, n, threads=1):
    y = np.empty(m, np.float32)
    lib().orc_gemv_q6_k(P(packed, _u8), P(f32(x)), P(y), m, n, threads)
    return y


def gemv_bf16(W, x, threads=1):
    m, n = W.shape
    y = np.empty(m, np.float32)
    lib().orc_gemv_bf16(P(W, _u16), P(f32(x)), P(y), m, n, threads)
    return y


def gemv_f16(W, x):
    m, n = W.shape
    y = np.empty(m, np.float32)
    lib().orc_gemv_f16(P(W, _u16), P(f32(x)), P(y), m, n)
    return y


def gemv_f32(W, x):
    m, n = W.shape
    y = np.empty(m, np.float32)
    lib().orc_gemv_f32(P(f32(W)), P(f32(x)), P(y), m, n)
    return y


def swiglu(g, u):
    g = f32(g)
    y = np.empty_like(g)
    lib().orc_swiglu(P(g), P(f32(u)), P(y), g.size)
    return y


def argmax_rows(logits):
    logits = f32(logits)
    rows, V = logits.shape
    out = np.empty(rows, np.int32)
    lib().orc_argmax_rows(P(logits), rows, V, out.ctypes.data_as(_i32))
    return out


def qwen3_rmsnorm(x, gamma, eps=1e-6):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_qwen3_rmsnorm(P(x), P(f32(gamma)) if gamma is not None else None, P(y), x.size, eps)
    return y


def gated_rmsnorm(x, z, gamma, eps=1e-6, gamma_n=0):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_gated_rmsnorm(P(x), P(f32(z)), P(f32(gamma)), P(y), x.size, eps, gamma_n)
    return y


def l2norm(x, eps=1e-6):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_l2norm(P(x), P(y), x.size, eps)
    return y


def conv1d_update(x_t, w, state):
    """Returns y; updates `state` ([dim][k] float32, C-contiguous) in place."""
    dim, k = state.shape
    y = np.empty(dim, np.float32)
    lib().orc_conv1d_update(P(f32(x_t)), P(f32(w)), P(state), P(y), dim, k)
    return y


def gdn_gates(a, b, A_log, dt_bias):
    nv = a.size
    beta = np.empty(nv, np.float32)
    gl = np.empty(nv, np.float32)
    lib().orc_gdn_gates(P(f32(a)), P(f32(b)), P(f32(A_log)), P(f32(dt_bias)), P(beta), P(gl), nv)
    return beta, gl


def delta_step(S, q, k, v, beta, g_log, eps=1e-6):
    """S: [nv][dk][dv] float32 updated in place; q,k: [nv][dk]; v: [nv][dv]."""
    nv, dk, dv = S.shape
    o = np.empty((nv, dv), np.float32)
    lib().orc_delta_step(P(S), P(f32(q)), P(f32(k)), P(f32(v)), P(f32(beta)), P(f32(g_log)), P(o), nv, dk, dv, eps)
    return o


def rope_partial(q, k, n_q, n_kv, hd, rot, pos, theta):
    q = f32(q).copy()
    k = f32(k).copy()
    lib().orc_rope_partial(P(q), P(k), n_q, n_kv, hd, rot, pos, theta)
    return q, k


def attn_decode(q, kc, vc, pos, n_q, n_kv, hd):
    o = np.empty(n_q * hd, np.float32)
    lib().orc_attn_decode(P(f32(q)), P(f32(kc)), P(f32(vc)), P(o), pos, n_q, n_kv, hd)
    return o


def greedy(logits):
    logits = f32(logits)
    return lib().orc_greedy(P(logits), logits.size)


def f16_round(a):
    """Round float32 -> fp16 -> float32 with the oracle's RNE conversion."""
    a = f32(a)
    L = lib()
    return np.array([L.orc_fp16_to_f32(L.orc_f32_to_fp16(float(v))) for v in a.ravel()], np.float32).reshape(a.shape)


class OracleModel:
    """CPU decode model (oracle.cpp Model): Session's fused one-token path with
    DualCache layouts.  kv_fp16 rounds cached K/V to fp16 like the device cache."""

    def __init__(self, spec, weights, ctx=4096, kv_fp16=True, threads=8):
        self.spec = spec
        self._cfg = spec.c_config()
        arr, n = weights.c_array()
        self._weights = weights
        self.h = lib().orc_model_create(C.byref(self._cfg), arr, n, ctx, 1 if kv_fp16 else 0, threads)
        if not self.h:
            raise RuntimeError("orc_model_create failed")

    def __del__(self):
        try:
            if self.h:
                lib().orc_model_free(self.h)
        except Exception:
            pass

    def reset(self):
        lib().orc_model_reset(self.h)

    def decode(self, token):
        """One token; returns (greedy, logits, hidden)."""
        lg = np.empty(self.spec.vocab, np.float32)
        hd = np.empty(self.spec.hidden, np.float32)
        g = lib().orc_model_decode(self.h, int(token), P(lg), P(hd))
        if g < 0:
            raise RuntimeError("oracle decode failed")
        return g, lg, hd

    def mtp_draft(self, first, n):
        out = np.zeros(n, np.int32)
        k = lib().orc_model_mtp_draft(self.h, int(first), n, out.ctypes.data_as(_i32))
        if k < 0:
            raise RuntimeError("oracle mtp_draft failed")
        return out[:k]

    def set_mtp_mode(self, mode):
        """0: stem (Session::mtp_draft); 1: stem + the MTP decoder layer
        (Session::mtp_layer_step)."""
        lib().orc_model_set_mtp_mode(self.h, int(mode))

    def mtp_hidden(self):
        """The last draft's hidden before the final MTP norm."""
        h = np.empty(self.spec.hidden, np.float32)
        if lib().orc_model_mtp_hidden(self.h, P(h)) != 0:
            raise RuntimeError("no MTP draft yet")
        return h

    def generate(self, prompt, max_new, spec_n=0):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max_new, np.int32)
        prop, acc = C.c_int(), C.c_int()
        k = lib().orc_model_generate(self.h, prompt.ctypes.data_as(_i32), prompt.size, max_new, spec_n,
                                     out.ctypes.data_as(_i32), C.byref(prop), C.byref(acc))
        if k < 0:
            raise RuntimeError("oracle generate failed")
        return out[:k].tolist(), prop.value, acc.value
