"""Host-side mirror of the reference's kernel surface (rapidllm::ops, include/
rapidllm/kernels/ops.h:112-231) on the gfx950 C ABI.

Functions keep the reference's names and argument meaning; host numpy arrays go in
and come out (device round trip), which is what parity tests need.  Device-resident
objects (Fp8Linear, Bf16Linear, ...) are for callers that keep data in HBM.
Every call goes to the HIP library; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip
from .hip import DeviceBuffer, call


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


class Fp8Linear:
    """Block-FP8 weight [m][n] (e4m3fn + fp32 128x128 scales) resident in HBM in the
    MFMA-tiled layout.  Mirrors QuantKind::FP8_E4M3_B128 weights consumed by
    ops::linear (reference src/kernels/ops.cpp:415-418)."""

    def __init__(self, w: np.ndarray, scale: np.ndarray, stream=None):
        m, n = w.shape
        assert scale.shape == ((m + 127) // 128, (n + 127) // 128)
        self.m, self.n = m, n
        L = hip.lib()
        self.w = DeviceBuffer(L.rl_hip_fp8_packed_bytes(m, n))
        self.ts = DeviceBuffer(4 * L.rl_hip_fp8_tile_scales(m, n))
        raw = DeviceBuffer.from_numpy(np.ascontiguousarray(w, np.uint8), stream)
        sc = DeviceBuffer.from_numpy(_f32(scale), stream)
        call("rl_hip_pack_fp8", raw.ptr, sc.ptr, self.w.ptr, self.ts.ptr, m, n, stream)
        call("rl_hip_stream_synchronize", stream)
        raw.free()
        sc.free()

    @property
    def weight_bytes(self) -> int:
        return self.m * self.n + 4 * ((self.m + 127) // 128) * ((self.n + 127) // 128)

    def forward_frag(self, frag_ptr, y_ptr, T, accumulate=False, stream=None):
        call("rl_hip_gemm_fp8_frag", self.w.ptr, self.ts.ptr, frag_ptr, y_ptr, self.m, self.n, T,
             1 if accumulate else 0, stream)


class Fp8GateUp:
    """MLP gate and up ([I][n] block-FP8 each) packed together for the SwiGLU
    epilogue in half tiles (tile k: gate rows 8k..8k+7, then up rows 8k..8k+7, each
    half with its own 128x128 block scale), as the engine keeps them.  m = 2*I."""

    def __init__(self, wg, sg, wu, su, stream=None):
        I, n = wg.shape
        assert wu.shape == (I, n) and I % 8 == 0
        self.m, self.n, self.I = 2 * I, n, I
        L = hip.lib()
        self.w = DeviceBuffer(L.rl_hip_fp8_packed_bytes(2 * I, n))
        self.ts = DeviceBuffer(4 * L.rl_hip_fp8_gate_up_tile_scales(I, n))
        bufs = [DeviceBuffer.from_numpy(np.ascontiguousarray(wg, np.uint8), stream),
                DeviceBuffer.from_numpy(_f32(sg), stream),
                DeviceBuffer.from_numpy(np.ascontiguousarray(wu, np.uint8), stream),
                DeviceBuffer.from_numpy(_f32(su), stream)]
        call("rl_hip_pack_fp8_gate_up", *[b.ptr for b in bufs], self.w.ptr, self.ts.ptr, I, n, stream)
        call("rl_hip_stream_synchronize", stream)
        for b in bufs:
            b.free()


class Bf16Linear:
    """BF16 weight [m][n] (QuantKind::BF16, e.g. lm_head) in the MFMA-tiled layout."""

    def __init__(self, w_bits: np.ndarray, stream=None):
        m, n = w_bits.shape
        self.m, self.n = m, n
        L = hip.lib()
        self.w = DeviceBuffer(L.rl_hip_bf16_packed_bytes(m, n))
        raw = DeviceBuffer.from_numpy(np.ascontiguousarray(w_bits, np.uint16), stream)
        call("rl_hip_pack_bf16", raw.ptr, self.w.ptr, m, n, stream)
        call("rl_hip_stream_synchronize", stream)
        raw.free()

    def forward_frag(self, frag_ptr, y_ptr, T, accumulate=False, stream=None):
        call("rl_hip_gemm_bf16_frag", self.w.ptr, frag_ptr, y_ptr, self.m, self.n, T, 1 if accumulate else 0,
             stream)


def act_frag_buffer(n: int, T: int) -> DeviceBuffer:
    return DeviceBuffer(hip.lib().rl_hip_act_frag_bytes(n, T))


def linear_T(lin, X: np.ndarray, stream=None) -> np.ndarray:
    """Y[T][m] = W . X[T][n] for a device-resident Fp8Linear / Bf16Linear."""
    X = _f32(X).reshape(-1, lin.n)
    T = X.shape[0]
    xd = DeviceBuffer.from_numpy(X, stream)
    frag = act_frag_buffer(lin.n, T)
    yd = DeviceBuffer(4 * T * lin.m)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, lin.n, T, stream)
    lin.forward_frag(frag.ptr, yd.ptr, T, stream=stream)
    return yd.numpy(np.float32, (T, lin.m), stream)


def linear_prefill(lin: Fp8Linear, X: np.ndarray, epilogue: int = 0, Y0: np.ndarray | None = None,
                   stream=None) -> np.ndarray:
    """Prefill linear over T (any) tokens: Y[T][m'] = W . X (epilogue 0 store, 1 add
    onto Y0, 2 SwiGLU over interleaved gate/up tiles, 5 SwiGLU over the Fp8GateUp
    half tiles: m' = m/2)."""
    X = _f32(X).reshape(-1, lin.n)
    T = X.shape[0]
    mo = lin.m // 2 if epilogue in (2, 5) else lin.m
    xd = DeviceBuffer.from_numpy(X, stream)
    frag = act_frag_buffer(lin.n, T)
    yd = DeviceBuffer.from_numpy(_f32(Y0).reshape(T, mo), stream) if Y0 is not None else DeviceBuffer(4 * T * mo)
    call("rl_hip_pack_act", xd.ptr, frag.ptr, lin.n, T, stream)
    call("rl_hip_gemm_fp8_prefill", lin.w.ptr, lin.ts.ptr, frag.ptr, yd.ptr, lin.m, lin.n, T, epilogue, mo, stream)
    return yd.numpy(np.float32, (T, mo), stream)


def gemv_fp8(W: np.ndarray, scale: np.ndarray, x: np.ndarray, block: int = 128) -> np.ndarray:
    """ops::gemv_fp8(W, scale, x, y, m, n, block) (reference src/kernels/ops.cpp:182)."""
    if block != 128:
        raise ValueError("only 128x128 block scales are supported (FP8_E4M3_B128)")
    return linear_T(Fp8Linear(W, scale), x)[0]


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """ops::e4m3_to_f32 over an array (reference src/kernels/ops.cpp:57)."""
    codes = np.ascontiguousarray(codes, np.uint8)
    d_in = DeviceBuffer.from_numpy(codes)
    d_out = DeviceBuffer(4 * codes.size)
    call("rl_hip_e4m3_to_f32", d_in.ptr, d_out.ptr, codes.size, None)
    return d_out.numpy(np.float32, codes.shape)


Q4_K, Q6_K = 6, 8  # RlQuant / rapidllm::QuantKind values


class KQuantLinear:
    """GGUF Q4_K / Q6_K weight [m][n] resident in HBM in the K-tiled layout
    (QuantKind::Q4_K / Q6_K consumed by ops::linear, reference ops.cpp:422-429)."""

    def __init__(self, qtype: int, blocks: np.ndarray, m: int, n: int, stream=None):
        assert qtype in (Q4_K, Q6_K) and n % 256 == 0
        bb = 144 if qtype == Q4_K else 210
        blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
        assert blocks.size == m * (n // 256) * bb
        self.qtype, self.m, self.n = qtype, m, n
        L = hip.lib()
        self.w = DeviceBuffer(L.rl_hip_kquant_tiled_bytes(qtype, m, n))
        raw = DeviceBuffer.from_numpy(blocks, stream)
        call("rl_hip_pack_kquant", qtype, raw.ptr, self.w.ptr, m, n, stream)
        call("rl_hip_stream_synchronize", stream)
        raw.free()
        self.weight_bytes = blocks.size

    def forward(self, x_ptr, y_ptr, T, ws, accumulate=False, stream=None):
        call("rl_hip_gemm_kquant", self.qtype, self.w.ptr, x_ptr, y_ptr, ws.ptr, ws.nbytes, self.m, self.n, T,
             1 if accumulate else 0, stream)


class KQuantGateUp:
    """The MLP's gate and up K-quant weights [I][n] (one type) as one launch that
    writes h = silu(gate . x) * (up . x) (reference MLP block: two ops::linear calls
    and ops::swiglu, ops.cpp:607-609)."""

    def __init__(self, qtype: int, gate_blocks: np.ndarray, up_blocks: np.ndarray, I: int, n: int, stream=None):
        assert qtype in (Q4_K, Q6_K) and n % 256 == 0 and I % 8 == 0
        bb = 144 if qtype == Q4_K else 210
        g = np.ascontiguousarray(gate_blocks, np.uint8).reshape(-1)
        u = np.ascontiguousarray(up_blocks, np.uint8).reshape(-1)
        assert g.size == u.size == I * (n // 256) * bb
        self.qtype, self.I, self.n = qtype, I, n
        self.w = DeviceBuffer(hip.lib().rl_hip_kquant_tiled_bytes(qtype, 2 * I, n))
        gd = DeviceBuffer.from_numpy(g, stream)
        ud = DeviceBuffer.from_numpy(u, stream)
        call("rl_hip_pack_kquant_gate_up", qtype, gd.ptr, ud.ptr, self.w.ptr, I, n, stream)
        call("rl_hip_stream_synchronize", stream)
        gd.free()
        ud.free()

    def forward(self, x_ptr, h_ptr, T, ws, stream=None):
        call("rl_hip_gemm_kquant_swiglu", self.qtype, self.w.ptr, x_ptr, h_ptr, ws.ptr, ws.nbytes, self.I, self.n, T,
             stream)

    def __call__(self, X: np.ndarray, stream=None) -> np.ndarray:
        X = _f32(X).reshape(-1, self.n)
        T = X.shape[0]
        xd = DeviceBuffer.from_numpy(X, stream)
        hd = DeviceBuffer(4 * T * self.I)
        self.forward(xd.ptr, hd.ptr, T, kquant_workspace(2 * self.I, self.n, T), stream=stream)
        return hd.numpy(np.float32, (T, self.I), stream)


def kquant_workspace(m: int, n: int, T: int) -> DeviceBuffer:
    """Workspace of one K-quant GEMV stream: split-K tickets + partials, zero-filled
    once (each launch leaves the tickets at zero again)."""
    ws = DeviceBuffer(hip.lib().rl_hip_kquant_workspace_bytes(m, n, T))
    call("rl_hip_memset", ws.ptr, 0, ws.nbytes, None)
    call("rl_hip_stream_synchronize", None)
    return ws


def kquant_linear_T(lin: KQuantLinear, X: np.ndarray, stream=None) -> np.ndarray:
    X = _f32(X).reshape(-1, lin.n)
    T = X.shape[0]
    xd = DeviceBuffer.from_numpy(X, stream)
    yd = DeviceBuffer(4 * T * lin.m)
    lin.forward(xd.ptr, yd.ptr, T, kquant_workspace(lin.m, lin.n, T), stream=stream)
    return yd.numpy(np.float32, (T, lin.m), stream)


def gemv_q4_k(packed: np.ndarray, x: np.ndarray, m: int, n: int) -> np.ndarray:
    """ops::gemv_q4_k(packed, x, y, m, n) (reference src/kernels/ops.h:203)."""
    return kquant_linear_T(KQuantLinear(Q4_K, packed, m, n), x)[0]


def gemv_q6_k(packed: np.ndarray, x: np.ndarray, m: int, n: int) -> np.ndarray:
    """ops::gemv_q6_k(packed, x, y, m, n) (reference src/kernels/ops.h:214)."""
    return kquant_linear_T(KQuantLinear(Q6_K, packed, m, n), x)[0]


def _dequant(qtype: int, packed: np.ndarray, n: int) -> np.ndarray:
    bb = 144 if qtype == Q4_K else 210
    packed = np.ascontiguousarray(packed, np.uint8).reshape(-1)
    nb = n // 256
    assert packed.size >= nb * bb
    src = DeviceBuffer.from_numpy(packed[: nb * bb])
    out = DeviceBuffer(4 * nb * 256)
    call("rl_hip_dequant_kquant", qtype, src.ptr, out.ptr, nb, None)
    return out.numpy(np.float32, (nb * 256,))


def dequant_q4_k(packed: np.ndarray, n: int) -> np.ndarray:
    """ops::dequant_q4_k(packed, out, n) (reference src/kernels/ops.cpp:255)."""
    return _dequant(Q4_K, packed, n)


def dequant_q6_k(packed: np.ndarray, n: int) -> np.ndarray:
    """ops::dequant_q6_k(packed, out, n) (reference src/kernels/ops.cpp:357)."""
    return _dequant(Q6_K, packed, n)


# ------------------------------------------------------------------ norms


def qwen3_rmsnorm(x: np.ndarray, gamma, eps: float = 1e-6) -> np.ndarray:
    """ops::qwen3_rmsnorm over each row of x [T][n] (reference ops.cpp:107)."""
    x = _f32(np.atleast_2d(x))
    T, n = x.shape
    xd = DeviceBuffer.from_numpy(x)
    gd = DeviceBuffer.from_numpy(_f32(gamma)) if gamma is not None else None
    yd = DeviceBuffer(x.nbytes)
    call("rl_hip_rmsnorm_pack", xd.ptr, n, gd.ptr if gd else None, yd.ptr, None, n, T, eps, None)
    return yd.numpy(np.float32, (T, n))


def gated_rmsnorm(o: np.ndarray, z: np.ndarray, gamma, eps: float = 1e-6, gamma_n: int = 0) -> np.ndarray:
    """ops::gated_rmsnorm over each row (reference ops.cpp:129)."""
    o = _f32(np.atleast_2d(o))
    z = _f32(np.atleast_2d(z))
    T, n = o.shape
    od, zd, yd = DeviceBuffer.from_numpy(o), DeviceBuffer.from_numpy(z), DeviceBuffer(o.nbytes)
    gd = DeviceBuffer.from_numpy(_f32(gamma)) if gamma is not None else None
    call("rl_hip_gated_rmsnorm_pack", od.ptr, zd.ptr, n, gd.ptr if gd else None, gamma_n, yd.ptr, None, n, T, eps,
         None)
    return yd.numpy(np.float32, (T, n))


# ------------------------------------------------------------------ DeltaNet


def gdn_decode(qkv, a, b, A_log, dt_bias, conv_w, conv_state, S, nk, nv, v_tiled=False):
    """T-token Gated DeltaNet decode (conv1d_update + gates + delta_recurrent_step,
    reference ops.cpp:458-534, ops_fused.cpp:105-130).  S in the reference layout
    [nv][dk][dv]; returns (o [T][nv*dv], S', conv_state')."""
    qkv = _f32(np.atleast_2d(qkv))
    T, conv_dim = qkv.shape
    nv_, dk, dv = S.shape
    assert nv_ == nv
    St = np.ascontiguousarray(np.transpose(S, (0, 2, 1)), np.float32)
    d_qkv = DeviceBuffer.from_numpy(qkv)
    d_A = DeviceBuffer.from_numpy(_f32(A_log))
    d_dt = DeviceBuffer.from_numpy(_f32(dt_bias))
    d_w = DeviceBuffer.from_numpy(_f32(conv_w))
    d_cin = DeviceBuffer.from_numpy(_f32(conv_state))
    d_cout = DeviceBuffer(d_cin.nbytes)
    d_S = DeviceBuffer.from_numpy(St)
    d_o = DeviceBuffer(4 * T * nv * dv)
    # a and b arrive as their own [T][nv] arrays here: row stride differs from qkv
    # (the engine passes one fused buffer); use a packed copy with a common stride.
    ld = conv_dim + 2 * nv
    fused = np.zeros((T, ld), np.float32)
    fused[:, :conv_dim] = qkv
    fused[:, conv_dim:conv_dim + nv] = np.atleast_2d(a)
    fused[:, conv_dim + nv:] = np.atleast_2d(b)
    d_f = DeviceBuffer.from_numpy(fused)
    call("rl_hip_gdn_decode", d_f.ptr, d_f.ptr + 4 * conv_dim, d_f.ptr + 4 * (conv_dim + nv), ld, d_A.ptr, d_dt.ptr,
         d_w.ptr, d_cin.ptr, d_cout.ptr, d_S.ptr, d_S.ptr, d_o.ptr, T, nk, nv, dk, dv, conv_w.shape[1],
         1 if v_tiled else 0, None)
    o = d_o.numpy(np.float32, (T, nv * dv))
    S_new = np.transpose(d_S.numpy(np.float32, (nv, dv, dk)), (0, 2, 1)).copy()
    conv_new = d_cout.numpy(np.float32, conv_state.shape)
    return o, S_new, conv_new


def gdn_prefill(qkv, a, b, A_log, dt_bias, conv_w, conv_state, S, nk, nv, v_tiled=False):
    """Prompt prefill of T (any) tokens of one Gated DeltaNet layer (same inputs and
    outputs as gdn_decode): conv + gates over all tokens, then the recurrence."""
    qkv = _f32(np.atleast_2d(qkv))
    T, conv_dim = qkv.shape
    nv_, dk, dv = S.shape
    assert nv_ == nv
    ld = conv_dim + 2 * nv
    fused = np.zeros((T, ld), np.float32)
    fused[:, :conv_dim] = qkv
    fused[:, conv_dim:conv_dim + nv] = np.atleast_2d(a)
    fused[:, conv_dim + nv:] = np.atleast_2d(b)
    d_f = DeviceBuffer.from_numpy(fused)
    d_A = DeviceBuffer.from_numpy(_f32(A_log))
    d_dt = DeviceBuffer.from_numpy(_f32(dt_bias))
    d_w = DeviceBuffer.from_numpy(_f32(conv_w))
    d_cin = DeviceBuffer.from_numpy(_f32(conv_state))
    d_cout = DeviceBuffer(d_cin.nbytes)
    d_S = DeviceBuffer.from_numpy(np.ascontiguousarray(np.transpose(S, (0, 2, 1)), np.float32))
    d_o = DeviceBuffer(4 * T * nv * dv)
    ws = DeviceBuffer(hip.lib().rl_hip_gdn_prefill_workspace_bytes(T, nk, nv, dk, dv))
    call("rl_hip_gdn_prefill", d_f.ptr, ld, conv_dim, conv_dim + nv, d_A.ptr, d_dt.ptr, d_w.ptr, d_cin.ptr,
         d_cout.ptr, d_S.ptr, d_o.ptr, ws.ptr, ws.nbytes, T, nk, nv, dk, dv, conv_w.shape[1], 1 if v_tiled else 0,
         None)
    o = d_o.numpy(np.float32, (T, nv * dv))
    S_new = np.transpose(d_S.numpy(np.float32, (nv, dv, dk)), (0, 2, 1)).copy()
    conv_new = d_cout.numpy(np.float32, conv_state.shape)
    return o, S_new, conv_new


# ------------------------------------------------------------------ attention


def kv_layout_k(K):
    """[n_kv][ctx][256] fp16 -> the device K layout, per kv head
    [pos/256][d/32][(pos/16)%16][(d/8)%4][pos%16][d%8]."""
    n_kv, ctx, hd = K.shape
    return np.ascontiguousarray(
        K.reshape(n_kv, ctx // 256, 16, 16, hd // 32, 4, 8).transpose(0, 1, 4, 2, 5, 3, 6))


def kv_layout_v(V):
    """[n_kv][ctx][256] fp16 -> the device V layout, per kv head
    [pos/32][d/16][(pos/8)%4][d%16][pos%8]."""
    n_kv, ctx, hd = V.shape
    return np.ascontiguousarray(V.reshape(n_kv, ctx // 32, 4, 8, hd // 16, 16).transpose(0, 1, 4, 2, 5, 3))


class AttnCache:
    """fp16 K and V caches in HBM, in the device's MFMA fragment order
    (include/rapidllm_hip.h, rl_hip_attn_decode_layer)."""

    def __init__(self, n_kv: int, ctx: int, hd: int = 256):
        assert ctx % 256 == 0
        self.n_kv, self.ctx, self.hd = n_kv, ctx, hd
        self.k = DeviceBuffer(2 * n_kv * ctx * hd)
        self.vt = DeviceBuffer(2 * n_kv * ctx * hd)
        self.k.zero()
        self.vt.zero()
        call("rl_hip_device_synchronize")

    def fill(self, K: np.ndarray, V: np.ndarray):
        """K, V: [pos][n_kv][hd] float values (rounded to fp16 here)."""
        L = K.shape[0]
        kc = np.zeros((self.n_kv, self.ctx, self.hd), np.float16)
        vc = np.zeros((self.n_kv, self.ctx, self.hd), np.float16)
        kc[:, :L, :] = np.transpose(K, (1, 0, 2)).astype(np.float16)
        vc[:, :L, :] = np.transpose(V, (1, 0, 2)).astype(np.float16)
        self.k.upload(kv_layout_k(kc))
        self.vt.upload(kv_layout_v(vc))


def attn_decode_layer(Y, cache: AttnCache, pos: int, q_norm, k_norm, n_q, n_kv, rotary_dim=64, theta=1e7,
                      eps=1e-6):
    """Gated attention for T tokens at positions pos..pos+T-1 from the fused
    projection rows Y [T][2*n_q*hd + 2*n_kv*hd]; returns o*sigmoid(gate) [T][n_q*hd]."""
    Y = _f32(np.atleast_2d(Y))
    T, ld = Y.shape
    hd = cache.hd
    d_Y = DeviceBuffer.from_numpy(Y)
    d_qn = DeviceBuffer.from_numpy(_f32(q_norm))
    d_kn = DeviceBuffer.from_numpy(_f32(k_norm))
    d_pos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    ws = DeviceBuffer(hip.lib().rl_hip_attn_workspace_bytes(n_kv, cache.ctx))
    ws.zero()
    d_out = DeviceBuffer(4 * T * n_q * hd)
    call("rl_hip_attn_decode_layer", d_Y.ptr, ld, d_qn.ptr, d_kn.ptr, cache.k.ptr, cache.vt.ptr, cache.ctx, d_pos.ptr,
         T, n_q, n_kv, hd, rotary_dim, theta, eps, ws.ptr, ws.nbytes, d_out.ptr, None, None)
    return d_out.numpy(np.float32, (T, n_q * hd))


def attn_prefill_layer(Y, cache: AttnCache, pos: int, q_norm, k_norm, n_q, n_kv, rotary_dim=64, theta=1e7,
                       eps=1e-6):
    """Prefill attention for T (any) tokens at positions pos..pos+T-1 (their K/V are
    written to `cache`); returns o*sigmoid(gate) [T][n_q*hd]."""
    Y = _f32(np.atleast_2d(Y))
    T, ld = Y.shape
    hd = cache.hd
    d_Y = DeviceBuffer.from_numpy(Y)
    d_qn = DeviceBuffer.from_numpy(_f32(q_norm))
    d_kn = DeviceBuffer.from_numpy(_f32(k_norm))
    d_pos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    ws = DeviceBuffer(hip.lib().rl_hip_attn_prefill_workspace_bytes(n_q, T))
    d_out = DeviceBuffer(4 * T * n_q * hd)
    call("rl_hip_attn_prefill_layer", d_Y.ptr, ld, d_qn.ptr, d_kn.ptr, cache.k.ptr, cache.vt.ptr, cache.ctx,
         d_pos.ptr, T, n_q, n_kv, hd, rotary_dim, theta, eps, ws.ptr, ws.nbytes, d_out.ptr, None)
    return d_out.numpy(np.float32, (T, n_q * hd))


# ------------------------------------------------------------------ sampling


def argmax_rows(logits: np.ndarray):
    """greedy_sample per row (reference sampler.cpp:8): (indices, values)."""
    logits = _f32(np.atleast_2d(logits))
    rows, V = logits.shape
    d_l = DeviceBuffer.from_numpy(logits)
    d_i = DeviceBuffer(4 * rows)
    d_v = DeviceBuffer(4 * rows)
    ws = DeviceBuffer(hip.lib().rl_hip_argmax_workspace_bytes(rows, V))
    call("rl_hip_argmax_rows", d_l.ptr, rows, V, d_i.ptr, d_v.ptr, ws.ptr, None)
    return d_i.numpy(np.int32, (rows,)), d_v.numpy(np.float32, (rows,))


def accept_prefix(toks, preds, pos: int):
    """Device greedy acceptance: returns (n_consumed, new_pos, next_token)."""
    toks = np.ascontiguousarray(toks, np.int32)
    preds = np.ascontiguousarray(preds, np.int32)
    d_t, d_p = DeviceBuffer.from_numpy(toks), DeviceBuffer.from_numpy(preds)
    d_pos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    d_n, d_nx = DeviceBuffer(4), DeviceBuffer(4)
    call("rl_hip_accept_prefix", d_t.ptr, d_p.ptr, toks.size, d_pos.ptr, d_n.ptr, d_nx.ptr, None)
    return (int(d_n.numpy(np.int32, (1,))[0]), int(d_pos.numpy(np.int32, (1,))[0]),
            int(d_nx.numpy(np.int32, (1,))[0]))


# ------------------------------------------------------------ device-seam single ops


def conv1d_update(x_t, w, state):
    """ops::conv1d_update(x_t, w, state, y, dim, k) (reference ops.cpp:458-468) on the
    device: returns (y, new state)."""
    state = _f32(state)
    dim, k = state.shape
    d_x, d_w, d_s = DeviceBuffer.from_numpy(_f32(x_t)), DeviceBuffer.from_numpy(_f32(w)), DeviceBuffer.from_numpy(state)
    d_y = DeviceBuffer(4 * dim)
    call("rl_hip_conv1d_update", d_x.ptr, d_w.ptr, d_s.ptr, d_y.ptr, dim, k, None)
    return d_y.numpy(np.float32, (dim,)), d_s.numpy(np.float32, (dim, k))


def delta_recurrent_step(S, q, k, v, beta, g_log, eps_l2=1e-6):
    """ops::delta_recurrent_step (reference ops.cpp:495-540) on the device, S
    row-major [n_v][dk][dv]: returns (o [n_v][dv], new S)."""
    S = _f32(S)
    n_v, dk, dv = S.shape
    bufs = [DeviceBuffer.from_numpy(_f32(a)) for a in (S, q, k, v, beta, g_log)]
    d_o = DeviceBuffer(4 * n_v * dv)
    call("rl_hip_delta_recurrent", *[b.ptr for b in bufs], d_o.ptr, n_v, dk, dv, eps_l2, None)
    return d_o.numpy(np.float32, (n_v, dv)), bufs[0].numpy(np.float32, S.shape)


def attn_decode(q, k_cache, v_cache, pos, n_q, n_kv, head_dim):
    """ops::attn_decode (reference ops.cpp:575-605) over fp32 caches [seq][n_kv][hd]."""
    d_q = DeviceBuffer.from_numpy(_f32(q))
    d_k, d_v = DeviceBuffer.from_numpy(_f32(k_cache)), DeviceBuffer.from_numpy(_f32(v_cache))
    d_o = DeviceBuffer(4 * n_q * head_dim)
    call("rl_hip_attn_decode_f32", d_q.ptr, d_k.ptr, d_v.ptr, d_o.ptr, pos, n_q, n_kv, head_dim, None)
    return d_o.numpy(np.float32, (n_q * head_dim,))
