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


def kquant_workspace(m: int, n: int, T: int) -> DeviceBuffer:
    return DeviceBuffer(hip.lib().rl_hip_kquant_workspace_bytes(m, n, T))


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
