"""ctypes binding to the gfx950 C ABI (include/rapidllm_hip.h).

The library is loaded from rapidllm_amd/_lib/librapidllm_hip.so, built in-tree by
rapidllm_amd/build.py.  There is no fallback: if the library is missing or the
device is not a gfx950, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "librapidllm_hip.so")

_vp = C.c_void_p
_sz = C.c_size_t
_i = C.c_int

# name -> (restype, argtypes); every entry point returns an RlStatus unless noted.
_SIGS = {
    "rl_hip_abi_version": (_i, []),
    "rl_hip_available": (_i, []),
    "rl_hip_last_error": (C.c_char_p, []),
    "rl_hip_device_info": (_i, [C.c_char_p, _i, C.POINTER(_i), C.POINTER(_sz)]),
    "rl_hip_malloc": (_i, [C.POINTER(_vp), _sz]),
    "rl_hip_free": (_i, [_vp]),
    "rl_hip_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "rl_hip_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "rl_hip_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "rl_hip_memset": (_i, [_vp, _i, _sz, _vp]),
    "rl_hip_host_alloc": (_i, [C.POINTER(_vp), _sz]),
    "rl_hip_host_free": (_i, [_vp]),
    "rl_hip_conv1d_update": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_delta_recurrent": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, C.c_float, _vp]),
    "rl_hip_attn_decode_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rl_hip_stream_create": (_i, [C.POINTER(_vp)]),
    "rl_hip_stream_destroy": (_i, [_vp]),
    "rl_hip_stream_synchronize": (_i, [_vp]),
    "rl_hip_device_synchronize": (_i, []),
    "rl_hip_event_create": (_i, [C.POINTER(_vp)]),
    "rl_hip_event_destroy": (_i, [_vp]),
    "rl_hip_event_record": (_i, [_vp, _vp]),
    "rl_hip_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(C.c_float)]),
    "rl_hip_e4m3_to_f32": (_i, [_vp, _vp, _sz, _vp]),
    "rl_hip_fp8_packed_bytes": (_sz, [_i, _i]),
    "rl_hip_fp8_tile_scales": (_sz, [_i, _i]),
    "rl_hip_bf16_packed_bytes": (_sz, [_i, _i]),
    "rl_hip_act_frag_bytes": (_sz, [_i, _i]),
    "rl_hip_pack_fp8": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_pack_bf16": (_i, [_vp, _vp, _i, _i, _vp]),
    "rl_hip_fp8_gate_up_tile_scales": (_sz, [_i, _i]),
    "rl_hip_pack_fp8_gate_up": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_pack_bf16_gate_up": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_pack_act": (_i, [_vp, _vp, _i, _i, _vp]),
    "rl_hip_gemm_fp8_frag": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rl_hip_gemm_bf16_frag": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rl_hip_set_gemm_config": (_i, [_i, _i, _i]),
    "rl_hip_kquant_tiled_bytes": (_sz, [_i, _i, _i]),
    "rl_hip_kquant_workspace_bytes": (_sz, [_i, _i, _i]),
    "rl_hip_pack_kquant": (_i, [_i, _vp, _vp, _i, _i, _vp]),
    "rl_hip_gemm_kquant": (_i, [_i, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "rl_hip_dequant_kquant": (_i, [_i, _vp, _vp, _sz, _vp]),
    "rl_hip_pack_kquant_gate_up": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_gemm_kquant_swiglu": (_i, [_i, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "rl_hip_gemm_kquant_noalloc": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rl_hip_gemm_kquant_noalloc_max_scratch": (_sz, []),
    "rl_hip_gdn_decode": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                               _i, _vp]),
    "rl_hip_gdn_prefill_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "rl_hip_gdn_prefill": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i,
                                _i, _vp]),
    "rl_hip_rmsnorm_pack": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, C.c_float, _vp]),
    "rl_hip_gated_rmsnorm_pack": (_i, [_vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i, C.c_float, _vp]),
    "rl_hip_embed_rows": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "rl_hip_attn_workspace_bytes": (_sz, [_i, _i]),
    "rl_hip_attn_prefill_workspace_bytes": (_sz, [_i, _i]),
    "rl_hip_attn_prefill_layer": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, C.c_float,
                                       C.c_float, _vp, _sz, _vp, _vp]),
    "rl_hip_attn_decode_layer": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, C.c_float, C.c_float,
                                      _vp, _sz, _vp, _vp, _vp]),
    "rl_hip_argmax_workspace_bytes": (_sz, [_i, _i]),
    "rl_hip_argmax_rows": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "rl_hip_accept_prefix": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp]),
    "rl_hip_engine_create": (_vp, [_vp, _vp, _i, _i, _i, C.POINTER(_i)]),
    "rl_hip_engine_create_synthetic": (_vp, [_vp, C.c_uint64, _i, _i, C.POINTER(_i)]),
    "rl_hip_engine_destroy": (None, [_vp]),
    "rl_hip_engine_reset": (_i, [_vp]),
    "rl_hip_engine_prefill": (_i, [_vp, _vp, _i]),
    "rl_hip_engine_decode_token": (_i, [_vp, C.c_int32]),
    "rl_hip_engine_decode_steps": (_i, [_vp, _i]),
    "rl_hip_engine_copy_gen_tokens": (_i, [_vp, _vp, _i]),
    "rl_hip_engine_copy_logits": (_i, [_vp, _vp]),
    "rl_hip_engine_copy_last_hidden": (_i, [_vp, _vp]),
    "rl_hip_engine_mtp_draft": (_i, [_vp, C.c_int32, _i, _vp, C.POINTER(_i)]),
    "rl_hip_engine_spec_verify": (_i, [_vp, _vp, _i, _vp, C.POINTER(_i)]),
    "rl_hip_engine_mtp_spec": (_i, [_vp, C.c_int32, _i, _vp, _vp, C.POINTER(_i)]),
    "rl_hip_engine_set_mtp_mode": (_i, [_vp, _i]),
    "rl_hip_engine_mtp_mode": (_i, [_vp, C.POINTER(_i), C.POINTER(_i)]),
    "rl_hip_engine_copy_mtp_hidden": (_i, [_vp, _vp]),
    "rl_hip_engine_greedy": (_i, [_vp, C.POINTER(C.c_int32)]),
    "rl_hip_engine_pos": (_i, [_vp, C.POINTER(_i)]),
    "rl_hip_engine_info": (_i, [_vp, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_sz)]),
    "rl_hip_engine_set_pos": (_i, [_vp, _i]),
    "rl_hip_engine_synthetic_context": (_i, [_vp, _i, C.c_uint64]),
    "rl_hip_engine_time_steps": (_i, [_vp, _i, _i, _i, C.POINTER(C.c_float)]),
    "rl_hip_engine_time_layer": (_i, [_vp, _i, _i, _i, C.POINTER(C.c_float)]),
    "rl_hip_engine_stream": (_vp, [_vp]),
    "rl_hip_engine_create_batch": (_vp, [_vp, _vp, _i, _i, _i, _i, C.POINTER(_i)]),
    "rl_hip_engine_create_synthetic_batch": (_vp, [_vp, C.c_uint64, _i, _i, _i, C.POINTER(_i)]),
    "rl_hip_engine_max_batch": (_i, [_vp, C.POINTER(_i)]),
    "rl_hip_engine_decode_tokens": (_i, [_vp, _vp, _vp, _i]),
    "rl_hip_engine_copy_logits_n": (_i, [_vp, _vp, _i]),
    "rl_hip_engine_copy_greedy_n": (_i, [_vp, _vp, _i]),
    "rl_hip_engine_replicate_slot0": (_i, [_vp, _i]),
    "rl_hip_engine_zero_slots": (_i, [_vp, _i]),
    "rl_hip_engine_prefill_slot": (_i, [_vp, _vp, _i, _i]),
    "rl_hip_engine_prefill_eq_batch": (_i, [_vp, _vp, _i, _i]),
    "rl_hip_engine_time_batch": (_i, [_vp, _i, _i, C.POINTER(C.c_float)]),
    "rl_hip_weights_open": (_vp, [C.c_char_p, _i, C.POINTER(C.c_int)]),
    "rl_hip_weights_close": (None, [_vp]),
    "rl_hip_weights_config": (_i, [_vp, _vp, C.POINTER(C.c_int)]),
    "rl_hip_weights_table": (_i, [_vp, _vp, C.POINTER(C.c_int)]),
    "rl_hip_weights_info": (_i, [_vp, _i, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_int64),
                                 C.POINTER(C.c_int), C.POINTER(C.c_uint64), C.POINTER(C.c_int)]),
    "rl_hip_map_name": (_i, [_i, C.c_char_p, C.c_char_p, _i]),
    "rl_hip_copy_probe": (_i, [_vp, _vp, _sz, _vp]),
    "rl_hip_read_probe": (_i, [_vp, _sz, _vp, _vp]),
    "rl_hip_norm_group_rows": (_i, []),
    "rl_hip_time_gemv_fp8_valu": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _vp, C.POINTER(C.c_float)]),
    "rl_hip_time_gemm_fp8": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp,
                                  C.POINTER(C.c_float)]),
    "rl_hip_gemm_fp8": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rl_hip_gemm_fp8_prefill": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "rl_hip_gemm_bf16_prefill": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "rl_hip_kquant_to_bf16x2": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_kquant_to_f16": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_act_frag_to_f16": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "rl_hip_gemm_f16_prefill": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "rl_hip_time_gemm_kquant": (_i, [_i, _vp, _i, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp, C.POINTER(C.c_float)]),
    "rl_hip_time_gdn": (_i, [_vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i,
                             _i, _vp, C.POINTER(C.c_float)]),
}

_lib = None


class HipError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (status {code}): {msg}")
        self.code = code


def lib() -> C.CDLL:
    """Load the HIP library; raises if it was not built (no CPU fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run rapidllm_amd/build.py (hipcc, gfx950)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def declared_symbols():
    return list(_SIGS)


def call(name: str, *args) -> None:
    """Call an RlStatus-returning entry point and raise on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise HipError(name, rc, lib().rl_hip_last_error().decode(errors="replace"))


def require_gpu() -> None:
    if not lib().rl_hip_available():
        raise RuntimeError("no gfx950 device visible to the HIP runtime")


class DeviceBuffer:
    """Owning device allocation (rl_hip_malloc / rl_hip_free)."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        call("rl_hip_malloc", C.byref(p), max(int(nbytes), 1))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_numpy(cls, a: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            call("rl_hip_memcpy_h2d", b.ptr, a.ctypes.data, a.nbytes, stream)
            call("rl_hip_stream_synchronize", stream)
        return b

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        call("rl_hip_memcpy_h2d", self.ptr, a.ctypes.data, a.nbytes, stream)
        call("rl_hip_stream_synchronize", stream)

    def numpy(self, dtype, shape, stream=None, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes
        if out.nbytes:
            call("rl_hip_memcpy_d2h", out.ctypes.data, self.ptr + offset, out.nbytes, stream)
        return out

    def zero(self, stream=None) -> None:
        call("rl_hip_memset", self.ptr, 0, self.nbytes, stream)

    def free(self) -> None:
        if self.ptr:
            call("rl_hip_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.rl_hip_free(self.ptr)
                self.ptr = None
        except Exception:
            pass


def synchronize() -> None:
    call("rl_hip_device_synchronize")


class Timer:
    """HIP events recorded on `stream` (the stream the kernels run on)."""

    def __init__(self, stream=None):
        self.stream = stream
        a, b = C.c_void_p(), C.c_void_p()
        call("rl_hip_event_create", C.byref(a))
        call("rl_hip_event_create", C.byref(b))
        self.a, self.b = a.value, b.value

    def start(self):
        call("rl_hip_event_record", self.a, self.stream)

    def stop(self) -> float:
        call("rl_hip_event_record", self.b, self.stream)
        ms = C.c_float()
        call("rl_hip_event_elapsed_ms", self.a, self.b, C.byref(ms))
        return ms.value

    def elapsed(self) -> float:
        """ms between the two recorded events (waits for the second)."""
        ms = C.c_float()
        call("rl_hip_event_elapsed_ms", self.a, self.b, C.byref(ms))
        return ms.value

    def __del__(self):
        try:
            if _lib is not None:
                _lib.rl_hip_event_destroy(self.a)
                _lib.rl_hip_event_destroy(self.b)
        except Exception:
            pass
