"""Host-side mirror of the reference's GPU engine seam, cuda_gen::Engine
(include/rapidllm/runtime/cuda_engine.h:13-83), over the C ABI rl_hip_engine_*.

Method names and meaning follow the reference: prefill, decode_token,
decode_steps, copy_gen_tokens, copy_logits, copy_last_hidden, mtp_draft,
spec_verify (returns n_consumed; preds[i] = greedy after toks[i]), greedy, pos.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip
from .hip import call
from .model import ModelSpec, WeightTable


class Engine:
    def __init__(self, spec: ModelSpec, weights: WeightTable | None = None, ctx: int = 4096, max_T: int = 4,
                 seed: int = 0):
        L = hip.lib()
        self.spec = spec
        self._cfg = spec.c_config()
        st = C.c_int(0)
        if weights is None:
            h = L.rl_hip_engine_create_synthetic(C.byref(self._cfg), seed, ctx, max_T, C.byref(st))
        else:
            arr, n = weights.c_array()
            h = L.rl_hip_engine_create(C.byref(self._cfg), arr, n, ctx, max_T, C.byref(st))
        if not h:
            raise hip.HipError("rl_hip_engine_create", st.value, L.rl_hip_last_error().decode(errors="replace"))
        self.h = h
        self.max_T = max_T
        v, hd, cap, nb = C.c_int(), C.c_int(), C.c_int(), C.c_size_t()
        call("rl_hip_engine_info", h, C.byref(v), C.byref(hd), C.byref(cap), C.byref(nb))
        self.vocab, self.hidden, self.ctx_capacity, self.device_bytes = v.value, hd.value, cap.value, nb.value

    def close(self):
        if getattr(self, "h", None):
            hip.lib().rl_hip_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- cuda_gen::Engine surface
    def reset(self):
        call("rl_hip_engine_reset", self.h)

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        call("rl_hip_engine_prefill", self.h, ids.ctypes.data, ids.size)

    def decode_token(self, token: int):
        call("rl_hip_engine_decode_token", self.h, int(token))

    def decode_steps(self, n: int):
        call("rl_hip_engine_decode_steps", self.h, n)

    def copy_gen_tokens(self, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        call("rl_hip_engine_copy_gen_tokens", self.h, out.ctypes.data, n)
        return out

    def copy_logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        call("rl_hip_engine_copy_logits", self.h, out.ctypes.data)
        return out

    def copy_last_hidden(self) -> np.ndarray:
        out = np.empty(self.hidden, np.float32)
        call("rl_hip_engine_copy_last_hidden", self.h, out.ctypes.data)
        return out

    def mtp_draft(self, first: int, n: int) -> np.ndarray:
        out = np.zeros(max(n, 1), np.int32)
        k = C.c_int()
        call("rl_hip_engine_mtp_draft", self.h, int(first), n, out.ctypes.data, C.byref(k))
        return out[: k.value]

    def spec_verify(self, toks):
        toks = np.ascontiguousarray(toks, np.int32)
        preds = np.zeros(toks.size, np.int32)
        k = C.c_int()
        call("rl_hip_engine_spec_verify", self.h, toks.ctypes.data, toks.size, preds.ctypes.data, C.byref(k))
        return k.value, preds

    def mtp_spec(self, t0: int, T: int):
        toks = np.zeros(T, np.int32)
        preds = np.zeros(T, np.int32)
        k = C.c_int()
        call("rl_hip_engine_mtp_spec", self.h, int(t0), T, toks.ctypes.data, preds.ctypes.data, C.byref(k))
        return k.value, toks, preds

    def greedy(self) -> int:
        t = C.c_int32()
        call("rl_hip_engine_greedy", self.h, C.byref(t))
        return t.value

    def pos(self) -> int:
        p = C.c_int()
        call("rl_hip_engine_pos", self.h, C.byref(p))
        return p.value

    # ---- benchmark support
    def set_pos(self, pos: int):
        call("rl_hip_engine_set_pos", self.h, pos)

    def synthetic_context(self, n: int, seed: int = 7):
        call("rl_hip_engine_synthetic_context", self.h, n, seed)

    def time_steps(self, T: int, iters: int, mtp_drafts: int = 0) -> float:
        ms = C.c_float()
        call("rl_hip_engine_time_steps", self.h, T, iters, mtp_drafts, C.byref(ms))
        return ms.value

    # ---- Session-level generate (session.cpp:687-829 semantics)
    def generate(self, prompt, max_new: int, spec_n: int = 0):
        """Greedy generation; spec_n > 0 uses MTP draft + verify at T = spec_n + 1.
        Returns (tokens, proposed, accepted)."""
        self.prefill(prompt)
        out = []
        proposed = accepted = 0
        while len(out) < max_new:
            t0 = self.greedy()
            out.append(t0)
            if len(out) >= max_new:
                break
            if spec_n > 0:
                T = min(spec_n + 1, self.max_T)
                k, toks, preds = self.mtp_spec(t0, T)
                proposed += T - 1
                for i in range(1, k):
                    if len(out) < max_new:
                        out.append(int(toks[i]))
                        accepted += 1
            else:
                self.decode_token(t0)
        return out[:max_new], proposed, accepted
