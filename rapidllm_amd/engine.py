"""Host-side mirror of the reference's GPU engine seam, cuda_gen::Engine
(include/rapidllm/runtime/cuda_engine.h:13-83), over the C ABI rl_hip_engine_*.

Method names and meaning follow the reference: prefill, decode_token,
decode_steps, copy_gen_tokens, copy_logits, copy_last_hidden, mtp_draft,
spec_verify (returns n_consumed; preds[i] = greedy after toks[i]), greedy, pos,
and the continuous-batch calls max_batch, decode_tokens, copy_logits_n,
copy_greedy_n, replicate_slot0, zero_slots, prefill_slot (cuda_engine.h:46-66).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip
from .hip import call
from .model import ModelSpec, WeightTable


MTP_STEM, MTP_LAYER = 0, 1


class Engine:
    def __init__(self, spec: ModelSpec, weights: WeightTable | None = None, ctx: int = 4096, max_T: int = 4,
                 seed: int = 0, max_batch: int = 1):
        L = hip.lib()
        self.spec = spec
        self._cfg = spec.c_config()
        st = C.c_int(0)
        if weights is None:
            h = L.rl_hip_engine_create_synthetic_batch(C.byref(self._cfg), seed, ctx, max_T, max_batch, C.byref(st))
        else:
            arr, n = weights.c_array()
            h = L.rl_hip_engine_create_batch(C.byref(self._cfg), arr, n, ctx, max_T, max_batch, C.byref(st))
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

    def set_mtp_mode(self, mode: int) -> None:
        """MTP_STEM (Session::mtp_draft) or MTP_LAYER (stem + mtp.layers[0],
        Session::mtp_layer_step)."""
        call("rl_hip_engine_set_mtp_mode", self.h, int(mode))

    def mtp_mode(self):
        """(mode, whether the model has the MTP decoder layer)."""
        m, a = C.c_int(), C.c_int()
        call("rl_hip_engine_mtp_mode", self.h, C.byref(m), C.byref(a))
        return m.value, bool(a.value)

    def copy_mtp_hidden(self) -> np.ndarray:
        h = np.empty(self.spec.hidden, np.float32)
        call("rl_hip_engine_copy_mtp_hidden", self.h, h.ctypes.data)
        return h

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

    def time_layer(self, layer: int, T: int, iters: int) -> float:
        """Average graph-replayed ms of layer `layer`'s launches alone (n_layers: the
        step's head and tail alone), T tokens (bench)."""
        ms = C.c_float()
        call("rl_hip_engine_time_layer", self.h, layer, T, iters, C.byref(ms))
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

    # ---- continuous batch (cuda_engine.h:46-66)
    def max_batch(self) -> int:
        b = C.c_int()
        call("rl_hip_engine_max_batch", self.h, C.byref(b))
        return b.value

    def decode_tokens(self, tokens, poss):
        tokens = np.ascontiguousarray(tokens, np.int32)
        poss = np.ascontiguousarray(poss, np.int32)
        assert tokens.size == poss.size
        call("rl_hip_engine_decode_tokens", self.h, tokens.ctypes.data, poss.ctypes.data, tokens.size)

    def copy_logits_n(self, B: int) -> np.ndarray:
        out = np.empty((B, self.vocab), np.float32)
        call("rl_hip_engine_copy_logits_n", self.h, out.ctypes.data, B)
        return out

    def copy_greedy_n(self, B: int) -> list:
        out = np.zeros(B, np.int32)
        call("rl_hip_engine_copy_greedy_n", self.h, out.ctypes.data, B)
        return [int(v) for v in out]

    def replicate_slot0(self, n_slots: int):
        call("rl_hip_engine_replicate_slot0", self.h, n_slots)

    def zero_slots(self, n_slots: int):
        call("rl_hip_engine_zero_slots", self.h, n_slots)

    def prefill_slot(self, ids, slot: int):
        ids = np.ascontiguousarray(ids, np.int32)
        call("rl_hip_engine_prefill_slot", self.h, ids.ctypes.data, ids.size, slot)

    def prefill_eq_batch(self, prompts):
        """Equal-length prompts into slots 0 .. B-1 (zero_slots first, as the
        Session does); then copy_logits_n / copy_greedy_n hold each slot's row."""
        ids = np.ascontiguousarray(np.asarray(prompts, np.int32).T)  # time-major [T][B]
        T, B = ids.shape
        call("rl_hip_engine_prefill_eq_batch", self.h, ids.ctypes.data, T, B)

    def time_batch(self, B: int, iters: int) -> float:
        ms = C.c_float()
        call("rl_hip_engine_time_batch", self.h, B, iters, C.byref(ms))
        return ms.value

    def generate_batch(self, prompts, max_new: int):
        """Session::generate_batch (src/runtime/session.cpp:832-964) for unequal or
        distinct prompts: prefill each sequence into its slot, then one decode_tokens
        per step for the sequences still running."""
        B = len(prompts)
        assert 1 <= B <= self.max_batch()
        outs, toks, poss = [], [], []
        for b, p in enumerate(prompts):
            self.prefill_slot(p, b)
            t0 = int(np.argmax(self.copy_logits()))
            outs.append([t0])
            toks.append(t0)
            poss.append(len(p))
        while min(len(o) for o in outs) < max_new:
            self.decode_tokens(toks, poss)
            nxt = self.copy_greedy_n(B)
            for b in range(B):
                poss[b] += 1
                toks[b] = nxt[b]
                if len(outs[b]) < max_new:
                    outs[b].append(nxt[b])
        return outs

