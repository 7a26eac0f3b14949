"""Checkpoint loading over the C ABI rl_hip_weights_* (host code, no GPU).

Mirrors the reference's WeightStore::open(path) (src/frontend/weight_store.cpp:
137-155): an HF directory of FP8 safetensors or a GGUF file becomes the table of
IR-named tensors plus the model description the engine is created from::

    ck = Checkpoint("/models/qwen36-27b-fp8")
    eng = Engine(ck.spec, ck, ctx=8192)

`Checkpoint` can stand wherever a WeightTable is taken (Engine, OracleModel): it
exposes the same c_array().  The mapped files stay open until close().
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import hip
from .model import ModelSpec, RlModelConfig, RlTensor

SOURCE_HF, SOURCE_GGUF = 0, 1
_ELEM = {0: np.float32, 1: np.uint16, 2: np.uint16, 3: np.uint8}


def map_name(src: str, gguf: bool = False) -> str:
    """IR name of a checkpoint tensor name (map_hf_name / map_gguf_name)."""
    buf = C.create_string_buffer(512)
    hip.call("rl_hip_map_name", 1 if gguf else 0, src.encode(), buf, len(buf))
    return buf.value.decode()


def spec_from_config(c: RlModelConfig) -> ModelSpec:
    kinds = [int(c.layer_kind[i]) for i in range(c.n_layers)]
    return ModelSpec(vocab=c.vocab, hidden=c.hidden, n_layers=c.n_layers, intermediate=c.intermediate,
                     n_k_heads=c.n_k_heads, n_v_heads=c.n_v_heads, k_dim=c.k_dim, v_dim=c.v_dim, conv_k=c.conv_k,
                     n_q=c.n_q, n_kv=c.n_kv, head_dim=c.head_dim, rotary_dim=c.rotary_dim,
                     rope_theta=float(c.rope_theta), rms_eps=float(c.rms_eps), v_tiled=bool(c.v_tiled),
                     has_mtp=bool(c.has_mtp), layer_kinds=kinds)


class Checkpoint:
    def __init__(self, path: str | os.PathLike, max_layers: int = -1):
        L = hip.lib()
        st = C.c_int(0)
        h = L.rl_hip_weights_open(os.fspath(path).encode(), max_layers, C.byref(st))
        if not h:
            raise hip.HipError("rl_hip_weights_open", st.value, L.rl_hip_last_error().decode(errors="replace"))
        self.h = h
        self.cfg = RlModelConfig()
        src = C.c_int(0)
        hip.call("rl_hip_weights_config", h, C.byref(self.cfg), C.byref(src))
        self.source = src.value
        self.spec = spec_from_config(self.cfg)
        ptr = C.c_void_p()
        n = C.c_int(0)
        hip.call("rl_hip_weights_table", h, C.byref(ptr), C.byref(n))
        self._n = n.value
        self._arr = C.cast(ptr, C.POINTER(RlTensor * max(n.value, 1))).contents if n.value else None
        self._index = {self._arr[i].name.decode(): i for i in range(self._n)} if self._n else {}

    def close(self):
        if getattr(self, "h", None):
            hip.lib().rl_hip_weights_close(self.h)
            self.h = None
            self._arr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- WeightTable surface
    def c_array(self):
        return self._arr, self._n

    def names(self):
        return list(self._index)

    def __contains__(self, name):
        return name in self._index

    def info(self, name: str) -> dict:
        """TensorDesc facts: src_name, shape, gguf_type, nbytes, n_scale."""
        i = self._index[name]
        src = C.c_char_p()
        nd, gt, ns = C.c_int(), C.c_int(), C.c_int()
        shp = (C.c_int64 * 4)()
        nb = C.c_uint64()
        hip.call("rl_hip_weights_info", self.h, i, C.byref(src), C.byref(nd), shp, C.byref(gt), C.byref(nb),
                 C.byref(ns))
        return dict(src_name=src.value.decode(), shape=tuple(shp[: nd.value]), gguf_type=gt.value, nbytes=nb.value,
                    n_scale=ns.value)

    def get(self, name: str):
        """(quant, rows, cols, data, scale): data as a numpy view of the stored
        elements (float32 / uint16 / uint8 / raw bytes for block formats)."""
        t = self._arr[self._index[name]]
        inf = self.info(name)
        nbytes = inf["nbytes"]
        raw = np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_uint8)), shape=(nbytes,)) if nbytes else \
            np.zeros(0, np.uint8)
        dt = _ELEM.get(t.quant)
        data = raw.view(dt) if dt is not None else raw
        scale = None
        if t.scale:
            scale = np.ctypeslib.as_array(C.cast(t.scale, C.POINTER(C.c_float)), shape=(inf["n_scale"],))
        return t.quant, t.rows, t.cols, data, scale


