"""Model description and weight tables for the hybrid decoder (C structs of
include/rl_model.h), shared by the HIP engine and the CPU oracle.

ModelSpec mirrors the reference's ModelDesc defaults (include/rapidllm/ir/
model_desc.h:55-147): Qwen3.6/3.8-27B = 64 layers (48 Gated DeltaNet + 16 gated
attention, pattern D D D A), hidden 5120, intermediate 17408, vocab 248320,
DeltaNet 16 k-heads / 48 v-heads of 128, attention 24 q / 4 kv heads of 256,
rotary 64 (partial factor 0.25), theta 1e7, eps 1e-6.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import synth

RL_MAX_LAYERS = 256
Q_F32, Q_F16, Q_BF16, Q_FP8, Q_Q4_K, Q_Q6_K = 0, 1, 2, 3, 6, 8
LAYER_DELTA, LAYER_ATTN = 0, 1


class RlModelConfig(C.Structure):
    _fields_ = [
        ("vocab", C.c_int), ("hidden", C.c_int), ("n_layers", C.c_int), ("intermediate", C.c_int),
        ("n_k_heads", C.c_int), ("n_v_heads", C.c_int), ("k_dim", C.c_int), ("v_dim", C.c_int), ("conv_k", C.c_int),
        ("n_q", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int), ("rotary_dim", C.c_int),
        ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("v_tiled", C.c_int), ("has_mtp", C.c_int),
        ("layer_kind", C.c_ubyte * RL_MAX_LAYERS),
    ]


class RlTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("quant", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("scale", C.c_void_p)]


@dataclass
class ModelSpec:
    vocab: int = 248320
    hidden: int = 5120
    n_layers: int = 64
    intermediate: int = 17408
    n_k_heads: int = 16
    n_v_heads: int = 48
    k_dim: int = 128
    v_dim: int = 128
    conv_k: int = 4
    n_q: int = 24
    n_kv: int = 4
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 1e7
    rms_eps: float = 1e-6
    v_tiled: bool = False
    has_mtp: bool = True
    mtp_layer: bool = False  # random_weights adds the MTP decoder layer mtp.layers[0].*
    layer_kinds: list = field(default_factory=list)

    def __post_init__(self):
        if not self.layer_kinds:
            # full attention every 4th layer (D D D A), as the 27B hybrid
            self.layer_kinds = [LAYER_ATTN if (i % 4) == 3 else LAYER_DELTA for i in range(self.n_layers)]

    @property
    def conv_dim(self):
        return 2 * self.n_k_heads * self.k_dim + self.n_v_heads * self.v_dim

    def c_config(self) -> RlModelConfig:
        c = RlModelConfig()
        for f, _ in RlModelConfig._fields_:
            if f == "layer_kind":
                continue
            v = getattr(self, f)
            setattr(c, f, int(v) if isinstance(v, bool) else v)
        for i, k in enumerate(self.layer_kinds):
            c.layer_kind[i] = k
        return c


def qwen27b_spec(**kw) -> ModelSpec:
    return ModelSpec(**kw)


class WeightTable:
    """Host weights by IR name, kept alive for the C side (RlTensor array)."""

    def __init__(self):
        self.t = {}  # name -> (quant, rows, cols, data ndarray, scale ndarray | None)

    def add(self, name, quant, data, rows, cols, scale=None):
        self.t[name] = (quant, rows, cols, np.ascontiguousarray(data),
                        None if scale is None else np.ascontiguousarray(scale, np.float32))

    def c_array(self):
        arr = (RlTensor * len(self.t))()
        self._names = []
        for i, (name, (q, r, c, d, s)) in enumerate(self.t.items()):
            nb = name.encode()
            self._names.append(nb)
            arr[i].name = nb
            arr[i].quant = q
            arr[i].rows = r
            arr[i].cols = c
            arr[i].data = d.ctypes.data
            arr[i].scale = s.ctypes.data if s is not None else None
        self._arr = arr
        return arr, len(self.t)


BIG = 1 << 26  # matrices of at least this many entries use the one-pass generators


def random_weights(spec: ModelSpec, seed: int = 1, linear_quant: int = Q_FP8, embed_quant: int = Q_BF16,
                   head_quant: int = Q_BF16, w_scale=(1e-3, 1e-1)) -> WeightTable:
    """Random-init weights of the architecture (benchmark distributions): FP8 linears
    with log-uniform block scales (or Q4_K / Q6_K blocks), bf16 embedding/lm_head."""
    r = synth.rng(seed)
    W = WeightTable()
    H, V = spec.hidden, spec.vocab

    def lin(name, m, n, quant=linear_quant):
        if quant == Q_FP8:
            w = synth.fp8_weight_wide(r, m, n) if m * n >= BIG else synth.fp8_weight(r, m, n)
            W.add(name, Q_FP8, w, m, n, synth.fp8_scales(r, m, n, *w_scale))
        elif quant == Q_BF16 and m * n >= BIG:
            W.add(name, Q_BF16, synth.bf16_random_bits(r, m, n), m, n)
        elif quant == Q_BF16:
            W.add(name, Q_BF16, synth.bf16_bits(r.standard_normal((m, n)).astype(np.float32) * 0.02), m, n)
        elif quant == Q_Q4_K:
            W.add(name, Q_Q4_K, synth.q4k_blocks(r, m, n), m, n)
        elif quant == Q_Q6_K:
            W.add(name, Q_Q6_K, synth.q6k_blocks(r, m, n), m, n)
        else:
            raise ValueError(quant)

    def vec(name, n, mean=0.0, std=0.1):
        W.add(name, Q_F32, (mean + std * r.standard_normal(n)).astype(np.float32), n, 1)

    if V * H >= BIG and embed_quant == Q_BF16:
        W.add("embed", Q_BF16, synth.bf16_random_bits(r, V, H), V, H)
    else:
        emb = (r.standard_normal((V, H)) * 0.02).astype(np.float32)
        if embed_quant == Q_BF16:
            W.add("embed", Q_BF16, synth.bf16_bits(emb), V, H)
        else:
            W.add("embed", Q_F32, emb, V, H)
    lin("lm_head", V, H, head_quant)
    vec("final_norm", H)
    nk, nv, dk, dv = spec.n_k_heads, spec.n_v_heads, spec.k_dim, spec.v_dim
    nq, nkv, hd, I = spec.n_q, spec.n_kv, spec.head_dim, spec.intermediate
    for i, kind in enumerate(spec.layer_kinds):
        p = f"layers[{i}]."
        vec(p + "attn_norm", H)
        vec(p + "ffn_norm", H)
        if kind == LAYER_DELTA:
            lin(p + "delta.gemm.in_proj_qkv", spec.conv_dim, H)
            lin(p + "delta.gemm.in_proj_z", nv * dv, H)
            lin(p + "delta.leftover.in_proj_a", nv, H, Q_FP8 if linear_quant == Q_FP8 else Q_BF16)
            lin(p + "delta.leftover.in_proj_b", nv, H, Q_FP8 if linear_quant == Q_FP8 else Q_BF16)
            lin(p + "delta.gemm.out_proj", H, nv * dv)
            vec(p + "delta.leftover.a_log", nv, 0.0, 0.5)
            vec(p + "delta.leftover.dt_bias", nv, 0.0, 0.5)
            W.add(p + "delta.leftover.conv1d", Q_F32, (r.standard_normal((spec.conv_dim, spec.conv_k)) * 0.5)
                  .astype(np.float32), spec.conv_dim, spec.conv_k)
            vec(p + "delta.leftover.norm", dv, 1.0, 0.1)
        else:
            lin(p + "attn.wq", 2 * nq * hd, H)
            lin(p + "attn.wk", nkv * hd, H)
            lin(p + "attn.wv", nkv * hd, H)
            lin(p + "attn.wo", H, nq * hd)
            vec(p + "attn.q_norm", hd)
            vec(p + "attn.k_norm", hd)
        lin(p + "mlp.gate", I, H)
        lin(p + "mlp.up", I, H)
        lin(p + "mlp.down", H, I)
    if spec.has_mtp:
        lin("mtp.fc", H, 2 * H)
        vec("mtp.pre_fc_norm_hidden", H)
        vec("mtp.pre_fc_norm_embedding", H)
        vec("mtp.norm", H)
        if spec.mtp_layer:
            p = "mtp.layers[0]."
            vec(p + "attn_norm", H)
            vec(p + "ffn_norm", H)
            lin(p + "attn.wq", 2 * nq * hd, H)
            lin(p + "attn.wk", nkv * hd, H)
            lin(p + "attn.wv", nkv * hd, H)
            lin(p + "attn.wo", H, nq * hd)
            vec(p + "attn.q_norm", hd)
            vec(p + "attn.k_norm", hd)
            lin(p + "mlp.gate", I, H)
            lin(p + "mlp.up", I, H)
            lin(p + "mlp.down", H, I)
    return W
