"""Loader for the tiny-hybrid fixture (tests/golden/tiny_hybrid.{npz,json}),
generated from the reference's python/goldens/tiny_hybrid.py."""
import json
import os

import numpy as np

from rapidllm_amd import model as M

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load():
    meta = json.load(open(os.path.join(GOLDEN, "tiny_hybrid.json")))
    c = meta["config"]
    kinds = [M.LAYER_DELTA if t == "linear_attention" else M.LAYER_ATTN for t in c["layer_types"]]
    spec = M.ModelSpec(vocab=c["vocab_size"], hidden=c["hidden_size"], n_layers=c["num_hidden_layers"],
                       intermediate=c["intermediate_size"], n_k_heads=c["linear_num_key_heads"],
                       n_v_heads=c["linear_num_value_heads"], k_dim=c["linear_key_head_dim"],
                       v_dim=c["linear_value_head_dim"], conv_k=c["linear_conv_kernel_dim"],
                       n_q=c["num_attention_heads"], n_kv=c["num_key_value_heads"], head_dim=c["head_dim"],
                       rotary_dim=int(c["head_dim"] * c["partial_rotary_factor"]), rope_theta=c["rope_theta"],
                       rms_eps=c["rms_norm_eps"], has_mtp=True, layer_kinds=kinds)
    W = M.WeightTable()
    with np.load(os.path.join(GOLDEN, "tiny_hybrid.npz")) as z:
        for name in z.files:
            a = np.ascontiguousarray(z[name], np.float32)
            rows, cols = (a.shape[0], a.shape[1]) if a.ndim == 2 else (a.shape[0], 1)
            W.add(name, M.Q_F32, a, rows, cols)
    return spec, W, meta
