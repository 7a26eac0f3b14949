"""Generate the tiny-hybrid model fixture from the reference's own golden script.

Runs reference python/goldens/tiny_hybrid.py (stdlib-only, its main():
tiny_hybrid.py:666-) into a temporary directory -- in the build container only,
where /root/reference exists -- and converts what it writes into two committed
fixtures:

  tiny_hybrid.npz   every F32 tensor of tiny_hybrid/model.safetensors under the
                    IR names the engine's weight table uses (mapping below,
                    following hf_tensors, tiny_hybrid.py:463-510)
  tiny_hybrid.json  the script's config (hidden 32, vocab 48, 8 layers D D D A ...)
                    and golden.json: prompt_ids, greedy_ids, mtp_draft_ids

The greedy ids come from the script's forward() (token-by-token prefill then
greedy decode, tiny_hybrid.py:221-354) and the drafts from mtp_draft_py()
(NextN stem: concat(norm(embed), norm(hidden)) -> fc -> norm -> lm_head,
tiny_hybrid.py:357-430).  Usage:  python tests/golden/make_tiny_hybrid.py
"""
from __future__ import annotations

import json
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

REF_SCRIPT = "/root/reference/python/goldens/tiny_hybrid.py"
HERE = os.path.dirname(os.path.abspath(__file__))


def read_safetensors_f32(path):
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        blob = f.read()
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        assert meta["dtype"] == "F32", (name, meta["dtype"])
        a, b = meta["data_offsets"]
        out[name] = np.frombuffer(blob[a:b], dtype="<f4").reshape(meta["shape"]).copy()
    return out


def ir_name(hf):
    """HF tensor name -> engine IR name (None for tensors the decode path never reads)."""
    lm = "model.language_model."
    fixed = {
        lm + "embed_tokens.weight": "embed",
        "lm_head.weight": "lm_head",
        lm + "norm.weight": "final_norm",
        "mtp.fc.weight": "mtp.fc",
        "mtp.norm.weight": "mtp.norm",
        "mtp.pre_fc_norm_hidden.weight": "mtp.pre_fc_norm_hidden",
        "mtp.pre_fc_norm_embedding.weight": "mtp.pre_fc_norm_embedding",
    }
    if hf in fixed:
        return fixed[hf]
    if not hf.startswith(lm + "layers."):
        return None  # vision stub, the MTP decoder layer (the stem draft skips it)
    rest = hf[len(lm + "layers."):]
    i, sub = rest.split(".", 1)
    p = f"layers[{int(i)}]."
    table = {
        "input_layernorm.weight": "attn_norm",
        "post_attention_layernorm.weight": "ffn_norm",
        "mlp.gate_proj.weight": "mlp.gate",
        "mlp.up_proj.weight": "mlp.up",
        "mlp.down_proj.weight": "mlp.down",
        "linear_attn.in_proj_qkv.weight": "delta.gemm.in_proj_qkv",
        "linear_attn.in_proj_z.weight": "delta.gemm.in_proj_z",
        "linear_attn.out_proj.weight": "delta.gemm.out_proj",
        "linear_attn.in_proj_a.weight": "delta.leftover.in_proj_a",
        "linear_attn.in_proj_b.weight": "delta.leftover.in_proj_b",
        "linear_attn.A_log": "delta.leftover.a_log",
        "linear_attn.dt_bias": "delta.leftover.dt_bias",
        "linear_attn.conv1d.weight": "delta.leftover.conv1d",
        "linear_attn.norm.weight": "delta.leftover.norm",
        "self_attn.q_proj.weight": "attn.wq",
        "self_attn.k_proj.weight": "attn.wk",
        "self_attn.v_proj.weight": "attn.wv",
        "self_attn.o_proj.weight": "attn.wo",
        "self_attn.q_norm.weight": "attn.q_norm",
        "self_attn.k_norm.weight": "attn.k_norm",
    }
    return p + table[sub]


def main():
    if not os.path.exists(REF_SCRIPT):
        sys.exit(f"{REF_SCRIPT} not found: the fixture is generated in the build container only")
    with tempfile.TemporaryDirectory() as tmp:
        subprocess.run([sys.executable, REF_SCRIPT, "--out", tmp], check=True, stdout=subprocess.DEVNULL)
        d = os.path.join(tmp, "tiny_hybrid")
        tensors = read_safetensors_f32(os.path.join(d, "model.safetensors"))
        cfg = json.load(open(os.path.join(d, "config.json")))["text_config"]
        golden = json.load(open(os.path.join(d, "golden.json")))
    arrays = {}
    for hf, a in tensors.items():
        name = ir_name(hf)
        if name is not None:
            arrays[name] = a.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "tiny_hybrid.npz"), **arrays)
    meta = {
        "source": "reference python/goldens/tiny_hybrid.py (run by tests/golden/make_tiny_hybrid.py)",
        "config": cfg,
        "prompt_ids": golden["prompt_ids"],
        "greedy_ids": golden["greedy_ids"],
        "mtp_draft_ids": golden["mtp_draft_ids"],
    }
    with open(os.path.join(HERE, "tiny_hybrid.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(f"wrote {len(arrays)} tensors; greedy {golden['greedy_ids']} drafts {golden['mtp_draft_ids']}")


if __name__ == "__main__":
    main()
