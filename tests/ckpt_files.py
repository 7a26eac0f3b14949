"""Writers of small checkpoint files for the loader tests: an HF directory
(config.json + safetensors, optionally sharded with model.safetensors.index.json)
and a GGUF v3 file, both from a WeightTable of IR-named tensors.

The file formats are the public safetensors and GGUF layouts.  Two GGUF naming
styles are written:
  - "plain": the tensor names of tests/fixtures/gguf_qwen36_27b_names.txt in the
    reference (ssm_in / ssm_z / ssm_out, ssm_a.weight = in_proj_a, ssm_a_log = raw
    A_log), MTP as nextn.*;
  - "llama": llama.cpp's qwen35 conversion as the reference's loader expects it
    (src/frontend/weight_store.cpp:27-84, model_desc.h:131-133): attn_qkv /
    attn_gate / ssm_out, ssm_alpha / ssm_beta, ssm_a = -exp(A_log), Qwen RMSNorm
    scales stored raw (1 + gamma), V heads tiled (head r * nk + k holds grouped
    head k * rep + r), the MTP block as blk.<n_layers>.nextn.*.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

from rapidllm_amd import model as M

_ST_DTYPE = {M.Q_F32: "F32", M.Q_F16: "F16", M.Q_BF16: "BF16", M.Q_FP8: "F8_E4M3"}
_GGML = {M.Q_F32: 0, M.Q_F16: 1, M.Q_BF16: 30, M.Q_Q4_K: 12, M.Q_Q6_K: 14, 5: 8, 7: 13}

_HF_LAYER = {
    "attn_norm": "input_layernorm.weight", "ffn_norm": "post_attention_layernorm.weight",
    "attn.wq": "self_attn.q_proj.weight", "attn.wk": "self_attn.k_proj.weight",
    "attn.wv": "self_attn.v_proj.weight", "attn.wo": "self_attn.o_proj.weight",
    "attn.q_norm": "self_attn.q_norm.weight", "attn.k_norm": "self_attn.k_norm.weight",
    "mlp.gate": "mlp.gate_proj.weight", "mlp.up": "mlp.up_proj.weight", "mlp.down": "mlp.down_proj.weight",
    "delta.gemm.in_proj_qkv": "linear_attn.in_proj_qkv.weight", "delta.gemm.in_proj_z": "linear_attn.in_proj_z.weight",
    "delta.gemm.out_proj": "linear_attn.out_proj.weight", "delta.leftover.in_proj_a": "linear_attn.in_proj_a.weight",
    "delta.leftover.in_proj_b": "linear_attn.in_proj_b.weight", "delta.leftover.a_log": "linear_attn.A_log",
    "delta.leftover.dt_bias": "linear_attn.dt_bias", "delta.leftover.conv1d": "linear_attn.conv1d.weight",
    "delta.leftover.norm": "linear_attn.norm.weight",
}
_GG_COMMON = {
    "attn_norm": "attn_norm.weight", "ffn_norm": "ffn_norm.weight", "attn.wq": "attn_q.weight",
    "attn.wk": "attn_k.weight", "attn.wv": "attn_v.weight", "attn.wo": "attn_output.weight",
    "attn.q_norm": "attn_q_norm.weight", "attn.k_norm": "attn_k_norm.weight", "mlp.gate": "ffn_gate.weight",
    "mlp.up": "ffn_up.weight", "mlp.down": "ffn_down.weight", "delta.leftover.conv1d": "ssm_conv1d.weight",
    "delta.leftover.norm": "ssm_norm.weight",
}
_GG_PLAIN = dict(_GG_COMMON, **{
    "delta.gemm.in_proj_qkv": "ssm_in.weight", "delta.gemm.in_proj_z": "ssm_z.weight",
    "delta.gemm.out_proj": "ssm_out.weight", "delta.leftover.in_proj_a": "ssm_a.weight",
    "delta.leftover.in_proj_b": "ssm_beta.weight", "delta.leftover.a_log": "ssm_a_log",
    "delta.leftover.dt_bias": "ssm_dt"})
_GG_LLAMA = dict(_GG_COMMON, **{
    "delta.gemm.in_proj_qkv": "attn_qkv.weight", "delta.gemm.in_proj_z": "attn_gate.weight",
    "delta.gemm.out_proj": "ssm_out.weight", "delta.leftover.in_proj_a": "ssm_alpha.weight",
    "delta.leftover.in_proj_b": "ssm_beta.weight", "delta.leftover.a_log": "ssm_a",
    "delta.leftover.dt_bias": "ssm_dt.bias"})
_MTP_TOP = {"mtp.fc": "fc.weight", "mtp.norm": "norm.weight", "mtp.pre_fc_norm_hidden": "pre_fc_norm_hidden.weight",
            "mtp.pre_fc_norm_embedding": "pre_fc_norm_embedding.weight"}
_NEXTN = {"mtp.fc": "eh_proj.weight", "mtp.norm": "shared_head_norm.weight",
          "mtp.pre_fc_norm_hidden": "hnorm.weight", "mtp.pre_fc_norm_embedding": "enorm.weight"}
# Qwen RMSNorm weights used as (1 + gamma) (weight_store.cpp:30-37)
_RMS_GAMMA = ("attn_norm", "ffn_norm", "final_norm", "mtp.norm", "pre_fc_norm", "q_norm", "k_norm")


def split_layer(ir):
    if ir.startswith("layers["):
        i, rest = ir[7:].split("].", 1)
        return int(i), rest
    return None, ir


def hf_name(ir):
    i, rest = split_layer(ir)
    if i is not None:
        return f"model.language_model.layers.{i}.{_HF_LAYER[rest]}"
    if ir in _MTP_TOP:
        return "mtp." + _MTP_TOP[ir]
    if ir.startswith("mtp.layers["):
        j, rest = ir[11:].split("].", 1)
        return f"mtp.layers.{j}.{_HF_LAYER[rest]}"
    return {"embed": "model.language_model.embed_tokens.weight", "lm_head": "lm_head.weight",
            "final_norm": "model.language_model.norm.weight"}[ir]


def gguf_name(ir, style, n_layers):
    table = _GG_LLAMA if style == "llama" else _GG_PLAIN
    i, rest = split_layer(ir)
    if i is not None:
        return f"blk.{i}.{table[rest]}"
    if ir in _MTP_TOP:
        return f"blk.{n_layers}.nextn.{_NEXTN[ir]}" if style == "llama" else "nextn." + _MTP_TOP[ir]
    if ir.startswith("mtp.layers["):
        j, rest = ir[11:].split("].", 1)
        return f"blk.{n_layers}.{table[rest]}" if style == "llama" else f"nextn.layers.{j}.{_HF_LAYER[rest]}"
    return {"embed": "token_embd.weight", "lm_head": "output.weight", "final_norm": "output_norm.weight"}[ir]


def hf_config(spec: M.ModelSpec, tie=False):
    return {"architectures": ["Qwen3_5ForConditionalGeneration"], "text_config": {
        "hidden_size": spec.hidden, "num_hidden_layers": spec.n_layers, "intermediate_size": spec.intermediate,
        "vocab_size": spec.vocab, "rms_norm_eps": spec.rms_eps,
        "layer_types": ["full_attention" if k == M.LAYER_ATTN else "linear_attention" for k in spec.layer_kinds],
        "linear_num_key_heads": spec.n_k_heads, "linear_num_value_heads": spec.n_v_heads,
        "linear_key_head_dim": spec.k_dim, "linear_value_head_dim": spec.v_dim,
        "linear_conv_kernel_dim": spec.conv_k, "num_attention_heads": spec.n_q,
        "num_key_value_heads": spec.n_kv, "head_dim": spec.head_dim,
        "rope_parameters": {"rope_theta": spec.rope_theta, "partial_rotary_factor": spec.rotary_dim / spec.head_dim},
        "tie_word_embeddings": tie, "mtp_num_hidden_layers": 1}}


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, shape, bytes)."""
    header, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def scale_bytes(scale, dtype):
    s = np.ascontiguousarray(scale, np.float32)
    if dtype == "F32":
        return s.tobytes()
    if dtype == "F16":
        return s.astype(np.float16).tobytes()
    return (s.view(np.uint32) >> 16).astype(np.uint16).tobytes()  # BF16 (truncation)


def write_hf(dirpath, spec: M.ModelSpec, W: M.WeightTable, scale_dtype="F32", shards=1, tie=False, skip=()):
    """HF directory; FP8 linears get `<name>_scale_inv` block scales in scale_dtype.
    1-D / conv tensors in F32 are written as given (BF16 checkpoints: use bf16 WeightTable entries)."""
    os.makedirs(dirpath, exist_ok=True)
    with open(os.path.join(dirpath, "config.json"), "w") as f:
        json.dump(hf_config(spec, tie), f)
    entries = {}
    for ir, (q, rows, cols, data, scale) in W.t.items():
        if ir in skip or (tie and ir == "lm_head"):
            continue
        name = hf_name(ir)
        shape = [rows, cols] if cols > 1 else [rows]
        if ir.endswith("delta.leftover.conv1d"):
            shape = [rows, 1, cols]
        entries[name] = (_ST_DTYPE[q], shape, np.ascontiguousarray(data).tobytes())
        if q == M.Q_FP8:
            entries[name + "_scale_inv"] = (scale_dtype, list(np.shape(scale)) if np.ndim(scale) == 2 else
                                            [(rows + 127) // 128, (cols + 127) // 128], scale_bytes(scale, scale_dtype))
    names = list(entries)
    if shards == 1:
        write_safetensors(os.path.join(dirpath, "model.safetensors"), entries)
        return
    wm = {}
    for s in range(shards):
        fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = {n: entries[n] for n in names[s::shards]}
        write_safetensors(os.path.join(dirpath, fn), part)
        wm.update({n: fn for n in part})
    with open(os.path.join(dirpath, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)


def tile_v_heads(spec: M.ModelSpec, W: M.WeightTable) -> M.WeightTable:
    """The same model with its DeltaNet V heads in llama.cpp's tiled order."""
    nk, nv, dk, dv = spec.n_k_heads, spec.n_v_heads, spec.k_dim, spec.v_dim
    rep = nv // nk
    perm = np.empty(nv, np.int64)  # perm[new] = old
    for k in range(nk):
        for r in range(rep):
            perm[r * nk + k] = k * rep + r
    chan = np.concatenate([np.arange(2 * nk * dk)] + [2 * nk * dk + perm[h] * dv + np.arange(dv) for h in range(nv)])
    rows_dv = np.concatenate([perm[h] * dv + np.arange(dv) for h in range(nv)])
    out = M.WeightTable()
    for ir, (q, rows, cols, data, scale) in W.t.items():
        a = data
        if ".delta." in ir:
            # rows of K-quant tensors are independent block rows; FP8 tiles are not
            assert q != M.Q_FP8, "tile_v_heads: FP8 block scales span 128 rows"
            if q in (M.Q_Q4_K, M.Q_Q6_K):
                assert not ir.endswith("out_proj"), "tile_v_heads: K-quant columns cannot be permuted"
                a = np.asarray(data).reshape(rows, -1)
            else:
                a = np.asarray(data).reshape(rows, cols) if cols > 1 else np.asarray(data).reshape(rows)
            if ir.endswith(("in_proj_qkv", "conv1d")):
                a = a[chan]
            elif ir.endswith("in_proj_z"):
                a = a[rows_dv]
            elif ir.endswith(("in_proj_a", "in_proj_b", "a_log", "dt_bias")):
                a = a[perm]
            elif ir.endswith("out_proj"):
                a = a[:, rows_dv]
        out.add(ir, q, np.ascontiguousarray(a), rows, cols, scale)
    return out


def _gguf_str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, value):
    out = _gguf_str(key)
    if isinstance(value, str):
        return out + struct.pack("<I", 8) + _gguf_str(value)
    if isinstance(value, float):
        return out + struct.pack("<If", 6, value)
    if isinstance(value, list):  # array of strings
        out += struct.pack("<IIQ", 9, 8, len(value))
        return out + b"".join(_gguf_str(v) for v in value)
    return out + struct.pack("<II", 4, value)


def write_gguf(path, spec: M.ModelSpec, W: M.WeightTable, style="llama", arch="qwen35", hparams=True,
               extra_tensors=(), skip=(), version=3, quant_override=None):
    """GGUF v3.  style "llama" applies llama.cpp's conventions (see module doc);
    quant_override: ir -> (ggml_type, raw bytes[, ggml dims]) replaces a tensor's stored form."""
    L = spec.n_layers
    if style == "llama":
        W = tile_v_heads(spec, W)
    kvs = [("general.architecture", arch), ("general.name", "loader-test"),
           ("tokenizer.ggml.tokens", ["a", "b", "c"])]
    if hparams:
        kvs += [(f"{arch}.block_count", L + (1 if style == "llama" and spec.has_mtp else 0)),
                (f"{arch}.embedding_length", spec.hidden), (f"{arch}.feed_forward_length", spec.intermediate),
                (f"{arch}.attention.head_count", spec.n_q), (f"{arch}.attention.head_count_kv", spec.n_kv),
                (f"{arch}.attention.key_length", spec.head_dim),
                (f"{arch}.attention.layer_norm_rms_epsilon", float(spec.rms_eps)),
                (f"{arch}.rope.freq_base", float(spec.rope_theta)), (f"{arch}.rope.dimension_count", spec.rotary_dim),
                (f"{arch}.ssm.conv_kernel", spec.conv_k), (f"{arch}.ssm.state_size", spec.k_dim),
                (f"{arch}.ssm.group_count", spec.n_k_heads), (f"{arch}.ssm.time_step_rank", spec.n_v_heads),
                (f"{arch}.ssm.inner_size", spec.n_v_heads * spec.v_dim)]
        if style == "llama" and spec.has_mtp:
            kvs.append((f"{arch}.nextn_predict_layers", 1))
    tensors = []
    for ir, (q, rows, cols, data, scale) in W.t.items():
        if ir in skip:
            continue
        name = gguf_name(ir, style, L)
        a = np.ascontiguousarray(data)
        ggml = _GGML[q]
        if style == "llama" and q == M.Q_F32:
            f = np.asarray(a, np.float32).reshape(-1)
            if ir.endswith("delta.leftover.a_log"):
                a = (-np.exp(f.astype(np.float64))).astype(np.float32)
            elif any(k in ir for k in _RMS_GAMMA) and "leftover.norm" not in ir:
                a = (f + np.float32(1.0)).astype(np.float32)
        dims = [cols, rows] if cols > 1 else [rows]
        if quant_override and ir in quant_override:
            ggml, raw = quant_override[ir][:2]
            dims = list(quant_override[ir][2]) if len(quant_override[ir]) > 2 else dims
        else:
            raw = np.ascontiguousarray(a).tobytes()
        tensors.append((name, dims, ggml, raw))
    tensors += list(extra_tensors)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(_kv(k, v) for k, v in kvs)
    info, blob = b"", b""
    for name, dims, ggml, raw in tensors:
        blob += b"\0" * (-len(blob) % 32)
        info += _gguf_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        info += struct.pack("<IQ", ggml, len(blob))
        blob += raw
    data = head + info
    data += b"\0" * (-len(data) % 32)
    with open(path, "wb") as f:
        f.write(data + blob)
