"""Checkpoint loading (rl_hip_weights_*, host code over the C ABI; no GPU).

Model: the reference's tests/test_loader.cpp (name-map cases, HF and GGUF loads,
rejection of a FP8 tensor without weight_scale_inv, of a bad GGUF and of a
quantised DeltaNet leftover).  Pinned three ways:
  - files written here from the tiny-hybrid golden fixture load back into a table
    on which the oracle model reproduces the reference golden script's greedy
    tokens and MTP drafts (HF, GGUF with plain names, GGUF with llama.cpp's
    conventions: raw RMSNorm scales, ssm_a = -exp(A_log), tiled V heads);
  - conversions against their definitions (scale dtypes, F16/BF16 -> F32,
    K-quant / Q8_0 dequantisation of leftovers);
  - where oracle/_ref is built, the reference's own loaders (src/frontend/*.cpp,
    WeightStore::open) on the same files: same names, sources, kinds, shapes,
    bytes and scales, same model description.
"""
import os

import numpy as np
import pytest

from rapidllm_amd import hip
from rapidllm_amd import model as M
from rapidllm_amd import synth
from rapidllm_amd.loader import SOURCE_GGUF, SOURCE_HF, Checkpoint, map_name
from tests import ckpt_files as F


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(hip.LIB_PATH):
        pytest.skip("library not built")
    return hip.lib()


@pytest.fixture(scope="module")
def tiny():
    from tests.tiny_hybrid import load

    return load()


def mini_spec(**kw):
    base = dict(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4, n_kv=2,
                layer_kinds=[0, 0, 0, 1])
    base.update(kw)
    return M.ModelSpec(**base)


def f16_to_f32(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------------ name maps
def test_map_names_reference_cases(L):
    """tests/test_loader.cpp:40-50 (GGUF); vision tensors are not part of the path."""
    cases = {
        "blk.64.nextn.eh_proj.weight": "mtp.fc",
        "blk.64.nextn.enorm.weight": "mtp.pre_fc_norm_embedding",
        "blk.64.nextn.hnorm.weight": "mtp.pre_fc_norm_hidden",
        "blk.64.nextn.shared_head_norm.weight": "mtp.norm",
        "blk.64.nextn.attn_q.weight": "mtp.layers[0].attn.wq",
        "nextn.fc.weight": "mtp.fc",
        "blk.0.attn_q.weight": "layers[0].attn.wq",
        "blk.0.ssm_a": "layers[0].delta.leftover.a_log",
        "blk.0.ssm_a_log": "layers[0].delta.leftover.a_log",
        "blk.0.ssm_a.weight": "layers[0].delta.leftover.in_proj_a",
        "blk.0.ssm_alpha.weight": "layers[0].delta.leftover.in_proj_a",
    }
    for src, ir in cases.items():
        assert map_name(src, gguf=True) == ir, src
    assert map_name("model.language_model.layers.7.linear_attn.A_log") == "layers[7].delta.leftover.a_log"
    assert map_name("mtp.layers.0.mlp.down_proj.weight") == "mtp.layers[0].mlp.down"
    assert map_name("model.visual.blocks.0.attn.qkv.weight") == ""
    assert map_name("blk.3.unknown.weight", gguf=True) == ""


def _all_names():
    spec = mini_spec()
    W = M.random_weights(spec, seed=1, linear_quant=M.Q_BF16)
    irs = list(W.t) + ["mtp.layers[0].attn.wq", "mtp.layers[0].mlp.up"]
    hf = [F.hf_name(n) for n in irs] + ["model.embed_tokens.weight", "model.norm.weight",
                                          "model.layers.2.linear_attn.in_proj_qkvz.weight",
                                          "model.layers.2.linear_attn.in_proj_ba.weight", "foo.bar"]
    gg = [F.gguf_name(n, s, 4) for n in irs for s in ("llama", "plain")]
    fixture = ["token_embd.weight", "output.weight", "output_norm.weight"] + [
        f"blk.{i}.{t}" for i in (0, 63) for t in (
            "attn_norm.weight", "ffn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
            "attn_output.weight", "attn_q_norm.weight", "attn_k_norm.weight", "ffn_gate.weight", "ffn_up.weight",
            "ffn_down.weight", "ssm_in.weight", "ssm_z.weight", "ssm_out.weight", "ssm_a.weight", "ssm_beta.weight",
            "ssm_a_log", "ssm_dt", "ssm_conv1d.weight", "ssm_norm.weight", "post_attention_norm.weight",
            "attn_o.weight", "ssm_dt.bias", "shortconv.weight", "in_proj_qkv.weight", "nextn.eh_proj")]
    return hf, gg + fixture


def test_map_names_agree_with_reference_loader(L, ref_lib):
    import ctypes as C

    hf, gg = _all_names()
    buf = C.create_string_buffer(512)
    for gguf, names in ((0, hf), (1, gg)):
        for n in names:
            ref_lib.ref_map_name(gguf, n.encode(), buf, 512)
            assert map_name(n, gguf=bool(gguf)) == buf.value.decode(), n


# ------------------------------------------------------------------ golden model through files
def _golden_check(spec, W, meta, orc):
    from oracle.oracle import OracleModel

    m = OracleModel(spec, W, ctx=64, kv_fp16=False, threads=1)
    got, _, _ = m.generate(meta["prompt_ids"], len(meta["greedy_ids"]))
    assert got == meta["greedy_ids"]
    m.reset()
    for t in meta["prompt_ids"]:
        g, _, _ = m.decode(t)
    assert m.mtp_draft(g, 3).tolist() == meta["mtp_draft_ids"]


def _same_spec(a: M.ModelSpec, b: M.ModelSpec, skip=()):
    for f in ("vocab", "hidden", "n_layers", "intermediate", "n_k_heads", "n_v_heads", "k_dim", "v_dim", "conv_k",
              "n_q", "n_kv", "head_dim", "rotary_dim", "has_mtp"):
        if f not in skip:
            assert getattr(a, f) == getattr(b, f), f
    assert abs(a.rope_theta - b.rope_theta) <= 1e-3 * b.rope_theta
    assert a.layer_kinds == b.layer_kinds


def test_tiny_hybrid_hf_dir_reproduces_golden(L, orc, tiny, tmp_path):
    spec, W, meta = tiny
    F.write_hf(tmp_path / "hf", spec, W)
    with Checkpoint(tmp_path / "hf") as ck:
        assert ck.source == SOURCE_HF and not ck.spec.v_tiled
        _same_spec(ck.spec, spec)
        assert sorted(ck.names()) == sorted(W.t)
        for name, (q, rows, cols, data, _) in W.t.items():
            q2, r2, c2, d2, _ = ck.get(name)
            assert (q2, r2, c2) == (q, rows, cols), name
            assert np.array_equal(d2, np.asarray(data, np.float32).reshape(-1)), name
        assert ck.info("layers[0].delta.leftover.conv1d")["shape"] == (80, 1, 4)
        _golden_check(ck.spec, ck, meta, orc)


def test_tiny_hybrid_gguf_plain_names(L, orc, tiny, tmp_path):
    spec, W, meta = tiny
    F.write_gguf(tmp_path / "t.gguf", spec, W, style="plain", hparams=False)
    with Checkpoint(tmp_path / "t.gguf") as ck:
        # no hyper-parameters in the file: the 8-layer test hybrid's description
        # (src/ir/model_desc.cpp:77-110)
        assert ck.source == SOURCE_GGUF and not ck.spec.v_tiled
        _same_spec(ck.spec, spec)
        for name, (q, rows, cols, data, _) in W.t.items():
            assert np.array_equal(ck.get(name)[3], np.asarray(data, np.float32).reshape(-1)), name
        _golden_check(ck.spec, ck, meta, orc)


def test_tiny_hybrid_gguf_llama_conventions(L, orc, tiny, tmp_path):
    """Raw (1 + gamma) RMSNorm scales, ssm_a = -exp(A_log) and tiled V heads come
    back as the engine's convention with v_tiled set; the model's output is the
    golden one."""
    spec, W, meta = tiny
    F.write_gguf(tmp_path / "t.gguf", spec, W, style="llama")
    with Checkpoint(tmp_path / "t.gguf") as ck:
        assert ck.spec.v_tiled and ck.spec.has_mtp and ck.spec.n_layers == 8
        _same_spec(ck.spec, spec)
        assert ck.info("layers[0].delta.leftover.a_log")["src_name"] == "blk.0.ssm_a"
        g = np.asarray(W.t["layers[0].attn_norm"][3], np.float32)
        assert np.allclose(ck.get("layers[0].attn_norm")[3], g, rtol=0, atol=2e-7)
        assert np.array_equal(ck.get("layers[0].delta.leftover.norm")[3], W.t["layers[0].delta.leftover.norm"][3])
        Wt = F.tile_v_heads(spec, W)
        a = np.asarray(Wt.t["layers[1].delta.leftover.a_log"][3], np.float32)
        assert np.allclose(ck.get("layers[1].delta.leftover.a_log")[3], a, rtol=1e-6, atol=1e-7)
        _golden_check(ck.spec, ck, meta, orc)


# ------------------------------------------------------------------ conversions
def test_fp8_scale_dtypes_and_bf16_leftovers(L, tmp_path):
    spec = mini_spec()
    W = M.random_weights(spec, seed=5, w_scale=(1e-3, 1e-2))
    # a BF16 checkpoint's norms / A_log / conv: materialised as F32
    Wb = M.WeightTable()
    for name, (q, rows, cols, data, scale) in W.t.items():
        if q == M.Q_F32 and name != "embed":
            Wb.add(name, M.Q_BF16, synth.bf16_bits(np.asarray(data, np.float32)), rows, cols)
        else:
            Wb.add(name, q, data, rows, cols, scale)
    for sdt in ("F32", "BF16", "F16"):
        d = tmp_path / sdt
        F.write_hf(d, spec, Wb, scale_dtype=sdt)
        with Checkpoint(d) as ck:
            q, rows, cols, data, scale = ck.get("layers[0].mlp.down")
            assert q == M.Q_FP8 and (rows, cols) == (256, 512)
            assert np.array_equal(data, W.t["layers[0].mlp.down"][3].reshape(-1))
            want = W.t["layers[0].mlp.down"][4].reshape(-1)
            if sdt == "BF16":
                want = synth.bf16_to_f32((want.view(np.uint32) >> 16).astype(np.uint16))
            elif sdt == "F16":
                want = want.astype(np.float16).astype(np.float32)
            assert np.array_equal(scale, want)
            qn, _, _, n, _ = ck.get("layers[0].attn_norm")
            assert qn == M.Q_F32
            assert np.array_equal(n, synth.bf16_to_f32(Wb.t["layers[0].attn_norm"][3]))
            qc, rc, cc, _, _ = ck.get("layers[0].delta.leftover.conv1d")
            assert (qc, rc, cc) == (M.Q_F32, spec.conv_dim, 4)
            assert ck.get("embed")[0] == M.Q_BF16  # embedding / linears stay as stored


def test_sharded_index_tied_head_and_max_layers(L, tmp_path):
    spec = mini_spec()
    W = M.random_weights(spec, seed=6, w_scale=(1e-3, 1e-2))
    F.write_hf(tmp_path / "s", spec, W, shards=3, tie=True)
    assert (tmp_path / "s" / "model.safetensors.index.json").exists()
    with Checkpoint(tmp_path / "s") as ck:
        assert np.array_equal(ck.get("lm_head")[3], ck.get("embed")[3])
        assert ck.info("lm_head")["src_name"].startswith("tied:")
        assert len(ck.names()) == len(W.t)
    with Checkpoint(tmp_path / "s", max_layers=2) as ck:
        assert ck.spec.n_layers == 2
        assert not any(n.startswith(("layers[2]", "layers[3]")) for n in ck.names())


def _q8_0_blocks(r, m, n):
    blk = np.empty((m * n // 32, 34), np.uint8)
    blk[:, 0:2] = r.uniform(1e-3, 1e-2, len(blk)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = r.integers(0, 256, (len(blk), 32), dtype=np.uint8)
    return blk.reshape(m, -1)


def _q5_k_blocks(r, m, n):
    blk = np.empty((m * n // 256, 176), np.uint8)
    blk[:, 0:2] = r.uniform(1e-4, 1e-2, len(blk)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = r.uniform(1e-4, 1e-2, len(blk)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blk[:, 4:] = r.integers(0, 256, (len(blk), 172), dtype=np.uint8)
    return blk.reshape(m, -1)


def test_quantised_leftovers_dequantised(L, orc, tmp_path):
    """GGUF in_proj_a / in_proj_b as Q8_0 / Q5_K / Q4_K / Q6_K become F32 by the
    block formats' definitions (Q4_K / Q6_K against the oracle's dequantisers)."""
    spec = mini_spec()
    W = M.random_weights(spec, seed=7, linear_quant=M.Q_BF16)
    r = synth.rng(8)
    nv, H = spec.n_v_heads, spec.hidden
    blocks = {"layers[0].delta.leftover.in_proj_a": (8, _q8_0_blocks(r, nv, H)),
              "layers[0].delta.leftover.in_proj_b": (13, _q5_k_blocks(r, nv, H)),
              "layers[1].delta.leftover.in_proj_a": (12, synth.q4k_blocks(r, nv, H)),
              "layers[1].delta.leftover.in_proj_b": (14, synth.q6k_blocks(r, nv, H))}
    F.write_gguf(tmp_path / "q.gguf", spec, W, style="plain",
                 quant_override={k: (t, b.tobytes()) for k, (t, b) in blocks.items()})
    with Checkpoint(tmp_path / "q.gguf") as ck:
        for name, (t, b) in blocks.items():
            q, rows, cols, data, _ = ck.get(name)
            assert (q, rows, cols) == (M.Q_F32, nv, H), name
            assert ck.info(name)["gguf_type"] == t
            raw = b.reshape(-1)
            if t == 8:
                blk = raw.reshape(-1, 34)
                d = f16_to_f32(blk[:, 0:2].copy().view(np.uint16).reshape(-1))
                want = (d[:, None] * blk[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)
            elif t == 13:
                blk = raw.reshape(-1, 176)
                d = f16_to_f32(blk[:, 0:2].copy().view(np.uint16).reshape(-1))
                dm = f16_to_f32(blk[:, 2:4].copy().view(np.uint16).reshape(-1))
                want = np.empty((len(blk), 256), np.float32)
                for i in range(len(blk)):
                    sc, qh, ql = blk[i, 4:16], blk[i, 16:48], blk[i, 48:176]
                    for c in range(4):
                        for h in range(2):
                            j = 2 * c + h
                            if j < 4:
                                s, m = sc[j] & 63, sc[j + 4] & 63
                            else:
                                s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)
                                m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
                            nib = (ql[32 * c:32 * c + 32] >> (4 * h)) & 0xF
                            hb = (qh >> j) & 1
                            qv = (nib.astype(np.int32) + 16 * hb).astype(np.float32)
                            want[i, 64 * c + 32 * h:64 * c + 32 * h + 32] = \
                                np.float32(d[i] * np.float32(s)) * qv - np.float32(dm[i] * np.float32(m))
                want = want.reshape(-1)
            elif t == 12:
                want = orc.dequant_q4_k(raw, nv * H)
            else:
                want = orc.dequant_q6_k(raw, nv * H)
            assert np.array_equal(data, np.asarray(want, np.float32).reshape(-1)), name


# ------------------------------------------------------------------ rejections
def _status(path):
    with pytest.raises(hip.HipError) as e:
        Checkpoint(path)
    return e.value.code, str(e.value)


def test_rejections(L, tmp_path):
    spec = mini_spec()
    W = M.random_weights(spec, seed=9, w_scale=(1e-3, 1e-2))
    # FP8 tensor without weight_scale_inv (bad_fp8)
    d = tmp_path / "bad_fp8"
    F.write_hf(d, spec, W)
    t = {}
    for name, (q, rows, cols, data, scale) in W.t.items():
        shape = [rows, 1, cols] if name.endswith("conv1d") else ([rows, cols] if cols > 1 else [rows])
        t[F.hf_name(name)] = ({M.Q_F32: "F32", M.Q_BF16: "BF16", M.Q_FP8: "F8_E4M3"}[q], shape,
                              np.ascontiguousarray(data).tobytes())
    F.write_safetensors(d / "model.safetensors", t)
    code, msg = _status(d)
    assert code == 2 and "weight_scale_inv" in msg
    # bad GGUF: wrong magic, truncated
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 64)
    assert _status(p)[0] == 2
    F.write_gguf(tmp_path / "ok.gguf", spec, M.random_weights(spec, seed=9, linear_quant=M.Q_BF16))
    full = (tmp_path / "ok.gguf").read_bytes()
    (tmp_path / "trunc.gguf").write_bytes(full[: len(full) - 1000])
    code, msg = _status(tmp_path / "trunc.gguf")
    assert code == 2 and "truncated" in msg
    # quantised DeltaNet leftover that must stay uncompressed (bad_leftover)
    Wq = M.random_weights(spec, seed=9, linear_quant=M.Q_BF16)
    r = synth.rng(3)
    F.write_gguf(tmp_path / "left.gguf", spec, Wq, style="plain",
                 quant_override={"layers[0].delta.leftover.a_log": (12, synth.q4k_blocks(r, 1, 256).tobytes(), [256])})
    code, msg = _status(tmp_path / "left.gguf")
    assert "leftover" in msg
    # paths
    assert _status(tmp_path / "nothing.bin")[0] == 1
    (tmp_path / "empty_dir").mkdir()
    assert _status(tmp_path / "empty_dir")[0] == 1


# ------------------------------------------------------------------ against the reference loaders
def _ref_table(R, path):
    import ctypes as C

    err = C.create_string_buffer(512)
    h = R.ref_weights_open(str(path).encode(), err, 512)
    assert h, err.value
    out = {}
    try:
        for i in range(R.ref_weights_count(h)):
            shp = (C.c_int64 * 4)()
            nd = R.ref_weights_shape(h, i, shp)
            nb = R.ref_weights_nbytes(h, i)
            data = C.string_at(R.ref_weights_data(h, i), nb) if nb else b""
            ns = R.ref_weights_nscale(h, i)
            sc = np.frombuffer(C.string_at(R.ref_weights_scale(h, i), 4 * ns), np.float32) if ns else None
            out[R.ref_weights_name(h, i).decode()] = dict(src=R.ref_weights_src(h, i).decode(),
                                                          quant=R.ref_weights_quant(h, i), shape=tuple(shp[:nd]),
                                                          data=data, scale=sc)
        m = (C.c_int * 8)()
        kinds = (C.c_ubyte * 256)()
        R.ref_weights_model(h, m, kinds)
        model = dict(n_layers=m[0], hidden=m[1], vocab=m[2], intermediate=m[3], v_tiled=m[4], has_mtp=m[5],
                     source=m[6], kinds=list(kinds[: m[0]]))
    finally:
        R.ref_weights_close(h)
    return out, model


def _compare_with_reference(R, path, ck):
    want, model = _ref_table(R, path)
    assert sorted(want) == sorted(ck.names())
    for name, w in want.items():
        q, rows, cols, data, scale = ck.get(name)
        inf = ck.info(name)
        assert inf["src_name"] == w["src"], name
        assert q == w["quant"], name
        assert inf["shape"] == w["shape"], name
        assert data.tobytes() == w["data"], name
        if w["scale"] is None:
            assert scale is None, name
        else:
            assert np.array_equal(scale, w["scale"]), name
    s = ck.spec
    assert (s.n_layers, s.hidden, s.vocab, int(s.v_tiled), int(s.has_mtp), ck.source) == (
        model["n_layers"], model["hidden"], model["vocab"], model["v_tiled"], model["has_mtp"], model["source"])
    assert s.layer_kinds == model["kinds"]
    return model


def test_tables_match_reference_loader(L, ref_lib, tiny, tmp_path):
    spec, W, _ = tiny
    F.write_hf(tmp_path / "hf", spec, W, shards=2)
    F.write_gguf(tmp_path / "llama.gguf", spec, W, style="llama")
    F.write_gguf(tmp_path / "plain.gguf", spec, W, style="plain", hparams=False)
    for p in ("hf", "llama.gguf", "plain.gguf"):
        with Checkpoint(tmp_path / p) as ck:
            model = _compare_with_reference(ref_lib, tmp_path / p, ck)
            assert model["intermediate"] == ck.spec.intermediate
    # FP8 with BF16 / F16 scales, BF16 leftovers, a tied head
    mspec = mini_spec()
    Wm = M.random_weights(mspec, seed=12, w_scale=(1e-3, 1e-2))
    Wb = M.WeightTable()
    for name, (q, rows, cols, data, scale) in Wm.t.items():
        if q == M.Q_F32:
            Wb.add(name, M.Q_BF16, synth.bf16_bits(np.asarray(data, np.float32)), rows, cols)
        else:
            Wb.add(name, q, data, rows, cols, scale)
    for sdt in ("BF16", "F16"):
        F.write_hf(tmp_path / sdt, mspec, Wb, scale_dtype=sdt, tie=(sdt == "F16"))
        with Checkpoint(tmp_path / sdt) as ck:
            _compare_with_reference(ref_lib, tmp_path / sdt, ck)
    # GGUF K-quant linears with quantised leftovers (dequantised by both loaders)
    Wk = M.random_weights(mspec, seed=13, linear_quant=M.Q_Q4_K)
    r = synth.rng(14)
    nv, H = mspec.n_v_heads, mspec.hidden
    ov = {"layers[0].delta.leftover.in_proj_a": (8, _q8_0_blocks(r, nv, H).tobytes()),
          "layers[0].delta.leftover.in_proj_b": (13, _q5_k_blocks(r, nv, H).tobytes()),
          "layers[1].delta.leftover.in_proj_a": (12, synth.q4k_blocks(r, nv, H).tobytes()),
          "layers[1].delta.leftover.in_proj_b": (14, synth.q6k_blocks(r, nv, H).tobytes())}
    F.write_gguf(tmp_path / "k.gguf", mspec, Wk, style="plain", quant_override=ov)
    with Checkpoint(tmp_path / "k.gguf") as ck:
        _compare_with_reference(ref_lib, tmp_path / "k.gguf", ck)
