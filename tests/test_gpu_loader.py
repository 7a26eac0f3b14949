"""Engines created from checkpoint files (rl_hip_weights_open -> rl_hip_engine_create):
an HF FP8 directory gives the same logits, bit for bit, as the engine created from
the in-memory table the file was written from; a GGUF file in llama.cpp's qwen35
conventions (K-quant linears and embedding, raw RMSNorm scales, ssm_a = -exp(A_log), tiled V
heads) matches the CPU oracle model run on the loaded table, and the untiled
model's greedy tokens."""
import numpy as np
import pytest

from oracle.oracle import OracleModel
from rapidllm_amd import model as M
from rapidllm_amd.engine import Engine
from rapidllm_amd.loader import Checkpoint
from tests import ckpt_files as F

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def mini_spec(**kw):
    base = dict(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4, n_kv=2,
                layer_kinds=[0, 0, 0, 1])
    base.update(kw)
    return M.ModelSpec(**base)


def test_hf_fp8_checkpoint_equals_in_memory_table(gpu, orc, tmp_path):
    spec = mini_spec()
    W = M.random_weights(spec, seed=3, w_scale=(1e-3, 1e-2))
    F.write_hf(tmp_path / "hf", spec, W, shards=2)
    prompt = [1, 2, 3, 4, 5, 6, 7]
    with Checkpoint(tmp_path / "hf") as ck:
        a = Engine(ck.spec, ck, ctx=512)
        b = Engine(spec, W, ctx=512)
        a.prefill(prompt)
        b.prefill(prompt)
        assert np.array_equal(a.copy_logits(), b.copy_logits())
        for _ in range(3):
            t = a.greedy()
            a.decode_token(t)
            b.decode_token(t)
            assert np.array_equal(a.copy_logits(), b.copy_logits())
        o = OracleModel(ck.spec, ck, ctx=512)
        for t in prompt:
            _, lg, _ = o.decode(t)
        a.prefill(prompt)
        assert rel_l2(a.copy_logits(), lg) < TOL
        a.close()
        b.close()


def test_gguf_llama_checkpoint_matches_oracle(gpu, orc, tmp_path):
    spec = mini_spec(n_layers=4, layer_kinds=[0, 1, 0, 0])
    W = M.random_weights(spec, seed=11, linear_quant=M.Q_Q4_K, head_quant=M.Q_Q6_K)
    r = np.random.default_rng(5)
    # GGUF token_embd as Q4_K: the engine dequantises it to an F32 table
    W.add("embed", M.Q_Q4_K, M.synth.q4k_blocks(r, spec.vocab, spec.hidden), spec.vocab, spec.hidden)
    for i, k in enumerate(spec.layer_kinds):
        if k == M.LAYER_DELTA:  # out_proj columns are permuted by the V-head tiling: keep it BF16
            n = f"layers[{i}].delta.gemm.out_proj"
            W.add(n, M.Q_BF16, M.synth.bf16_bits((r.standard_normal((spec.hidden, 512)) * 0.02).astype(np.float32)),
                  spec.hidden, 512)
    F.write_gguf(tmp_path / "m.gguf", spec, W, style="llama")
    prompt = [10, 20, 30, 40, 50]
    with Checkpoint(tmp_path / "m.gguf") as ck:
        assert ck.spec.v_tiled and ck.spec.intermediate == spec.intermediate
        eng = Engine(ck.spec, ck, ctx=512)
        orc_m = OracleModel(ck.spec, ck, ctx=512)
        eng.prefill(prompt)
        for t in prompt:
            g, lg, _ = orc_m.decode(t)
        assert rel_l2(eng.copy_logits(), lg) < TOL
        for _ in range(3):
            eng.decode_token(g)
            g, lg, _ = orc_m.decode(g)
            assert rel_l2(eng.copy_logits(), lg) < TOL
        # the same model in HF head order, gammas as written
        ref = Engine(spec, W, ctx=512)
        ref.prefill(prompt)
        eng.prefill(prompt)
        assert rel_l2(eng.copy_logits(), ref.copy_logits()) < TOL
        got, _, _ = eng.generate(prompt, 8)
        want, _, _ = ref.generate(prompt, 8)
        assert got == want
        eng.close()
        ref.close()
