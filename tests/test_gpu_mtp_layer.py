"""The MTP decoder-layer draft mode (RL_MTP_LAYER): the stem's fc output passes
through mtp.layers[0] -- gated attention over the layer's own fp16 KV cache at
draft positions 0, 1, ... of the call, then the MLP -- before the final MTP norm
and the lm_head (Session::mtp_layer_step, session.cpp:561-617; the reference's
CUDA engine drafts through that layer for official checkpoints,
cuda_engine.cu:16304-16357).  Checked against the oracle model's mtp_draft in
mode 1 (itself pinned to the reference's fused_attn_decode / fused_mlp_decode in
test_oracle_kernels.py) on FP8 and K-quant models, for 1..7 drafts, inside the
one-submission mtp_spec, and for the greedy invariant."""
import numpy as np
import pytest

from oracle.oracle import OracleModel
from rapidllm_amd import model as M
from rapidllm_amd.engine import MTP_LAYER, MTP_STEM, Engine
from rapidllm_amd.hip import HipError

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def mini_spec(**kw):
    base = dict(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4, n_kv=2,
                layer_kinds=[0, 0, 0, 1], mtp_layer=True)
    base.update(kw)
    return M.ModelSpec(**base)


def run_prompt(eng, om, prompt):
    eng.prefill(prompt)
    om.reset()
    for t in prompt:
        g, lg, _ = om.decode(t)
    return g


@pytest.mark.parametrize("quant", ["fp8", "q4_k"])
def test_mtp_layer_drafts_match_oracle(gpu, orc, quant):
    spec = mini_spec()
    if quant == "fp8":
        W = M.random_weights(spec, seed=31, w_scale=(1e-3, 1e-2))
    else:
        W = M.random_weights(spec, seed=32, linear_quant=M.Q_Q4_K, head_quant=M.Q_Q6_K)
    eng = Engine(spec, W, ctx=512)
    om = OracleModel(spec, W, ctx=512)
    try:
        assert eng.mtp_mode() == (MTP_STEM, True)
        g = run_prompt(eng, om, [4, 8, 15, 16, 23, 42])
        assert eng.greedy() == g
        eng.set_mtp_mode(MTP_LAYER)
        om.set_mtp_mode(1)
        for n in (1, 3, 7):
            got = eng.mtp_draft(g, n)
            want = om.mtp_draft(g, n)
            assert rel_l2(eng.copy_mtp_hidden(), om.mtp_hidden()) < TOL, n
            assert got.tolist() == want.tolist(), n
        # a second call starts from an empty draft cache again
        assert eng.mtp_draft(g, 3).tolist() == om.mtp_draft(g, 3).tolist()
        # inside the one-submission draft + verify
        k, toks, preds = eng.mtp_spec(g, 4)
        assert toks[1:].tolist() == om.mtp_draft(g, 3).tolist()
        # greedy invariant with layer drafts
        off, _, _ = eng.generate([9, 9, 1], 14, spec_n=0)
        on, prop, acc = eng.generate([9, 9, 1], 14, spec_n=3)
        assert on == off
        ref_on, _, _ = om.generate([9, 9, 1], 14, spec_n=3)
        assert ref_on == off
    finally:
        eng.close()


def test_mtp_layer_mode_needs_the_layer(gpu, orc):
    spec = mini_spec(mtp_layer=False)
    W = M.random_weights(spec, seed=33, w_scale=(1e-3, 1e-2))
    eng = Engine(spec, W, ctx=512)
    try:
        assert eng.mtp_mode() == (MTP_STEM, False)
        with pytest.raises(HipError):
            eng.set_mtp_mode(MTP_LAYER)
        eng.set_mtp_mode(MTP_STEM)
    finally:
        eng.close()


def test_mtp_layer_drafts_and_batch_steps_keep_their_own_graphs(gpu, orc):
    """An engine with batch slots and the MTP decoder layer records a 3-draft call
    and a 3-slot batch step as two different HIP graphs: each replays its own
    kernels, in either order (drafts against the oracle, batch rows bit-identical
    to single-sequence decoding)."""
    spec = mini_spec()
    W = M.random_weights(spec, seed=34, w_scale=(1e-3, 1e-2))
    eng = Engine(spec, W, ctx=512, max_batch=4)
    ref = Engine(spec, W, ctx=512)
    om = OracleModel(spec, W, ctx=512)
    prompts = [[1, 2, 3], [7, 7], [5, 9, 11, 2]]

    def plain(p):
        ref.prefill(p)
        t0 = ref.greedy()
        ref.decode_token(t0)
        return t0, ref.copy_logits()

    def batch_step():
        eng.zero_slots(3)
        toks, poss, want = [], [], []
        for b, p in enumerate(prompts):
            eng.prefill_slot(p, b)
            t0, lg = plain(p)
            toks.append(t0)
            poss.append(len(p))
            want.append(lg)
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(3)
        for b in range(3):
            assert np.array_equal(rows[b], want[b]), b

    def drafts():
        g = run_prompt(eng, om, [4, 8, 15, 16])
        assert eng.mtp_draft(g, 3).tolist() == om.mtp_draft(g, 3).tolist()

    try:
        eng.set_mtp_mode(MTP_LAYER)
        om.set_mtp_mode(1)
        drafts()
        batch_step()
        drafts()
        batch_step()
    finally:
        eng.close()
        ref.close()
