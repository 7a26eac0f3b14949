"""One engine, every recorded HIP graph in turn: the T=1 decode step, the T=4 MTP
verify (mtp_spec), MTP drafts of 1..3 tokens through the stem and through the MTP
decoder layer, and continuous-batch steps of 2..4 slots, interleaved over several
rounds in a seeded random order.  Each graph is recorded once and replayed later
after the others, so a recording that picked up another's kernels or stale state
shows up as a wrong result: decode and draft results are checked against the oracle
model, batch rows against single-sequence decoding bit for bit."""
import numpy as np
import pytest

from oracle.oracle import OracleModel
from rapidllm_amd import model as M
from rapidllm_amd.engine import MTP_LAYER, MTP_STEM, Engine

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def margin_ok(logits, tol=TOL):
    s = np.sort(logits.astype(np.float64))
    return (s[-1] - s[-2]) > tol * np.linalg.norm(logits)


@pytest.mark.parametrize("seed,quant", [(1, "fp8"), (2, "fp8"), (3, "q4_k")])
def test_interleaved_graph_recordings(gpu, orc, seed, quant):
    spec = M.ModelSpec(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4,
                       n_kv=2, layer_kinds=[0, 0, 0, 1], mtp_layer=True)
    if quant == "fp8":
        W = M.random_weights(spec, seed=40 + seed, w_scale=(1e-3, 1e-2))
    else:
        W = M.random_weights(spec, seed=40 + seed, linear_quant=M.Q_Q4_K, head_quant=M.Q_Q6_K)
    eng = Engine(spec, W, ctx=512, max_T=4, max_batch=4)
    ref = Engine(spec, W, ctx=512)
    om = OracleModel(spec, W, ctx=512)
    rng = np.random.default_rng(seed)
    try:
        for rnd in range(3):
            # single sequence on slot 0
            prompt = [int(t) for t in rng.integers(0, spec.vocab, 3 + rnd)]
            eng.prefill(prompt)
            om.reset()
            for t in prompt:
                g, lg, _ = om.decode(t)
            assert rel_l2(eng.copy_logits(), lg) < TOL
            if margin_ok(lg):
                assert eng.greedy() == g
            g = eng.greedy()
            for op in rng.choice(["decode", "stem", "layer", "spec"], 7):
                if op == "decode":
                    eng.decode_token(g)
                    g2, lg, _ = om.decode(g)
                    assert rel_l2(eng.copy_logits(), lg) < TOL, (rnd, op)
                    if margin_ok(lg):
                        assert eng.greedy() == g2, (rnd, op)
                    g = eng.greedy()
                elif op in ("stem", "layer"):
                    eng.set_mtp_mode(MTP_STEM if op == "stem" else MTP_LAYER)
                    om.set_mtp_mode(0 if op == "stem" else 1)
                    n = int(rng.integers(1, 4))
                    assert eng.mtp_draft(g, n).tolist() == om.mtp_draft(g, n).tolist(), (rnd, op, n)
                else:
                    drafts = om.mtp_draft(g, 3)
                    k, toks, preds = eng.mtp_spec(g, 4)
                    assert toks[0] == g and toks[1:].tolist() == drafts.tolist(), (rnd, op)
                    for t in toks[:k]:
                        g2, lg, _ = om.decode(int(t))
                    assert rel_l2(eng.copy_logits(), lg) < TOL, (rnd, op, k)
                    if margin_ok(lg):
                        assert eng.greedy() == g2, (rnd, op, k)
                    g = eng.greedy()
            # a continuous batch over slots 0 .. B-1
            B = int(rng.integers(2, 5))
            prompts = [[int(t) for t in rng.integers(0, spec.vocab, 2 + b)] for b in range(B)]
            want = []
            for p in prompts:
                ref.prefill(p)
                t0 = ref.greedy()
                ref.decode_token(t0)
                want.append((t0, ref.copy_logits()))
            eng.zero_slots(B)
            for b, p in enumerate(prompts):
                eng.prefill_slot(p, b)
            eng.decode_tokens([w[0] for w in want], [len(p) for p in prompts])
            rows = eng.copy_logits_n(B)
            for b in range(B):
                assert np.array_equal(rows[b], want[b][1]), (rnd, B, b)
    finally:
        eng.close()
        ref.close()
