"""GPU parity of the whole decode engine against the CPU oracle model on small
models of the real architecture (head dims 128/256, FP8 or K-quant linears):
logits within 1e-3 relative L2, identical greedy tokens where the top-1 margin
exceeds that tolerance, MTP stem drafts, the greedy invariant (spec == spec off)
and speculative rollback."""
import numpy as np
import pytest

from oracle.oracle import OracleModel
from rapidllm_amd import model as M
from rapidllm_amd.engine import Engine

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


def margin_ok(logits, tol=TOL):
    s = np.sort(logits.astype(np.float64))
    return (s[-1] - s[-2]) > tol * np.linalg.norm(logits)


@pytest.fixture(scope="module")
def fp8_pair(orc):
    spec = mini_spec()
    W = M.random_weights(spec, seed=3, w_scale=(1e-3, 1e-2))
    return spec, W, Engine(spec, W, ctx=1024), OracleModel(spec, W, ctx=1024)


def test_decode_logits_match_oracle(gpu, fp8_pair):
    spec, W, eng, orc_m = fp8_pair
    prompt = [1, 2, 3, 4, 5, 6, 7]
    eng.prefill(prompt)
    orc_m.reset()
    for t in prompt:
        g, lg, hd = orc_m.decode(t)
    assert rel_l2(eng.copy_logits(), lg) < TOL
    assert rel_l2(eng.copy_last_hidden(), hd) < TOL
    if margin_ok(lg):
        assert eng.greedy() == g
    tok = g
    for _ in range(6):
        eng.decode_token(tok)
        g, lg, _ = orc_m.decode(tok)
        assert rel_l2(eng.copy_logits(), lg) < TOL
        if margin_ok(lg):
            assert eng.greedy() == g
        tok = g


def test_greedy_generate_matches_oracle(gpu, fp8_pair):
    spec, W, eng, orc_m = fp8_pair
    prompt = [5, 9, 13]
    want, _, _ = orc_m.generate(prompt, 12)
    got, _, _ = eng.generate(prompt, 12)
    assert got == want


def test_mtp_draft_matches_oracle(gpu, fp8_pair):
    spec, W, eng, orc_m = fp8_pair
    prompt = [7, 8, 9, 10, 11]
    eng.prefill(prompt)
    orc_m.reset()
    for t in prompt:
        g, _, _ = orc_m.decode(t)
    assert eng.greedy() == g
    assert eng.mtp_draft(g, 3).tolist() == orc_m.mtp_draft(g, 3).tolist()


def test_spec_invariant_and_oracle_spec(gpu, fp8_pair):
    """Greedy invariant (tests/test_spec.cpp:46-79): MTP speculation changes speed,
    never tokens; GPU T=4 verify == GPU T=1 decode == CPU oracle with MTP."""
    spec, W, eng, orc_m = fp8_pair
    prompt = [3, 1, 4, 1, 5]
    off, _, _ = eng.generate(prompt, 16, spec_n=0)
    on, prop, acc = eng.generate(prompt, 16, spec_n=3)
    assert on == off
    ref_on, rprop, racc = orc_m.generate(prompt, 16, spec_n=3)
    assert ref_on == off
    assert acc == racc


def test_spec_verify_rollback(gpu, fp8_pair):
    """A rejected draft leaves the state exactly as the accepted prefix: after
    verifying [t0, d1, wrong, x] the next logits equal a T=1 replay."""
    spec, W, eng, orc_m = fp8_pair
    prompt = [2, 4, 6]
    eng.prefill(prompt)
    t0 = eng.greedy()
    eng.decode_token(t0)
    d1 = eng.greedy()
    ref_logits = eng.copy_logits()
    eng.prefill(prompt)
    wrong = (d1 + 1) % spec.vocab
    k, preds = eng.spec_verify([t0, d1, wrong, 17])
    assert preds[0] == d1
    assert k == (3 if preds[1] == wrong else 2)
    if k == 2:
        # state = after [prompt, t0, d1]; compare with a plain T=1 run
        eng2_logits = eng.copy_logits()
        eng.prefill(prompt)
        eng.decode_token(t0)
        eng.decode_token(d1)
        assert np.array_equal(eng.copy_logits(), eng2_logits)
        assert eng.pos() == len(prompt) + 2
    del ref_logits


@pytest.fixture(scope="module")
def q4k_pair(orc):
    spec = mini_spec()
    W = M.random_weights(spec, seed=5, linear_quant=M.Q_Q4_K)
    return spec, W, Engine(spec, W, ctx=1024), OracleModel(spec, W, ctx=1024)


@pytest.mark.parametrize("pair", ["fp8_pair", "q4k_pair"])
@pytest.mark.parametrize("n_ok", [1, 2, 3, 4])
def test_spec_verify_then_decode_matches_plain_decode(gpu, request, pair, n_ok):
    """After a verify that consumes n_ok of 4 tokens, the following steps see the
    recurrent state after exactly those tokens: two more T=1 steps and another
    verify give the logits of plain T=1 decoding, bit for bit.  Block-FP8 and Q4_K
    models (the latter with the K-quant folded norms, the DeltaNet a/b rows as
    K-slices and the fused DeltaNet kernel's records)."""
    spec, W, eng, orc_m = request.getfixturevalue(pair)
    prompt = [3, 1, 4, 1, 5]
    eng.prefill(prompt)
    chain = [eng.greedy()]
    for _ in range(7):
        eng.decode_token(chain[-1])
        chain.append(eng.greedy())
    # plain decoding of chain[0 .. n_ok + 3], logits after each token
    eng.prefill(prompt)
    plain = []
    for t in chain[: n_ok + 4]:
        eng.decode_token(t)
        plain.append(eng.copy_logits())
    # verify [chain[0], .., chain[n_ok - 1], wrong ...]: exactly n_ok consumed
    eng.prefill(prompt)
    toks = chain[:n_ok] + [(chain[n_ok] + 1) % spec.vocab] * (4 - n_ok)
    k, preds = eng.spec_verify(toks[:4])
    assert k == n_ok and list(preds[:k]) == chain[1 : k + 1]
    assert eng.pos() == len(prompt) + n_ok
    eng.decode_token(chain[n_ok])
    assert np.array_equal(eng.copy_logits(), plain[n_ok])
    eng.decode_token(chain[n_ok + 1])
    assert np.array_equal(eng.copy_logits(), plain[n_ok + 1])
    # a second verify after the replayed records: its first row again
    k2, preds2 = eng.spec_verify([chain[n_ok + 2], (chain[n_ok + 3] + 1) % spec.vocab])
    assert k2 == 1 and preds2[0] == chain[n_ok + 3]
    assert np.array_equal(eng.copy_logits(), plain[n_ok + 2])


def test_wide_delta_in_proj_slices_match_oracle(gpu, orc):
    """27B DeltaNet head counts (16 k-heads, 48 v-heads) on a narrow model: the fused
    in_proj has 16480 rows, past two workgroups per CU, so its a/b rows are computed
    as K-slice partials that the DeltaNet kernel sums.  Prefill, decode and a
    partly rejected verify match the oracle and plain decoding."""
    spec = mini_spec(n_k_heads=16, n_v_heads=48, n_layers=4, layer_kinds=[0, 0, 0, 1])
    W = M.random_weights(spec, seed=21, w_scale=(1e-3, 1e-2))
    eng, orc_m = Engine(spec, W, ctx=512), OracleModel(spec, W, ctx=512)
    prompt = [5, 9, 2, 7, 1]
    eng.prefill(prompt)
    orc_m.reset()
    for t in prompt:
        g, lg, _ = orc_m.decode(t)
    assert rel_l2(eng.copy_logits(), lg) < TOL
    chain = []
    tok = g
    for _ in range(4):
        eng.decode_token(tok)
        g, lg, _ = orc_m.decode(tok)
        assert rel_l2(eng.copy_logits(), lg) < TOL
        chain.append((tok, eng.copy_logits()))
        tok = g
    # verify consuming 2 of 4, then plain decode equality
    eng.prefill(prompt)
    t0 = chain[0][0]
    toks = [t0, chain[1][0], (chain[2][0] + 1) % spec.vocab, 3]
    k, preds = eng.spec_verify(toks)
    if preds[0] == chain[1][0] and preds[1] != toks[2]:
        assert k == 2
        eng.decode_token(chain[2][0])
        assert np.array_equal(eng.copy_logits(), chain[2][1])
    eng.close()


@pytest.mark.parametrize("quant", [M.Q_Q4_K, M.Q_Q6_K, M.Q_BF16])
def test_other_weight_formats_match_oracle(gpu, orc, quant):
    spec = mini_spec(n_layers=4, layer_kinds=[0, 1, 0, 0])
    W = M.random_weights(spec, seed=11, linear_quant=quant)
    eng = Engine(spec, W, ctx=512)
    orc_m = OracleModel(spec, W, ctx=512)
    prompt = [10, 20, 30, 40, 50]
    eng.prefill(prompt)
    for t in prompt:
        g, lg, _ = orc_m.decode(t)
    assert rel_l2(eng.copy_logits(), lg) < TOL
    for _ in range(3):
        eng.decode_token(g)
        g, lg, _ = orc_m.decode(g)
        assert rel_l2(eng.copy_logits(), lg) < TOL


@pytest.mark.parametrize("quant", [None, M.Q_Q4_K, M.Q_Q6_K])
def test_norm_kernels_and_folded_norm_agree(gpu, orc, monkeypatch, quant):
    """The step with RMSNorm folded into the GEMMs (the default: FP8 / BF16 models
    fold it into the GEMM epilogues and prologues, K-quant models into the residual
    GEMVs' final write and the next GEMVs' x fragments) and the step with separate
    norm kernels (RL_FOLD_NORM=0) both match the oracle on the same model, at T=1
    and in a T=4 verify."""
    spec = mini_spec()
    if quant is None:
        W = M.random_weights(spec, seed=11, w_scale=(1e-3, 1e-2))
    else:
        W = M.random_weights(spec, seed=11, linear_quant=quant)
    orc_m = OracleModel(spec, W, ctx=512)
    prompt = [3, 1, 4, 1, 5, 9, 2]
    orc_m.reset()
    for t in prompt:
        g, lg, _ = orc_m.decode(t)
    outs = []
    for fold in ("1", "0"):
        monkeypatch.setenv("RL_FOLD_NORM", fold)
        eng = Engine(spec, W, ctx=512)
        eng.prefill(prompt)
        assert rel_l2(eng.copy_logits(), lg) < TOL, fold
        if margin_ok(lg):
            assert eng.greedy() == g
        toks = [g, 7, 8, 9]
        n, preds = eng.spec_verify(toks)
        outs.append((eng.copy_logits(), list(preds[:n]), n))
        eng.close()
    assert outs[0][1:] == outs[1][1:]
    assert rel_l2(outs[0][0], outs[1][0]) < TOL


def test_long_prefill_chunks_match_oracle_and_decode(gpu, fp8_pair):
    """A prompt of many max_T chunks (uploaded once, chunks fed on the device):
    logits equal the oracle's and equal a token-by-token decode of the same prompt,
    and a decode after the prefill continues correctly."""
    spec, W, eng, orc_m = fp8_pair
    rng = np.random.default_rng(99)
    prompt = [int(t) for t in rng.integers(0, spec.vocab, 41)]
    eng.prefill(prompt)
    lg_prefill = eng.copy_logits()
    orc_m.reset()
    for t in prompt:
        g, lg, _ = orc_m.decode(t)
    assert rel_l2(lg_prefill, lg) < TOL
    eng.prefill(prompt[:1])
    for t in prompt[1:]:
        eng.decode_token(t)
    assert rel_l2(eng.copy_logits(), lg_prefill) < TOL
    eng.prefill(prompt)
    eng.decode_token(g)
    g2, lg2, _ = orc_m.decode(g)
    assert rel_l2(eng.copy_logits(), lg2) < TOL


def test_mixed_kquant_types_within_projections(gpu, orc):
    """A Q4_K_M-style table: Q4_K linears with Q6_K parts inside fused projections
    (DeltaNet z beside Q4_K q|k|v, attention v beside Q4_K q|gate and k, MLP up
    beside a Q4_K gate, the way llama.cpp mixes attn_v / ffn_down types), so each
    type boundary splits a projection into groups and gate/up take the
    separate-launch path.  Logits match the oracle at T=1 and after a T=4 verify."""
    spec = mini_spec(n_layers=4, layer_kinds=[0, 1, 0, 0])
    W = M.random_weights(spec, seed=13, linear_quant=M.Q_Q4_K)
    r = np.random.default_rng(5)
    from rapidllm_amd import synth

    g = synth.rng(17)
    for name, (q, rows, cols, data, s) in list(W.t.items()):
        if name.endswith(("delta.gemm.in_proj_z", "attn.wv", "mlp.up")) or (
                name.endswith("mlp.down") and "layers[2]" in name):
            W.add(name, M.Q_Q6_K, synth.q6k_blocks(g, rows, cols), rows, cols)
    eng = Engine(spec, W, ctx=512)
    orc_m = OracleModel(spec, W, ctx=512)
    prompt = [int(t) for t in r.integers(0, spec.vocab, 6)]
    eng.prefill(prompt)
    for t in prompt:
        gt, lg, _ = orc_m.decode(t)
    assert rel_l2(eng.copy_logits(), lg) < TOL
    for _ in range(2):
        eng.decode_token(gt)
        gt, lg, _ = orc_m.decode(gt)
        assert rel_l2(eng.copy_logits(), lg) < TOL
    toks = [gt, 5, 6, 7]
    k, preds = eng.spec_verify(toks)
    want = []
    for i, t in enumerate(toks):
        gg, lg, _ = orc_m.decode(t)
        want.append((gg, lg))
        if i + 1 < len(toks) and gg != toks[i + 1]:
            break
    assert k == len(want)
    assert rel_l2(eng.copy_logits(), want[-1][1]) < TOL
    eng.close()
