"""Continuous batch decode (cuda_engine.h:46-66, Session::generate_batch,
src/runtime/session.cpp:832-964): B sequences in B slots, one weight pass per
step.  Every row of the batched linears and every slot's DeltaNet / attention runs
the same arithmetic as a single-sequence T=1 step, so each slot's logits equal
plain decoding of that sequence bit for bit."""
import numpy as np
import pytest

from oracle.oracle import OracleModel
from rapidllm_amd import model as M
from rapidllm_amd.engine import Engine

pytestmark = pytest.mark.gpu


def mini_spec(**kw):
    base = dict(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4, n_kv=2,
                layer_kinds=[0, 0, 0, 1])
    base.update(kw)
    return M.ModelSpec(**base)


TOL = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def margin_ok(logits, tol=TOL):
    s = np.sort(logits.astype(np.float64))
    return (s[-1] - s[-2]) > tol * np.linalg.norm(logits)


def plain_chain(eng, prompt, n):
    """greedy tokens and logits of single-sequence decoding (slot 0)."""
    eng.prefill(prompt)
    toks, logits = [eng.greedy()], [eng.copy_logits()]
    for _ in range(n - 1):
        eng.decode_token(toks[-1])
        toks.append(eng.greedy())
        logits.append(eng.copy_logits())
    return toks, logits


@pytest.fixture(scope="module")
def batch_pair():
    spec = mini_spec()
    W = M.random_weights(spec, seed=31, w_scale=(1e-3, 1e-2))
    return spec, Engine(spec, W, ctx=512, max_batch=4), Engine(spec, W, ctx=512)


@pytest.mark.parametrize("B", [2, 3, 4])
def test_batch_decode_equals_plain_decode(gpu, batch_pair, B):
    spec, eng, ref = batch_pair
    assert eng.max_batch() == 4
    rng = np.random.default_rng(B)
    prompts = [[int(t) for t in rng.integers(0, spec.vocab, 3 + 2 * b)] for b in range(B)]
    n = 5
    want = [plain_chain(ref, p, n) for p in prompts]
    # prefill each slot, then n-1 batched steps, comparing every step's rows
    toks, poss = [], []
    for b, p in enumerate(prompts):
        eng.prefill_slot(p, b)
        assert np.array_equal(eng.copy_logits(), want[b][1][0])
        toks.append(want[b][0][0])
        poss.append(len(p))
    for step in range(1, n):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(B)
        greedy = eng.copy_greedy_n(B)
        for b in range(B):
            assert np.array_equal(rows[b], want[b][1][step]), (B, step, b)
            assert greedy[b] == want[b][0][step]
        toks = greedy
        poss = [p + 1 for p in poss]


def test_replicate_slot0_and_generate_batch(gpu, batch_pair):
    spec, eng, ref = batch_pair
    prompt = [7, 3, 9, 1, 4, 4]
    toks, _ = plain_chain(ref, prompt, 6)
    eng.prefill(prompt)
    eng.replicate_slot0(3)
    t = [toks[0]] * 3
    poss = [len(prompt)] * 3
    for step in range(1, 6):
        eng.decode_tokens(t, poss)
        g = eng.copy_greedy_n(3)
        assert g == [toks[step]] * 3
        t, poss = g, [p + 1 for p in poss]
    # distinct prompts through the Session-style driver
    prompts = [[5, 6, 7], [1, 2, 3, 4, 5, 6, 7, 8], [9]]
    outs = eng.generate_batch(prompts, 4)
    for b, p in enumerate(prompts):
        assert outs[b] == plain_chain(ref, p, 4)[0]


def test_zero_slots_and_prefill_slot_isolation(gpu, batch_pair):
    spec, eng, ref = batch_pair
    eng.zero_slots(4)
    a, b = [2, 8, 5], [11, 13, 17, 19]
    eng.prefill_slot(a, 0)
    eng.prefill_slot(b, 1)  # must not touch slot 0
    ta, la = plain_chain(ref, a, 3)
    tb, lb = plain_chain(ref, b, 3)
    eng.decode_tokens([ta[0], tb[0]], [len(a), len(b)])
    rows = eng.copy_logits_n(2)
    assert np.array_equal(rows[0], la[1]) and np.array_equal(rows[1], lb[1])


def test_batch_decode_wide_in_proj(gpu):
    """27B DeltaNet head counts: the in_proj's a/b rows come as K-slice partials with
    B rows; each slot still equals plain decoding bit for bit."""
    spec = mini_spec(n_k_heads=16, n_v_heads=48)
    W = M.random_weights(spec, seed=41, w_scale=(1e-3, 1e-2))
    eng, ref = Engine(spec, W, ctx=512, max_batch=2), Engine(spec, W, ctx=512)
    prompts = [[3, 5, 7, 9], [2, 4]]
    want = [plain_chain(ref, p, 3) for p in prompts]
    for b, p in enumerate(prompts):
        eng.prefill_slot(p, b)
    toks, poss = [w[0][0] for w in want], [len(p) for p in prompts]
    for step in range(1, 3):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(2)
        for b in range(2):
            assert np.array_equal(rows[b], want[b][1][step]), (step, b)
        toks, poss = eng.copy_greedy_n(2), [p + 1 for p in poss]
    eng.close()
    ref.close()


def test_long_prompts_prefilled_into_slots(gpu, batch_pair):
    """Prompts long enough for the chunked prefill path, prefilled into slots 1 and
    0 (the chunked path works on the selected slot's caches and state only); batched
    decoding then equals plain decoding of each sequence bit for bit."""
    spec, eng, ref = batch_pair
    eng.zero_slots(4)
    rng = np.random.default_rng(77)
    a = [int(t) for t in rng.integers(0, spec.vocab, 100)]
    b = [int(t) for t in rng.integers(0, spec.vocab, 61)]
    ta, la = plain_chain(ref, a, 4)
    tb, lb = plain_chain(ref, b, 4)
    eng.prefill_slot(b, 1)
    eng.prefill_slot(a, 0)
    assert np.array_equal(eng.copy_logits(), la[0])
    toks, poss = [ta[0], tb[0]], [len(a), len(b)]
    for step in range(1, 4):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(2)
        assert np.array_equal(rows[0], la[step]) and np.array_equal(rows[1], lb[step]), step
        toks, poss = eng.copy_greedy_n(2), [p + 1 for p in poss]


@pytest.mark.parametrize("B", [2, 3, 4])
def test_batch_decode_vs_oracle(gpu, orc, B):
    """Each slot of the batch step against its own oracle model (the reference CPU
    Session decoding that sequence alone, session.cpp:325-411): logits within 1e-3
    relative L2 and identical greedy tokens where the top-1 margin exceeds that,
    with different prompts, lengths and positions per slot (27B DeltaNet head
    counts, so the wide in_proj path runs with B rows)."""
    spec = mini_spec(n_k_heads=16, n_v_heads=48)
    W = M.random_weights(spec, seed=50 + B, w_scale=(1e-3, 1e-2))
    eng = Engine(spec, W, ctx=512, max_batch=4)
    rng = np.random.default_rng(60 + B)
    prompts = [[int(t) for t in rng.integers(0, spec.vocab, 2 + 3 * b)] for b in range(B)]
    oms = [OracleModel(spec, W, ctx=512) for _ in range(B)]
    toks, poss = [], []
    for b, p in enumerate(prompts):
        eng.prefill_slot(p, b)
        for t in p:
            g, lg, _ = oms[b].decode(t)
        assert rel_l2(eng.copy_logits(), lg) < TOL
        toks.append(g)
        poss.append(len(p))
    for step in range(4):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(B)
        greedy = eng.copy_greedy_n(B)
        for b in range(B):
            g, lg, _ = oms[b].decode(toks[b])
            assert rel_l2(rows[b], lg) < TOL, (B, step, b, rel_l2(rows[b], lg))
            if margin_ok(lg):
                assert greedy[b] == g, (B, step, b)
            toks[b] = g  # follow the oracle's chain
        poss = [p + 1 for p in poss]
    eng.close()


KQ_CASES = [([0, 0, 0, 1], M.Q_Q4_K, 2), ([0, 1], M.Q_Q6_K, 4), ([1, 1], M.Q_Q4_K, 3), ([0, 0], M.Q_Q4_K, 4),
            ([0, 0, 0, 1], M.Q_Q4_K, 8), ([0, 1], M.Q_Q6_K, 6)]


@pytest.mark.parametrize("kinds,quant,B", KQ_CASES)
def test_kquant_batch_decode_vs_oracle(gpu, orc, kinds, quant, B):
    """Batch decode of a K-quant (GGUF Q4_K / Q6_K) model: each slot against its own
    oracle model (session.cpp:325-411) with different prompts and positions, and
    every slot's logits equal to single-sequence decoding of that sequence bit for
    bit (the K-quant GEMV quantises each row's x on its own and sums the split-K
    slices in a fixed order, whatever the row count)."""
    spec = mini_spec(n_layers=len(kinds), layer_kinds=kinds)
    W = M.random_weights(spec, seed=70 + B, linear_quant=quant, w_scale=(1e-3, 1e-2))
    eng = Engine(spec, W, ctx=512, max_batch=max(4, B))
    ref = Engine(spec, W, ctx=512)
    rng = np.random.default_rng(80 + B)
    prompts = [[int(t) for t in rng.integers(0, spec.vocab, 2 + 3 * b)] for b in range(B)]
    oms = [OracleModel(spec, W, ctx=512) for _ in range(B)]
    n = 4
    want = [plain_chain(ref, p, n + 1) for p in prompts]
    toks, poss = [], []
    for b, p in enumerate(prompts):
        eng.prefill_slot(p, b)
        for t in p:
            g, lg, _ = oms[b].decode(t)
        assert rel_l2(eng.copy_logits(), lg) < TOL
        toks.append(want[b][0][0])
        poss.append(len(p))
    for step in range(1, n + 1):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(B)
        greedy = eng.copy_greedy_n(B)
        for b in range(B):
            assert np.array_equal(rows[b], want[b][1][step]), (kinds, B, step, b)
            assert greedy[b] == want[b][0][step]
            g, lg, _ = oms[b].decode(toks[b])
            assert rel_l2(rows[b], lg) < TOL, (kinds, B, step, b, rel_l2(rows[b], lg))
            if margin_ok(lg):
                assert greedy[b] == g, (kinds, B, step, b)
        toks = greedy
        poss = [p + 1 for p in poss]
    eng.close()
    ref.close()


@pytest.mark.parametrize("kinds,quant,B", [([1, 1], M.Q_Q4_K, 6), ([0, 1], M.Q_Q6_K, 5), ([1, 1], M.Q_Q4_K, 11),
                                           ([0, 0, 0, 1], M.Q_Q4_K, 16), ([0, 0, 0, 1], None, 12),
                                           ([0, 0, 0, 1], None, 16), ([0, 1], None, 9)])
def test_batch_slot_groups(gpu, kinds, quant, B):
    """More slots than one batch step's rows (the K-quant GEMV takes 8): decode_tokens
    runs the slots in groups, one weight pass each; FP8 / BF16 steps take up to 16
    rows in one pass.  Every slot's logits equal single-sequence decoding of its
    sequence bit for bit (the reference allows up to min(ctx, 128) slots,
    cuda_engine.cu:20057-20062)."""
    spec = mini_spec(n_layers=len(kinds), layer_kinds=kinds)
    if quant is None:
        W = M.random_weights(spec, seed=12, w_scale=(1e-3, 1e-2))
    else:
        W = M.random_weights(spec, seed=9, linear_quant=quant, head_quant=M.Q_Q6_K)
    eng = Engine(spec, W, ctx=256, max_batch=16)
    ref = Engine(spec, W, ctx=256)
    assert eng.max_batch() == 16
    rng = np.random.default_rng(B)
    prompts = [[int(t) for t in rng.integers(0, spec.vocab, 2 + b % 5)] for b in range(B)]
    want = [plain_chain(ref, p, 3) for p in prompts]
    eng.zero_slots(B)
    toks, poss = [], []
    for b, p in enumerate(prompts):
        eng.prefill_slot(p, b)
        toks.append(want[b][0][0])
        poss.append(len(p))
    for step in range(1, 3):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(B)
        greedy = eng.copy_greedy_n(B)
        for b in range(B):
            assert np.array_equal(rows[b], want[b][1][step]), (B, step, b)
            assert greedy[b] == want[b][0][step]
        toks, poss = greedy, [p + 1 for p in poss]
    eng.close()
    ref.close()


def test_batch_attention_across_chunk_boundaries(gpu, batch_pair):
    """Slots whose positions straddle the attention's 256-position chunks (one slot
    crossing 255 -> 256 during the steps, one starting in the second chunk, one at
    position 1): the one attention launch set over all slots reads each slot's own
    position, cache and workspace, so every row equals plain decoding bit for bit."""
    spec, eng, ref = batch_pair
    eng.zero_slots(4)
    rng = np.random.default_rng(91)
    lens = [253, 1, 256, 40]
    prompts = [[int(t) for t in rng.integers(0, spec.vocab, n)] for n in lens]
    n = 5
    want = [plain_chain(ref, p, n) for p in prompts]
    for b, p in enumerate(prompts):
        eng.prefill_slot(p, b)
    toks, poss = [w[0][0] for w in want], list(lens)
    for step in range(1, n):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(4)
        for b in range(4):
            assert np.array_equal(rows[b], want[b][1][step]), (step, b, poss[b])
        toks, poss = eng.copy_greedy_n(4), [p + 1 for p in poss]


@pytest.mark.parametrize("quant", [M.Q_Q4_K, M.Q_Q6_K])
def test_kquant_batch_then_speculative_on_one_engine(gpu, quant):
    """A K-quant engine alternating between batch and single-sequence work: slot 0
    replicated into 3 slots and decoded as a batch, Session-style generate_batch with
    distinct prompts, then speculative (MTP, spec_n = 3) generation on slot 0.  Every
    token equals plain greedy decoding on a separate single-slot engine, so the batch
    steps leave no state behind that the verify's rollback reads."""
    spec = mini_spec()
    W = M.random_weights(spec, seed=123, linear_quant=quant, w_scale=(1e-3, 1e-2))
    eng, ref = Engine(spec, W, ctx=512, max_batch=4), Engine(spec, W, ctx=512)
    prompt = [7, 3, 9, 1, 4, 4]
    toks, _ = plain_chain(ref, prompt, 6)
    eng.prefill(prompt)
    eng.replicate_slot0(3)
    t, poss = [toks[0]] * 3, [len(prompt)] * 3
    for step in range(1, 6):
        eng.decode_tokens(t, poss)
        g = eng.copy_greedy_n(3)
        assert g == [toks[step]] * 3, step
        t, poss = g, [p + 1 for p in poss]
    prompts = [[5, 6, 7], [1, 2, 3, 4, 5, 6, 7, 8], [9]]
    outs = eng.generate_batch(prompts, 4)
    for b, p in enumerate(prompts):
        assert outs[b] == plain_chain(ref, p, 4)[0], b
    plain, _, _ = ref.generate(prompt, 12, spec_n=0)
    on, prop, acc = eng.generate(prompt, 12, spec_n=3)
    assert on == plain and prop > 0
    eng.close()
    ref.close()


@pytest.mark.parametrize("T,B", [(3, 4), (9, 2), (300, 3)])
def test_prefill_eq_batch_vs_oracle(gpu, orc, T, B):
    """Engine::prefill_eq_batch (cuda_engine.h:66-68, called by
    Session::generate_batch for equal-length prompts after zero_slots,
    session.cpp:882-893): each slot's last-token logits and greedy token against its
    own oracle model, then batch decode steps continue from position T.  T <= B
    runs T batch steps; T > B each sequence's chunked prefill."""
    spec = mini_spec()
    W = M.random_weights(spec, seed=70 + T, w_scale=(1e-3, 1e-2))
    eng = Engine(spec, W, ctx=512, max_batch=4)
    rng = np.random.default_rng(T * 10 + B)
    prompts = [[int(t) for t in rng.integers(0, spec.vocab, T)] for _ in range(B)]
    oms = [OracleModel(spec, W, ctx=512) for _ in range(B)]
    want = []
    for b in range(B):
        for t in prompts[b]:
            g, lg, _ = oms[b].decode(t)
        want.append((g, lg))
    eng.decode_token(5)  # slot 0 holds another sequence before the reset
    eng.zero_slots(B)
    eng.prefill_eq_batch(prompts)
    rows = eng.copy_logits_n(B)
    greedy = eng.copy_greedy_n(B)
    toks = []
    for b in range(B):
        g, lg = want[b]
        assert rel_l2(rows[b], lg) < TOL, (b, rel_l2(rows[b], lg))
        if margin_ok(lg):
            assert greedy[b] == g, b
        toks.append(g)
    poss = [T] * B
    for step in range(2):
        eng.decode_tokens(toks, poss)
        rows = eng.copy_logits_n(B)
        for b in range(B):
            g, lg, _ = oms[b].decode(toks[b])
            assert rel_l2(rows[b], lg) < TOL, (step, b)
            toks[b] = g
        poss = [p + 1 for p in poss]
    eng.close()
