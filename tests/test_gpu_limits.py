"""Error paths and limits of the engine ABI (the reference's context-full and
bad-argument behaviour: the Session refuses a step past the context; invalid
arguments become RapidError codes, api.h:11-25): every case is checked on the host
before anything is launched, so a refused call leaves the engine usable.  Covered:
an empty or too-long prompt, token ids outside the vocabulary, decoding up to the
last position of the context and one past it, a verify that would cross the end,
batch calls with bad slot counts or positions, and MTP calls for no or too many
drafts."""
import numpy as np
import pytest

from rapidllm_amd import model as M
from rapidllm_amd.engine import Engine
from rapidllm_amd.hip import HipError

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small():
    spec = M.ModelSpec(vocab=1000, hidden=256, n_layers=4, intermediate=512, n_k_heads=2, n_v_heads=4, n_q=4,
                       n_kv=2, layer_kinds=[0, 0, 0, 1])
    W = M.random_weights(spec, seed=77, w_scale=(1e-3, 1e-2))
    eng = Engine(spec, W, ctx=512, max_T=4, max_batch=2)
    yield spec, eng
    eng.close()


def test_prompt_limits(gpu, small):
    spec, eng = small
    cap = eng.ctx_capacity
    with pytest.raises(HipError):
        eng.prefill([])
    with pytest.raises(HipError):
        eng.prefill([1] * (cap + 1))
    with pytest.raises(HipError):
        eng.prefill([1, 2, spec.vocab])  # token id outside the vocabulary
    with pytest.raises(HipError):
        eng.prefill([1, -1, 2])
    eng.prefill([5, 6, 7])  # still usable after the refusals
    assert 0 <= eng.greedy() < spec.vocab
    assert eng.pos() == 3


def test_context_end(gpu, small):
    spec, eng = small
    cap = eng.ctx_capacity
    eng.prefill([3] * (cap - 2))
    assert eng.pos() == cap - 2
    g = eng.greedy()
    with pytest.raises(HipError):
        eng.mtp_spec(g, 4)  # would cross the end of the context
    with pytest.raises(HipError):
        eng.decode_steps(3)
    eng.decode_token(g)
    eng.decode_token(eng.greedy())
    assert eng.pos() == cap
    with pytest.raises(HipError):
        eng.decode_token(eng.greedy())  # context full
    with pytest.raises(HipError):
        eng.spec_verify([eng.greedy(), 1])
    eng.prefill([9, 9])  # a new prompt resets the sequence
    assert eng.pos() == 2


def test_batch_arguments(gpu, small):
    spec, eng = small
    cap = eng.ctx_capacity
    eng.zero_slots(2)
    eng.prefill_slot([1, 2], 0)
    eng.prefill_slot([3, 4, 5], 1)
    with pytest.raises(HipError):
        eng.decode_tokens([1, 2, 3], [2, 3, 4])  # more slots than max_batch
    with pytest.raises(HipError):
        eng.decode_tokens([1, 2], [2, cap])  # a position past the context
    with pytest.raises(HipError):
        eng.prefill_slot([1, 2], 2)  # slot out of range
    eng.decode_tokens([1, 2], [2, 3])
    assert eng.copy_logits_n(2).shape == (2, spec.vocab)
    assert eng.mtp_draft(1, 0).size == 0  # no drafts requested: none made
    with pytest.raises(HipError):
        eng.mtp_draft(1, 8)  # more drafts than the draft cache takes
