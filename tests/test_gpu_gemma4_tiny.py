"""The Gemma 4 text model at small width (hero_amd.gemma4.GEMMA4_TINY: 12
layers, full attention on layers 5 and 11, the last 4 reusing the K/V of
layers 7 and 5, a 64-position window, d_model 512, vocabulary 4096) on the
GPU against the oracle's restatement of the reference (oracle.Gemma4, pinned
by the reference's E4B goldens in test_gpu_gemma4.py).

Prompts run past the window (the rings wrap, the K/V-sharing layers read
windows of another layer's ring), states smaller than the window, and the
error paths. Bar: logits bit-identical, greedy ids equal."""
import os
import tempfile

import numpy as np
import pytest

from hero_amd import ContextExhausted, HeroError

pytestmark = pytest.mark.gpu

SEED = 77


@pytest.fixture(scope="module")
def paths():
    from hero_amd.gemma4 import GEMMA4_TINY, write_synthetic_gemma4

    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "gemma4_tiny.gguf")
        write_synthetic_gemma4(path, GEMMA4_TINY, seed=SEED)
        yield path


@pytest.fixture(scope="module")
def model(paths):
    from hero_amd.gemma4 import Gemma4Model

    m = Gemma4Model.open(paths)
    yield m
    m.close()


@pytest.fixture(scope="module")
def ref(paths):
    import oracle

    oracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    r = oracle.Gemma4(path=paths)
    yield r
    r.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# (1100, ...) and (3900, ...): the full-attention layers' softmax totals over
# 1024 or more keys (the exact parallel sum) and over more keys than one
# shared-memory chunk holds (3840: the scores re-read chunk by chunk)
@pytest.mark.timeout(600)
@pytest.mark.parametrize("prompt_len,steps,max_tokens", [(100, 20, 256), (30, 8, 40), (1, 70, 128), (1100, 4, 1200), (3900, 4, 4096)])
def test_tiny_gemma4_matches_oracle(model, ref, prompt_len, steps, max_tokens):
    rng = np.random.default_rng(prompt_len)
    prompt = rng.integers(0, model.V, prompt_len).astype(np.int32)
    state = model.new_state(max_tokens)
    logits = model.forward(state, prompt)
    ref.reset()
    want = ref.forward(prompt)
    assert np.array_equal(bits(logits.values), bits(want)), f"prefill logits differ: max |d| {np.abs(logits.values - want).max():.3g}"
    first = logits.argmax()
    ids, last = model.decode_greedy(state, first, steps, want_logits=True)
    got = [first]
    for _ in range(steps):
        lg = ref.forward([got[-1]])
        got.append(int(np.argmax(lg)))
    assert [int(i) for i in ids] == got[1:]
    assert np.array_equal(bits(last.values), bits(lg))
    assert state.tokens() == prompt_len + steps


def test_tiny_gemma4_forward_in_pieces_equals_one_forward(model):
    """T ids in one call, in pieces, or as greedy passes: the same logits (every
    row attends over the same visible keys)."""
    prompt = np.random.default_rng(3).integers(0, model.V, 90).astype(np.int32)
    a = model.new_state(128)
    whole = model.forward(a, prompt)
    b = model.new_state(128)
    for i in range(0, 90, 37):
        part = model.forward(b, prompt[i:i + 37])
    assert np.array_equal(bits(whole.values), bits(part.values))
    a.reset()
    again = model.forward(a, prompt)
    assert np.array_equal(bits(whole.values), bits(again.values))


def test_tiny_gemma4_errors(model):
    state = model.new_state(16)
    model.forward(state, [1, 2, 3])
    with pytest.raises(ContextExhausted):
        model.forward(state, list(range(20)))
    assert state.tokens() == 3  # rejected before anything ran (the reference's length_error)
    with pytest.raises(HeroError):
        model.forward(state, [model.V])
    with pytest.raises(HeroError):
        model.new_state(model.CTX + 1)
    e = model.embed([5, 6])
    assert e.shape == (2, model.D) and np.isfinite(e).all()
