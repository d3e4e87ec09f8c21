"""The tiny hybrid model with the tensor types of a Q4_K_M checkpoint on the GPU
(Q6_K embedding = tied head, Q5_K attn_qkv / attn_output on their
fp32-activation form, Q6_K ffn_down / attn_v, Q8_0 ssm_alpha / ssm_beta, Q4_K
elsewhere) against the REFERENCE's own outputs (tests/golden/tiny_kmix_model.npz)
and against the oracle: prefill logits, greedy ids and last logits bit for bit,
every linear in its own type (nm/src/quant_i8.hpp:352-383, 415-495)."""
import numpy as np
import pytest

import hero_amd
import oracle
from gpu_util import bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(kmix_gguf):
    import torch

    assert torch.cuda.is_available()
    m = hero_amd.Qwen35Model.open(kmix_gguf)
    yield m
    m.close()


@pytest.fixture(scope="module")
def cpu(kmix_gguf):
    m = oracle.Model(path=kmix_gguf)
    yield m
    m.close()


def same_bits(got, ref, what):
    bad = np.flatnonzero(bits(got) != bits(ref))
    assert bad.size == 0, f"{what}: {bad.size} of {ref.size} differ, max|d|={np.max(np.abs(got - ref)):.3g}"


def test_kquant_model_matches_reference(model, kmix_golden):
    """16-token prefill (the chunk path), then 32 graph-replayed decode passes"""
    with pytest.raises(hero_amd.HeroError):  # the Q8_0 matvec timing is not for this model
        model.time_gemvs(model.new_state(8))
    state = model.new_state(256)
    lg = model.forward(state, ids=kmix_golden["prompt"])
    same_bits(lg.values, kmix_golden["logits_prefill"], "prefill")
    ids, last = model.decode_greedy(state, lg.argmax(), len(kmix_golden["ids"]) - 1, want_logits=True)
    assert np.array_equal(np.array([lg.argmax()] + [int(i) for i in ids], np.int32), kmix_golden["ids"])
    same_bits(last.values, kmix_golden["logits_last"], "last pass")


def test_kquant_model_single_steps_and_embedding_match_oracle(model, cpu, kmix_golden):
    """forward() one token at a time (the step path without the graph), and
    the Q6_K embedding gather against the oracle's"""
    prompt = kmix_golden["prompt"][:6]
    assert np.array_equal(bits(model.embed(prompt)), bits(cpu.embed(prompt)))
    state = model.new_state(64)
    cpu.reset()
    for t in prompt:
        got = model.forward(state, ids=[int(t)]).values
        ref = cpu.forward_ids([int(t)])
        same_bits(got, ref, f"token {t}")


def test_kquant_model_long_prefill_in_chunks_matches_oracle(kmix_gguf, cpu):
    """1200 tokens through 1024-row chunks (two chunks: the second one's rows
    attend to the first's cache and continue its recurrent state), then a
    decode pass"""
    m = hero_amd.Qwen35Model.open(kmix_gguf)
    try:
        rng = np.random.default_rng(11)
        prompt = rng.integers(0, 32000, 1200).astype(np.int32)
        state = m.new_state(2048)
        got = m.forward(state, ids=prompt).values
        cpu.reset()
        ref = cpu.forward_ids(prompt)
        same_bits(got, ref, "1200-token prefill")
        nxt = int(np.argmax(ref))
        same_bits(m.forward(state, ids=[nxt]).values, cpu.forward_ids([nxt]), "decode after the prefill")
    finally:
        m.close()


def test_kquant_model_batch_decode_matches_single_sequences(model, cpu):
    """three sequences decoded together (every linear over 3 rows, each row
    its own sequence) equal the oracle's separate runs"""
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, 32000, n).astype(np.int32) for n in (5, 9, 2)]
    steps = 6
    bs = model.new_batch_state(64, 3)
    firsts = []
    for i, p in enumerate(prompts):
        firsts.append(model.forward_seq(bs, i, ids=p).argmax())
    out = model.decode_batch(bs, firsts, steps)
    out = np.asarray(out[0] if isinstance(out, tuple) else out).reshape(steps, 3)
    for i, p in enumerate(prompts):
        cpu.reset()
        ids, _ = cpu.greedy(p, steps)[:2]
        assert ids[0] == firsts[i]
        assert np.array_equal(out[:, i], ids[1:]), (i, out[:, i], ids[1:])


def test_q8_ffn_mix_model_matches_reference(q8ffn_gguf, q8ffn_golden):
    """SwiGLU width 3584, wider than every input projection, with Q8_0 gate and
    up (strided outputs through the typed path's scratch) beside K-quant
    tensors: the 20-token prefill, 32 decode passes and a 3-sequence batch
    step equal the reference's golden bit for bit"""
    m = hero_amd.Qwen35Model.open(q8ffn_gguf)
    try:
        state = m.new_state(256)
        lg = m.forward(state, ids=q8ffn_golden["prompt"])
        same_bits(lg.values, q8ffn_golden["logits_prefill"], "prefill")
        ids, last = m.decode_greedy(state, lg.argmax(), len(q8ffn_golden["ids"]) - 1, want_logits=True)
        assert np.array_equal(np.array([lg.argmax()] + [int(i) for i in ids], np.int32), q8ffn_golden["ids"])
        same_bits(last.values, q8ffn_golden["logits_last"], "last pass")
        bs = m.new_batch_state(64, 3)
        firsts = [m.forward_seq(bs, i, ids=q8ffn_golden["prompt"]).argmax() for i in range(3)]
        assert firsts == [int(q8ffn_golden["ids"][0])] * 3
        out = m.decode_batch(bs, firsts, 4)
        out = np.asarray(out[0] if isinstance(out, tuple) else out).reshape(4, 3)
        for i in range(3):
            assert np.array_equal(out[:, i], q8ffn_golden["ids"][1:5]), (i, out[:, i])
    finally:
        m.close()
