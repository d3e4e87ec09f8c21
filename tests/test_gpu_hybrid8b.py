"""The ~8B Q8_0 hybrid (32 layers: 24 gated delta-net + 8 GQA every 4th layer;
d_model 4096, 32 q / 8 kv heads of 128, delta-net 32 heads of 128, SwiGLU
12288, vocab 151936) against the oracle on the same model bytes, the way the
reference's check tool drives it (tools/qwen35_check.cpp:43-70): prefill a
prompt, then feed each greedy id back in.

The prompt is 600 tokens long: it prefills as one chunk of 600 rows, whose
delta-net in-projection and gate/up GEMMs take the 128-row tile (the 4096-row
out- and down-projections the 64-row tile); the decode passes run the batch-1
hipGraph (fused RMSNorm / SwiGLU GEMV forms, the 151936-row LM head).
The same prompt then runs as one sequence of a 16-sequence batch state, whose
decode takes the skinny GEMMs at their real shapes.

The reference itself, compiled from its sources, ran the same model bytes and
prompt (tests/golden/hybrid8b_model.npz, manifest "hybrid8b_model": its greedy
ids and the sha256 of its prefill and last logit vectors); both the GPU and
the oracle must reproduce them.

Bar: greedy ids identical and logits bit-identical (the kernels replay the
reference's fp32 operation order; the north star's 1e-2 abs / 1e-3 rel is the
stated tolerance, bit equality is what this path delivers). The top-2 margin of
every step is printed, so a near tie would be visible (none can flip while the
logits are bit-identical)."""
import dataclasses
import hashlib
import os
import time

import numpy as np
import pytest

import hero_amd
import oracle
from gpu_util import bits, check

pytestmark = pytest.mark.gpu

SEED = 20260101
PROMPT = 600
STEPS = 32


def say(msg):
    print(msg, flush=True)


def margin(v):
    top = np.partition(v, -2)[-2:]
    return float(top[1] - top[0])


def oracle_greedy(ref, prompt, steps):
    ref.reset()
    prefill = ref.forward_ids(prompt)
    ids = [int(np.argmax(prefill))]
    last = prefill
    for _ in range(steps):
        last = ref.forward_ids([ids[-1]])
        ids.append(int(np.argmax(last)))
    return prefill, ids, last


@pytest.fixture(scope="module")
def hybrid8b():
    import torch

    assert torch.cuda.is_available()
    oracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    t = time.perf_counter()
    image = hero_amd.synthetic_gguf_image(hero_amd.HYBRID_8B_CONFIG, seed=SEED, ctx=1024)
    say(f"[8b] synthetic GGUF image {image.nbytes / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s")
    model = hero_amd.Qwen35Model.open_image(image)
    ref = oracle.Model(image=image)
    yield image, model, ref
    model.close()
    ref.close()


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


@pytest.mark.timeout(1200)
def test_hybrid8b_prefill_and_greedy_decode_match_oracle(hybrid8b, manifest):
    import ctypes

    golden = np.load(os.path.join(os.path.dirname(__file__), "golden", "hybrid8b_model.npz"))
    g = manifest["hybrid8b_model"]
    assert (g["prompt_len"], g["decode_steps"], g["seed"], g["ctx"]) == (PROMPT, STEPS, SEED, 1024)

    _, model, ref = hybrid8b
    from hero_amd._lib import lib

    tiles = {}
    for n in (16448, 24576, 10240, 4096):  # delta-net in-proj, gate|up, attention in-proj, out-proj
        tile = ctypes.c_int32()
        check(lib.hero_q8_0_gemm_plan(PROMPT, n, 4096, ctypes.byref(tile)))
        tiles[(PROMPT, n)] = tile.value
    say(f"[8b] prefill GEMM tiles ((rows, N): rows per tile): {tiles}")
    assert tiles[(PROMPT, 16448)] == 128 and tiles[(PROMPT, 24576)] == 128
    prompt = np.random.default_rng(SEED).integers(0, model.V, PROMPT).astype(np.int32)
    assert np.array_equal(prompt, golden["prompt"])
    t = time.perf_counter()
    ref_prefill, ref_ids, ref_last = oracle_greedy(ref, prompt, STEPS)
    say(f"[8b] oracle: {PROMPT}-token prefill + {STEPS} greedy passes in {time.perf_counter() - t:.1f} s; ids {ref_ids}")
    assert ref_ids == [int(i) for i in golden["ids"]], "oracle ids differ from the reference's"
    assert digest(ref_prefill) == g["logits_prefill_sha256"] and digest(ref_last) == g["logits_last_sha256"]

    state = model.new_state(1024)
    lg = model.forward(state, ids=prompt)
    exact = float(np.mean(bits(lg.values) == bits(ref_prefill)))
    say(f"[8b] prefill logits: exact fraction {exact:.6f}, max|d| {np.abs(lg.values - ref_prefill).max():.3g}, "
        f"top-2 margin {margin(lg.values):.4g}")
    assert np.array_equal(bits(lg.values), bits(ref_prefill))
    ids, last = model.decode_greedy(state, lg.argmax(), STEPS, want_logits=True)
    got = [lg.argmax()] + [int(i) for i in ids]
    say(f"[8b] GPU greedy ids {got}; last-step top-2 margin {margin(last.values):.4g}")
    assert got == ref_ids, f"first divergence at step {next(i for i, (a, b) in enumerate(zip(got, ref_ids)) if a != b)}"
    assert np.array_equal(bits(last.values), bits(ref_last))
    assert digest(lg.values) == g["logits_prefill_sha256"] and digest(last.values) == g["logits_last_sha256"]
    say("[8b] GPU ids and prefill / last logits equal the reference's (sha256)")
    assert state.tokens() == PROMPT + STEPS
    state.close()

    # the same prompt as sequence 5 of a 16-sequence batch, next to sequences
    # with short prompts; sequence 0's prompt also runs through the oracle
    short = np.random.default_rng(SEED + 1).integers(0, model.V, 6).astype(np.int32)
    bs = model.new_batch_state(1024, 16)
    firsts = []
    for b in range(16):
        p = prompt if b == 5 else (short if b == 0 else np.random.default_rng(SEED + 2 + b).integers(0, model.V, 1 + b % 9).astype(np.int32))
        firsts.append(model.forward_seq(bs, b, ids=p).argmax())
    out, logits = model.decode_batch(bs, firsts, STEPS, want_logits=True)
    assert [firsts[5]] + [int(v) for v in out[:, 5]] == ref_ids
    assert np.array_equal(bits(logits[5]), bits(ref_last))
    t = time.perf_counter()
    _, ref_ids0, ref_last0 = oracle_greedy(ref, short, STEPS)
    say(f"[8b] oracle short prompt in {time.perf_counter() - t:.1f} s")
    assert [firsts[0]] + [int(v) for v in out[:, 0]] == ref_ids0
    assert np.array_equal(bits(logits[0]), bits(ref_last0))
    say("[8b] batch of 16: sequences 0 and 5 equal the oracle bit for bit")
    bs.close()


ATOL, RTOL = 1e-2, 1e-3  # the stated tolerance, for the paths that reorder fp32 sums


@pytest.mark.timeout(600)
def test_hybrid8b_width_paged_caches_match_oracle():
    """The opt-in attention caches at 8B width (32 q / 8 kv heads of 128,
    d_model 4096; 4 layers, the attention layer last): the fp16 and the Q8_0
    paged caches against the oracle with the matching cache switch (K/V rows
    stored as fp16, or as their Q8_0 round trip), a 64-token prefill (one
    chunk of 64 rows) and 8 greedy passes (the page-streaming split at one
    sequence). The split-K attention merges its partial sums in another order
    than the reference's single pass, so the bar is the stated tolerance: ids
    identical, logits within 1e-2 abs / 1e-3 rel. A 2-sequence batch state
    with the same cache gives its sequence the single state's ids and logits
    bit for bit.

    Why not at 32 layers: the attention output is quantized to Q8_0 for the
    out-projection, so a last-ulp difference of the reordered sums sometimes
    moves one int8 by a step (1/127 of its block), and the random-weight model
    amplifies such steps layer by layer: at 32 layers the paged caches land
    ~0.2 from the oracle in the logits, as far as the oracle's own fp16 cache
    lands from its fp32 cache (0.245). With the attention layer last, only
    the last row's output reaches the logits."""
    import oracle

    shape = dataclasses.replace(hero_amd.HYBRID_8B_CONFIG, layers=4)
    image = hero_amd.synthetic_gguf_image(shape, seed=SEED + 40, ctx=1024)
    oracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    model = hero_amd.Qwen35Model.open_image(image)
    ref = oracle.Model(image=image)
    try:
        prompt = np.random.default_rng(SEED + 41).integers(0, model.V, 64).astype(np.int32)
        steps = 8
        for name, kw, switch in (("fp16", {"kv_fp16": True}, ref.set_kv_fp16), ("q8_0", {"kv_q8": True}, ref.set_kv_q8)):
            switch(True)
            try:
                ref.reset()
                ref_ids, ref_last, _, _ = ref.greedy(prompt, steps)
            finally:
                switch(False)
            st = model.new_state(1024, **kw)
            first = model.forward(st, ids=prompt)
            ids, last = model.decode_greedy(st, first.argmax(), steps, want_logits=True)
            st.close()
            got = [first.argmax()] + [int(v) for v in ids]
            d = np.abs(last.values - ref_last)
            say(f"[8b-width {name} cache] ids {got}; last pass max|d| {d.max():.3g}, exact {np.mean(bits(last.values) == bits(ref_last)):.4f}")
            assert got[:-1] == [int(v) for v in ref_ids[:-1]]
            assert np.all(d <= ATOL + RTOL * np.abs(ref_last))
            bs = model.new_batch_state(1024, 2, **kw)
            f0 = model.forward_seq(bs, 0, ids=prompt[:5]).argmax()
            f1 = model.forward_seq(bs, 1, ids=prompt).argmax()
            out, logits = model.decode_batch(bs, [f0, f1], 4, want_logits=True)
            bs.close()
            st2 = model.new_state(1024, **kw)
            model.forward(st2, ids=prompt)
            ids2, lg2 = model.decode_greedy(st2, f1, 4, want_logits=True)
            st2.close()
            assert np.array_equal(out[:, 1], ids2)
            assert np.array_equal(bits(logits[1]), bits(lg2.values))
    finally:
        model.close()
        ref.close()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("mix", [hero_amd.WEIGHTS_K_MIX, hero_amd.WEIGHTS_Q8_FFN_MIX])
def test_hybrid8b_width_kquant_mixes_match_oracle(mix):
    """Mixed-type checkpoints at 8B width (d_model 4096, SwiGLU 12288, vocab
    151936, 32 q / 8 kv heads; 4 layers: 3 delta-net + 1 attention, untied
    head): the Q4_K_M-style mix (Q4_K, Q5_K, Q6_K, Q8_0 tensors) and the mix
    with Q8_0 in-projections and gate / up (12288 rows each, written into the
    interleaved gate|up rows through the typed linears' strided scratch)
    beside a Q6_K embedding and down projection and Q4_K output projections.
    16-token prefill and 4 greedy passes against the oracle on the same bytes:
    ids identical and logits bit-identical (the integer sums are exact and
    the fp32 chains run in the reference's order)."""
    import oracle

    shape = dataclasses.replace(hero_amd.HYBRID_8B_CONFIG, layers=4)
    t = time.perf_counter()
    image = hero_amd.synthetic_gguf_image(shape, seed=SEED + 50 + mix, ctx=256, tied=False, weight_mix=mix)
    say(f"[8b-width mix {mix}] synthetic GGUF image {image.nbytes / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s")
    oracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    model = hero_amd.Qwen35Model.open_image(image)
    ref = oracle.Model(image=image)
    try:
        prompt = np.random.default_rng(SEED + 60 + mix).integers(0, model.V, 16).astype(np.int32)
        t = time.perf_counter()
        ref_prefill, ref_ids, ref_last = oracle_greedy(ref, prompt, 4)
        say(f"[8b-width mix {mix}] oracle prefill + 4 passes in {time.perf_counter() - t:.1f} s; ids {ref_ids}")
        st = model.new_state(256)
        lg = model.forward(st, ids=prompt)
        assert np.array_equal(bits(lg.values), bits(ref_prefill))
        ids, last = model.decode_greedy(st, lg.argmax(), 4, want_logits=True)
        assert [lg.argmax()] + [int(v) for v in ids] == ref_ids
        assert np.array_equal(bits(last.values), bits(ref_last))
        st.close()
    finally:
        model.close()
        ref.close()
