"""The benchmark's own workload on the ~8B Q8_0 hybrid (32 layers: 24 gated
delta-net + 8 GQA; d_model 4096, FFN 12288, vocab 151936), against the
REFERENCE's outputs for it (tests/golden/hybrid8b_2k_model.npz, manifest
"hybrid8b_2k_model", written by the compiled reference through
PrefixCache::evaluate, tools/qwen35_check.cpp:43-70):

* batch 1: the bench's 2048-token prompt (two 1024-row prefill chunks: every
  prefill GEMM on the 128-row tile), then 64 greedy passes of the batch-1
  decode graph at context 2049..2112;
* batch 16: the bench's 16 prompts of 2048 tokens prefilled into one batch
  state, then 64 greedy passes of the batch decode graph (skinny GEMMs);
  sequences 0 and 15 are checked.

Bar: the greedy ids equal the reference's, and the prefill and last-pass logit
vectors are bit-identical to the reference's (sha256)."""
import ctypes
import hashlib
import json
import os
import time

import numpy as np
import pytest

import hero_amd
from gpu_util import check

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def say(msg):
    print(msg, flush=True)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(HERE, "golden", "manifest.json")) as f:
        g = json.load(f)["hybrid8b_2k_model"]
    return g, dict(np.load(os.path.join(HERE, "golden", "hybrid8b_2k_model.npz")))


@pytest.fixture(scope="module")
def model(golden):
    import torch

    assert torch.cuda.is_available()
    g, _ = golden
    t = time.perf_counter()
    image = hero_amd.synthetic_gguf_image(hero_amd.HYBRID_8B_CONFIG, seed=g["seed"], ctx=g["ctx"])
    sha = hashlib.sha256(memoryview(image)).hexdigest()
    say(f"[8b-2k] synthetic GGUF image {image.nbytes / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s")
    assert sha == g["gguf_sha256"], "synthetic 8B model bytes differ from the reference run's"
    m = hero_amd.Qwen35Model.open_image(image)
    del image
    yield m
    m.close()


def prompt_of(g, run):
    return np.random.default_rng(g["runs"][run]["prompt_seed"]).integers(0, 151936, g["prompt_len"]).astype(np.int32)


@pytest.mark.timeout(600)
def test_benchmark_workload_batch1_matches_reference(model, golden):
    from hero_amd._lib import lib

    g, gold = golden
    tiles = {}
    for n, k in ((16448, 4096), (24576, 4096), (10240, 4096), (4096, 4096), (4096, 12288)):
        tile = ctypes.c_int32()
        check(lib.hero_q8_0_gemm_plan(1024, n, k, ctypes.byref(tile)))
        tiles[(n, k)] = tile.value
    say(f"[8b-2k] 1024-row chunk GEMM tiles ((N, K): rows per tile): {tiles}")
    assert set(tiles.values()) == {128}
    prompt = prompt_of(g, "b1")
    state = model.new_state(g["ctx"])
    lg = model.forward(state, ids=prompt)
    assert digest(lg.values) == g["runs"]["b1"]["logits_prefill_sha256"], "2048-token prefill logits differ from the reference's"
    ids, last = model.decode_greedy(state, lg.argmax(), g["decode_steps"], want_logits=True)
    got = [lg.argmax()] + [int(i) for i in ids]
    ref = [int(i) for i in gold["b1_ids"]]
    assert got == ref, f"first divergence at pass {next(i for i, (a, b) in enumerate(zip(got, ref)) if a != b)}"
    assert digest(last.values) == g["runs"]["b1"]["logits_last_sha256"], "last-pass logits differ from the reference's"
    assert state.tokens() == g["prompt_len"] + g["decode_steps"]
    say(f"[8b-2k] batch 1: 2048-token prefill and {g['decode_steps']} greedy passes equal the reference's (ids, sha256)")
    state.close()


@pytest.mark.timeout(600)
def test_benchmark_workload_batch16_matches_reference(model, golden):
    g, gold = golden
    steps = g["decode_steps"]
    bctx = ((g["prompt_len"] + steps + 8 + 255) // 256) * 256  # bench.py's batch-state size
    bs = model.new_batch_state(bctx, 16)
    seeds = [g["seed"] + 1 + b for b in range(16)]  # bench.py's batch prompts
    assert seeds[0] == g["runs"]["seq0"]["prompt_seed"] and seeds[15] == g["runs"]["seq15"]["prompt_seed"]
    firsts = []
    for b, s in enumerate(seeds):
        p = np.random.default_rng(s).integers(0, 151936, g["prompt_len"]).astype(np.int32)
        if b in (0, 15):
            lg = model.forward_seq(bs, b, ids=p)
            assert digest(lg.values) == g["runs"][f"seq{b}"]["logits_prefill_sha256"], f"sequence {b}: prefill logits differ"
            firsts.append(lg.argmax())
        else:
            firsts.append(model.forward_seq(bs, b, ids=p, want_logits=False))
    out, logits = model.decode_batch(bs, firsts, steps, want_logits=True)
    for b in (0, 15):
        got = [firsts[b]] + [int(v) for v in out[:, b]]
        ref = [int(i) for i in gold[f"seq{b}_ids"]]
        assert got == ref, f"sequence {b}: first divergence at pass {next(i for i, (x, y) in enumerate(zip(got, ref)) if x != y)}"
        assert digest(logits[b]) == g["runs"][f"seq{b}"]["logits_last_sha256"], f"sequence {b}: last-pass logits differ"
    say(f"[8b-2k] batch 16: sequences 0 and 15 equal the reference's over 2048-token prefills and {steps} passes")
    bs.close()
