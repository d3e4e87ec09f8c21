"""Gemma 4 E4B text on the GPU against the REFERENCE's outputs
(tests/golden/gemma4_e4b_model.npz, manifest "gemma4_e4b_model", written by
the compiled reference's Gemma4E4BModel through PrefixCache::evaluate, the
loop of tools/gemma4_text.cpp:16-52).

The reference's Gemma classes are fixed to the E4B configuration
(nm/src/gemma4.hpp:19-35), so the model is full size: 42 layers (every sixth
attends over the whole context with 512-wide heads, the others over a
512-position window with 256-wide heads; the last 18 reuse the K/V of layers
22 and 23), d_model 2560, GELU FFN 10240, per-layer inputs of 256, vocabulary
262144, tied and soft-capped head; a seeded synthetic 7.9 GB Q8_0 GGUF built
on the box and checked by sha256. The 600-token prompt runs past the window,
so the rings wrap and the K/V-sharing layers read windows of layer 22's ring.

Bar: the greedy ids equal the reference's and the prefill and last-pass logit
vectors are bit-identical (sha256)."""
import ctypes
import hashlib
import json
import os
import time

import numpy as np
import pytest

from gpu_util import check

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def say(msg):
    print(msg, flush=True)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def test_gelu_and_softcap_equal_glibc_arithmetic():
    """The device's gelu_pytorch_tanh and soft-cap (hero_gemma_math_eval) against
    the same fp32 expressions on the host with glibc's tanhf (ctypes), on a
    spread of magnitudes and the edge values."""
    import torch

    from hero_amd import lib

    libm = ctypes.CDLL("libm.so.6")
    libm.tanhf.restype = ctypes.c_float
    libm.tanhf.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(3000).astype(np.float32) * s for s in (0.01, 1.0, 5.0, 40.0)]
                       + [np.array([0.0, -0.0, 1e-30, -1e-30, 9.0, -9.0, 22.0, -22.0, 1e4, -1e4, np.inf, -np.inf], np.float32)])
    f = np.float32
    cap = f(30.0)
    want = np.empty((len(x), 2), np.float32)
    for i, v in enumerate(x):
        v = f(v)
        with np.errstate(over="ignore", invalid="ignore"):
            inner = f(f(0.7978845608) * f(v + f(f(f(f(0.044715) * v) * v) * v)))
            want[i, 0] = f(f(f(0.5) * v) * f(f(1.0) + f(libm.tanhf(inner))))
            want[i, 1] = f(cap * f(libm.tanhf(f(v / cap))))
    xd = torch.from_numpy(x).cuda()
    out = torch.empty(2 * len(x), dtype=torch.float32, device="cuda")
    check(lib.hero_gemma_math_eval(xd.data_ptr(), out.data_ptr(), len(x), float(cap), None))
    got = out.cpu().numpy().reshape(-1, 2)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{int((~same).sum())} differ, first at x={x[np.argwhere(~same)[0][0]]!r}"


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(HERE, "golden", "manifest.json")) as f:
        g = json.load(f)["gemma4_e4b_model"]
    return g, dict(np.load(os.path.join(HERE, "golden", "gemma4_e4b_model.npz")))


@pytest.fixture(scope="module")
def image(golden):
    from hero_amd.gemma4 import GEMMA4_E4B, synthetic_gemma4_image

    g, _ = golden
    t = time.perf_counter()
    img = synthetic_gemma4_image(GEMMA4_E4B, seed=g["seed"])
    sha = hashlib.sha256(memoryview(img)).hexdigest()
    say(f"[gemma4] synthetic E4B GGUF image {img.nbytes / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s")
    assert sha == g["gguf_sha256"], "synthetic Gemma 4 model bytes differ from the reference run's"
    return img


@pytest.fixture(scope="module")
def model(image):
    import torch

    from hero_amd.gemma4 import Gemma4Model

    assert torch.cuda.is_available()
    t = time.perf_counter()
    m = Gemma4Model.open_image(image)
    say(f"[gemma4] loaded in {time.perf_counter() - t:.1f} s, {m.dims.device_bytes / 1e9:.2f} GB of weights")
    yield m
    m.close()


def test_gemma4_e4b_matches_reference(model, golden):
    g, gold = golden
    prompt = gold["prompt"]
    state = model.new_state(1024)
    t = time.perf_counter()
    logits = model.forward(state, prompt)
    say(f"[gemma4] {len(prompt)}-token prompt (token by token) in {time.perf_counter() - t:.1f} s")
    head = len(gold["prefill_head"])
    diff = np.abs(logits.values[:head] - gold["prefill_head"])
    say(f"[gemma4] prefill logits: max |diff| over the first {head}: {diff.max():.3g}; exact {np.mean(diff == 0):.4f}")
    assert digest(logits.values) == g["logits_prefill_sha256"], "prefill logits differ from the reference's"
    ids = [int(i) for i in gold["ids"]]
    assert logits.argmax() == ids[0]
    out, last = model.decode_greedy(state, ids[0], g["decode_steps"], want_logits=True)
    say(f"[gemma4] {g['decode_steps']} greedy passes: {model.last_decode_seconds() * 1e3 / g['decode_steps']:.3f} ms/pass")
    assert [int(i) for i in out] == ids[1:], "greedy ids differ from the reference's"
    assert np.array_equal(last.values[:head], gold["last_head"])
    assert digest(last.values) == g["logits_last_sha256"], "last-pass logits differ from the reference's"
    assert state.tokens() == len(prompt) + g["decode_steps"]


def test_gemma4_e4b_short_run_gpu_and_oracle_match_reference(model, image, golden):
    """The 16-token prompt and 4 greedy passes of the golden (short_*): the GPU
    and the oracle's restatement (batched prefill, as the reference runs it)
    both give the reference's logits bit for bit."""
    import oracle

    g, gold = golden
    prompt, ids = gold["short_prompt"], [int(i) for i in gold["short_ids"]]
    state = model.new_state(64)
    logits = model.forward(state, prompt)
    assert digest(logits.values) == g["short_logits_prefill_sha256"]
    out, last = model.decode_greedy(state, ids[0], g["short_decode_steps"], want_logits=True)
    assert [int(i) for i in out] == ids[1:]
    assert digest(last.values) == g["short_logits_last_sha256"]

    t = time.perf_counter()
    ref = oracle.Gemma4(image=image)
    pre = ref.forward(prompt)
    assert np.array_equal(pre[:len(gold["short_prefill_head"])], gold["short_prefill_head"])
    assert digest(pre) == g["short_logits_prefill_sha256"], "the oracle's prefill logits differ from the reference's"
    got = [int(np.argmax(pre))]
    for _ in range(g["short_decode_steps"]):
        lg = ref.forward([got[-1]])
        got.append(int(np.argmax(lg)))
    assert got == ids and digest(lg) == g["short_logits_last_sha256"], "the oracle's decode differs from the reference's"
    say(f"[gemma4] oracle short run in {time.perf_counter() - t:.1f} s")
    ref.close()
