"""Write the golden vectors of tests/golden/ by running the REFERENCE engine.

The reference (flywithfang/hero, nm/src) is compiled from its own sources by
oracle/Makefile into oracle/_ref/ref_harness (this needs the reference tree,
so it runs in the build container only). This script:

  1. writes seeded inputs for every kernel case, runs `ref_harness kernels`,
     and stores inputs + outputs in kernels.npz;
  2. writes the tiny Q8_0 hybrid model as GGUF with the package's seeded
     synthetic writer, runs `ref_harness model tiny` (16-token random prompt,
     128 greedy decode passes through PrefixCache::evaluate) and stores the
     greedy ids, per-step top-5 and three full logit vectors in tiny_model.npz;
  3. `window`: causal and sliding-window attention over the reference's own
     FullAttentionCache / LocalAttentionCache (widths 3 and 1024, 1100
     positions, probes before and after the ring starts evicting) -> window.npz;
  4. `variant`: the tiny shape with 4 delta-net key heads tiled over 8 value
     heads and an untied output.weight -> tiny_hk4u_model.npz;
  5. `kmix`: the tiny shape with the tensor types of a Q4_K_M checkpoint
     (Q4_K, Q5_K, Q6_K and Q8_0 tensors) -> tiny_kmix_model.npz;
  6. `hybrid8b`: the ~8B shape (the benchmark's model, seed 20260101, a
     600-token prompt, 32 greedy passes) -> hybrid8b_model.npz with the ids,
     per-step top-5 and the sha256 of the prefill and last logit vectors;
  8. `q8ffn`: the tiny shape with SwiGLU width 3584 (above every input
     projection's width) and Q8_0 in-projections, gate and up beside a Q6_K
     embedding and down projection and Q4_K output projections ->
     tiny_q8ffn_model.npz;
  9. `hybrid8b_2k`: the ~8B shape on the benchmark's workload: 2048-token
     prompts (the batch-1 prompt and sequences 0 and 15 of the 16-sequence
     batch) and 64 greedy passes each -> hybrid8b_2k_model.npz (ids, top-5,
     and the sha256 of the prefill and last logit vectors in the manifest);
  10. `gemma4`: the reference's Gemma 4 E4B text model (its classes are fixed
     to the E4B configuration, so the model is full size: a seeded synthetic
     7.9 GB Q8_0 GGUF), a 600-token prompt (past the 512-position window, so
     the rings wrap and the K/V-sharing layers read the window) and 32 greedy
     passes, and a 16-token prompt with 4 passes (short_*) -> gemma4_e4b_model.npz
     (ids, top-5, the first 8192 logits of the prefill and last passes) and
     the sha256 of every full logit vector;
  7. `dh256`: the attention geometry of the reference's Qwen 3.5 4B / 9B
     configs (256-wide heads, a quarter rotating, RoPE base 1e7, Hk 4 over
     Hv 8, untied head) at tiny width -> tiny_dh256_model.npz.

manifest.json records seeds, shapes, the GGUF's sha256 and the compiler
flags (-O3 -march=x86-64-v3 -ffp-contract=off: no FMA contraction).

Run:  python tests/golden/make_golden.py [kernels] [tiny] [window] [variant] [kmix] [hybrid8b] [dh256] [q8ffn] [hybrid8b_2k] [gemma4]
      (no argument: all parts; the manifest keeps the entries of parts not rerun)
"""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(ROOT, "oracle", "_ref", "ref_harness")

TINY_SEED = 1234
PROMPT_SEED = 7
PROMPT_LEN = 16
DECODE_STEPS = 128


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def kernel_inputs(rng: np.random.Generator) -> dict[str, np.ndarray]:
    inp = {}
    # fp16 encoder: special values, exact ties, subnormals, random bit patterns
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, np.inf, -np.inf, np.nan,
                        5.960464477539063e-08, 2.9802322387695312e-08, 2.98023224e-08 * 1.5, 6.103515625e-05,
                        6.097555160522461e-05, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -11 + 2.0 ** -20,
                        2049.0, 2051.0, 1e-8, 1e-12, 3.14159265], dtype=np.float32)
    bits = rng.integers(0, 2 ** 32, 50000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    mags = (rng.standard_normal(20000) * np.exp(rng.uniform(-20, 12, 20000))).astype(np.float32)
    inp["fp16_encode"] = f32(np.concatenate([special, bits, mags]))
    # quantizer input: 128 blocks of varied magnitude + crafted blocks
    x = rng.standard_normal(4096).astype(np.float32) * np.repeat(np.exp(rng.uniform(-8, 4, 128)), 32).astype(np.float32)
    x[0:32] = 0.0                                          # zero block: d = 0, q = 0
    x[32:64] = np.arange(-15.5, 16.5, 1.0)                 # amax 16.5 -> exercise .5 ties
    x[64:96] = np.float32(127.0) * rng.uniform(-1, 1, 32)  # d near 1
    x[64] = 127.0
    x[65:73] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]  # exact ties at id = 1
    x[96:128] = rng.standard_normal(32) * 1e-6            # tiny d (fp16 subnormal scale)
    inp["quant"] = f32(x)
    inp["gemv_w"] = f32(rng.standard_normal((64, 4096)) * 0.02)
    inp["gemv_x"] = f32(rng.standard_normal((8, 4096)))
    for n in (128, 1024, 4096):
        inp[f"rms{n}"] = f32(np.concatenate([rng.standard_normal(n) * 3, 1 + 0.1 * rng.standard_normal(n)]))
    inp["l2"] = f32(rng.standard_normal((16, 128)))
    act = np.concatenate([np.linspace(-30, 30, 4001), [0.0, 20.0, -20.0, 20.000002, 19.999998, 88.0, -88.0, 1e-20]])
    inp["act"] = f32(np.concatenate([act, rng.standard_normal(87) * 5]))
    inp["conv_taps"] = f32(rng.standard_normal((256, 4)) * 0.5)
    inp["conv_x"] = f32(rng.standard_normal((6, 256)))
    inp["delta_state"] = f32(rng.standard_normal(128 * 128) * 0.1)
    tok = []
    for _ in range(4):
        q = rng.standard_normal(128)
        k = rng.standard_normal(128)
        q = q / np.linalg.norm(q) / np.sqrt(128)
        k = k / np.linalg.norm(k)
        v = rng.standard_normal(128)
        gate = -np.log1p(np.exp(rng.standard_normal()))
        beta = 1 / (1 + np.exp(-rng.standard_normal()))
        tok.append(np.concatenate([q, k, v, [gate, beta]]))
    inp["delta_tok"] = f32(np.concatenate(tok))
    inp["rope"] = f32(rng.standard_normal((8, 128)))
    ctx = 300
    inp["attn_q"] = f32(rng.standard_normal(128) / np.sqrt(128))
    inp["attn_k"] = f32(rng.standard_normal((ctx, 128)) / np.sqrt(128))
    inp["attn_v"] = f32(rng.standard_normal((ctx, 128)) / np.sqrt(128))
    # K-quants: activations [4][4096] with crafted Q8_K blocks in row 1, and
    # raw Q4_K / Q6_K weight blocks [64 rows][16 blocks] from random bytes
    kx = (rng.standard_normal((4, 4096)) * np.repeat(np.exp(rng.uniform(-6, 3, (4, 16))), 256, axis=1)).astype(np.float32)
    kx[1, 0:256] = 0.0                                    # zero block: d = 0, all zero
    kx[1, 256 + 7] = kx[1, 256 + 99] = -3 * np.abs(kx[1, 256:512]).max()  # negative max, twice
    kx[1, 512:768] = rng.integers(-126, 127, 256) + 0.5   # max -127 below: scale 1, exact ties
    kx[1, 512 + 3] = -127.0
    kx[1, 768 + 10], kx[1, 768 + 20] = 5.0, -5.0          # equal magnitudes: the first sets the sign
    kx[1, 768:1024] = np.clip(kx[1, 768:1024], -4.9, 4.9)
    kx[1, 768 + 10], kx[1, 768 + 20] = 5.0, -5.0
    inp["kq_x"] = f32(kx)
    f16 = lambda a: np.asarray(a, np.float16).view(np.uint8).reshape(*np.shape(a), 2)  # noqa: E731
    nb = 64 * 16
    w4 = np.concatenate([f16(rng.uniform(0.2, 2.0, nb) * 1e-2), f16(rng.uniform(0.0, 2.0, nb) * 1e-2),
                         rng.integers(0, 256, (nb, 12)).astype(np.uint8), rng.integers(0, 256, (nb, 128)).astype(np.uint8)], axis=1)
    inp["kq_w4"] = np.ascontiguousarray(w4.astype(np.uint8))
    w6 = np.concatenate([rng.integers(0, 256, (nb, 128 + 64)).astype(np.uint8), rng.integers(-128, 128, (nb, 16)).astype(np.int8).view(np.uint8),
                         f16(rng.uniform(0.2, 2.0, nb) * 1e-3)], axis=1)
    inp["kq_w6"] = np.ascontiguousarray(w6.astype(np.uint8))
    # sampling: 8 rows of 32000 distinct logits at a few temperatures' scales
    inp["sample_logits"] = f32(rng.standard_normal((8, 32000)) * np.array([1, 2, 3, 4, 6, 8, 0.5, 12])[:, None])
    # raw Q5_K weight blocks [64 rows][16 blocks] from random bytes (drawn last,
    # so the inputs above keep their values)
    w5 = np.concatenate([f16(rng.uniform(0.2, 2.0, nb) * 1e-2), f16(rng.uniform(0.0, 2.0, nb) * 1e-2),
                         rng.integers(0, 256, (nb, 12 + 32 + 128)).astype(np.uint8)], axis=1)
    inp["kq_w5"] = np.ascontiguousarray(w5.astype(np.uint8))
    return inp


OUTPUTS = {  # name -> dtype of the .out.bin
    "fp16_encode": np.uint16, "quant_act": np.uint8, "quant_weight": np.uint8, "gemv_wq": np.uint8,
    "gemv_y": np.float32, "gemm_y": np.float32, "rms128": np.float32, "rms1024": np.float32, "rms4096": np.float32,
    "l2": np.float32, "silu": np.float32, "sigmoid": np.float32, "softplus": np.float32, "conv": np.float32,
    "delta_out": np.float32, "delta_state": np.float32, "rope": np.float32, "attn_scaled": np.float32, "attn_unit": np.float32,
    "kq_act": np.uint8, "kq_y4": np.float32, "kq_y6": np.float32, "sample": np.float32,
    "kq_y5": np.float32, "kq_dq4": np.float32, "kq_dq5": np.float32, "kq_dq6": np.float32,
}


def make_kernels(tmp: str) -> dict:
    rng = np.random.default_rng(20260101)
    inp = kernel_inputs(rng)
    for k, v in inp.items():
        v.tofile(os.path.join(tmp, f"{k}.in.bin"))
    subprocess.run([HARNESS, "kernels", tmp], check=True)
    # the fp32 GEMV weights are only the quantizer's input; the reference's
    # quantized blocks (out_gemv_wq) are what the GEMV cases consume
    out = {f"in_{k}": v for k, v in inp.items() if k != "gemv_w"}
    for k, dt in OUTPUTS.items():
        out[f"out_{k}"] = np.fromfile(os.path.join(tmp, f"{k}.out.bin"), dtype=dt)
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **out)
    return {"seed": 20260101, "cases": sorted(OUTPUTS)}


def make_tiny(tmp: str) -> dict:
    import hero_amd

    gguf = os.path.join(tmp, "tiny.gguf")
    hero_amd.write_synthetic_gguf(gguf, hero_amd.TINY_CONFIG, seed=TINY_SEED, ctx=4096)
    sha = hashlib.sha256(open(gguf, "rb").read()).hexdigest()
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, hero_amd.TINY_CONFIG.vocab, PROMPT_LEN).astype(np.int32)
    prompt.tofile(os.path.join(tmp, "prompt.i32"))
    outdir = os.path.join(tmp, "tiny_out")
    os.makedirs(outdir, exist_ok=True)
    subprocess.run([HARNESS, "model", "tiny", gguf, os.path.join(tmp, "prompt.i32"), str(DECODE_STEPS), outdir], check=True)
    rd = lambda n, dt: np.fromfile(os.path.join(outdir, n), dtype=dt)  # noqa: E731
    np.savez_compressed(
        os.path.join(HERE, "tiny_model.npz"),
        prompt=prompt,
        ids=rd("ids.i32", np.int32),
        top5_ids=rd("top5_ids.i32", np.int32).reshape(-1, 5),
        top5_logits=rd("top5_logits.f32", np.float32).reshape(-1, 5),
        logits_prefill=rd("logits_prefill.f32", np.float32),
        logits_mid=rd("logits_mid.f32", np.float32),
        logits_last=rd("logits_last.f32", np.float32),
    )
    times = open(os.path.join(outdir, "times.txt")).read()
    return {"seed": TINY_SEED, "prompt_seed": PROMPT_SEED, "prompt_len": PROMPT_LEN, "decode_steps": DECODE_STEPS,
            "ctx": 4096, "gguf_sha256": sha, "gguf_bytes": os.path.getsize(gguf), "reference_times": times,
            "logits_mid_after_pass": DECODE_STEPS // 2}


WINDOW_SEED = 1103
WINDOW_CTX = 1100
WINDOW_PROBES = [0, 1, 2, 3, 4, 7, 500, 1022, 1023, 1024, 1025, 1099]


def window_inputs(seed: int = WINDOW_SEED, ctx: int = WINDOW_CTX):
    """4 query heads over 2 K/V heads of 128: K, V N(0,1)/sqrt(128), q N(0,1)
    (tests/conftest.py regenerates the same arrays and checks their sha256)"""
    rng = np.random.default_rng(seed)
    s = np.float32(1 / np.sqrt(128.0))
    k = f32(rng.standard_normal((ctx, 256)) * s)
    v = f32(rng.standard_normal((ctx, 256)) * s)
    q = f32(rng.standard_normal((ctx, 512)))
    return k, v, q


def make_window(tmp: str) -> dict:
    k, v, q = window_inputs()
    for name, a in (("window_k", k), ("window_v", v), ("window_q", q), ("window_probes", f32(WINDOW_PROBES))):
        a.tofile(os.path.join(tmp, f"{name}.in.bin"))
    subprocess.run([HARNESS, "window", tmp], check=True)
    out = {"probes": np.array(WINDOW_PROBES, np.int32)}
    for name in ("window_full", "window_w3", "window_w1024"):
        r = np.fromfile(os.path.join(tmp, f"{name}.out.bin"), np.float32).reshape(len(WINDOW_PROBES), 512 + 2)
        out[name] = r[:, :512].copy()
        out[name + "_rows"] = r[:, 512:].astype(np.int64)  # [first, end) of the visible cache rows
    np.savez_compressed(os.path.join(HERE, "window.npz"), **out)
    inputs_sha = hashlib.sha256(k.tobytes() + v.tobytes() + q.tobytes()).hexdigest()
    return {"seed": WINDOW_SEED, "ctx": WINDOW_CTX, "probes": WINDOW_PROBES, "q_heads": 4, "kv_heads": 2, "head_dim": 128,
            "inputs_sha256": inputs_sha,
            "cases": {"window_full": "FullAttentionCache, scale 1/sqrt(128)", "window_w3": "LocalAttentionCache(3), scale 1",
                      "window_w1024": "LocalAttentionCache(1024), scale 1"}}


VARIANT_SEED = 4321
HYBRID8B_SEED = 20260101
HYBRID8B_PROMPT = 600
HYBRID8B_STEPS = 32


def run_model_case(tmp: str, cfg: str, shape, seed: int, ctx: int, tied: bool, prompt: np.ndarray, steps: int, where: str,
                   weight_mix: int = 0):
    import hero_amd

    gguf = os.path.join(where, f"{cfg}.gguf")
    hero_amd.write_synthetic_gguf(gguf, shape, seed=seed, ctx=ctx, tied=tied, weight_mix=weight_mix)
    h = hashlib.sha256()
    with open(gguf, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    size = os.path.getsize(gguf)
    prompt.tofile(os.path.join(tmp, f"{cfg}_prompt.i32"))
    outdir = os.path.join(tmp, f"{cfg}_out")
    os.makedirs(outdir, exist_ok=True)
    subprocess.run([HARNESS, "model", cfg, gguf, os.path.join(tmp, f"{cfg}_prompt.i32"), str(steps), outdir], check=True)
    os.remove(gguf)
    rd = lambda n, dt: np.fromfile(os.path.join(outdir, n), dtype=dt)  # noqa: E731
    times = open(os.path.join(outdir, "times.txt")).read()
    return rd, h.hexdigest(), size, times


def make_variant(tmp: str) -> dict:
    import hero_amd

    shape = hero_amd.HybridShape(vocab=32000, d_model=1024, layers=4, ffn=2816, q_heads=8, kv_heads=2, head_dim=128,
                                 key_heads=4, value_heads=8)
    prompt = np.random.default_rng(VARIANT_SEED + 1).integers(0, 32000, 16).astype(np.int32)
    rd, sha, size, times = run_model_case(tmp, "tiny_hk4u", shape, VARIANT_SEED, 4096, False, prompt, 32, tmp)
    np.savez_compressed(
        os.path.join(HERE, "tiny_hk4u_model.npz"), prompt=prompt, ids=rd("ids.i32", np.int32),
        top5_ids=rd("top5_ids.i32", np.int32).reshape(-1, 5), top5_logits=rd("top5_logits.f32", np.float32).reshape(-1, 5),
        logits_prefill=rd("logits_prefill.f32", np.float32), logits_last=rd("logits_last.f32", np.float32))
    return {"seed": VARIANT_SEED, "key_heads": 4, "value_heads": 8, "tied": False, "ctx": 4096, "prompt_len": 16,
            "decode_steps": 32, "gguf_sha256": sha, "gguf_bytes": size, "reference_times": times}


DH256_SEED = 2560
# the reference's Qwen 3.5 4B / 9B attention geometry at tiny width
DH256_SHAPE = dict(vocab=32000, d_model=1024, layers=4, ffn=2816, q_heads=8, kv_heads=2, head_dim=256, key_heads=4,
                   value_heads=8, rope_base=1e7)


def make_dh256(tmp: str) -> dict:
    import hero_amd

    shape = hero_amd.HybridShape(**DH256_SHAPE)
    prompt = np.random.default_rng(DH256_SEED + 1).integers(0, 32000, 24).astype(np.int32)
    rd, sha, size, times = run_model_case(tmp, "tiny_dh256", shape, DH256_SEED, 4096, False, prompt, 32, tmp)
    np.savez_compressed(
        os.path.join(HERE, "tiny_dh256_model.npz"), prompt=prompt, ids=rd("ids.i32", np.int32),
        top5_ids=rd("top5_ids.i32", np.int32).reshape(-1, 5), top5_logits=rd("top5_logits.f32", np.float32).reshape(-1, 5),
        logits_prefill=rd("logits_prefill.f32", np.float32), logits_last=rd("logits_last.f32", np.float32))
    return {"seed": DH256_SEED, "shape": DH256_SHAPE, "tied": False, "ctx": 4096, "prompt_len": 24, "decode_steps": 32,
            "gguf_sha256": sha, "gguf_bytes": size, "reference_times": times}


KMIX_SEED = 5150


def make_kmix(tmp: str) -> dict:
    import hero_amd

    prompt = np.random.default_rng(KMIX_SEED + 1).integers(0, 32000, 16).astype(np.int32)
    rd, sha, size, times = run_model_case(tmp, "tiny", hero_amd.TINY_CONFIG, KMIX_SEED, 4096, True, prompt, 32, tmp,
                                          weight_mix=hero_amd.WEIGHTS_K_MIX)
    np.savez_compressed(
        os.path.join(HERE, "tiny_kmix_model.npz"), prompt=prompt, ids=rd("ids.i32", np.int32),
        top5_ids=rd("top5_ids.i32", np.int32).reshape(-1, 5), top5_logits=rd("top5_logits.f32", np.float32).reshape(-1, 5),
        logits_prefill=rd("logits_prefill.f32", np.float32), logits_last=rd("logits_last.f32", np.float32))
    return {"seed": KMIX_SEED, "weight_mix": hero_amd.WEIGHTS_K_MIX, "tied": True, "ctx": 4096, "prompt_len": 16,
            "decode_steps": 32, "gguf_sha256": sha, "gguf_bytes": size, "reference_times": times,
            "types": "token_embd Q6_K; attn_qkv, attn_output Q5_K; ffn_down, attn_v Q6_K; ssm_alpha, ssm_beta Q8_0; "
                     "other projections Q4_K"}


Q8FFN_SEED = 3584
Q8FFN_SHAPE = dict(vocab=32000, d_model=1024, layers=4, ffn=3584, q_heads=8, kv_heads=2, head_dim=128, key_heads=8,
                   value_heads=8)


def make_q8ffn(tmp: str) -> dict:
    import hero_amd

    shape = hero_amd.HybridShape(**Q8FFN_SHAPE)
    prompt = np.random.default_rng(Q8FFN_SEED + 1).integers(0, 32000, 20).astype(np.int32)
    rd, sha, size, times = run_model_case(tmp, "tiny_ff3584", shape, Q8FFN_SEED, 4096, True, prompt, 32, tmp,
                                          weight_mix=hero_amd.WEIGHTS_Q8_FFN_MIX)
    np.savez_compressed(
        os.path.join(HERE, "tiny_q8ffn_model.npz"), prompt=prompt, ids=rd("ids.i32", np.int32),
        top5_ids=rd("top5_ids.i32", np.int32).reshape(-1, 5), top5_logits=rd("top5_logits.f32", np.float32).reshape(-1, 5),
        logits_prefill=rd("logits_prefill.f32", np.float32), logits_last=rd("logits_last.f32", np.float32))
    return {"seed": Q8FFN_SEED, "shape": Q8FFN_SHAPE, "weight_mix": hero_amd.WEIGHTS_Q8_FFN_MIX, "tied": True,
            "ctx": 4096, "prompt_len": 20, "decode_steps": 32, "gguf_sha256": sha, "gguf_bytes": size,
            "reference_times": times,
            "types": "token_embd, ffn_down Q6_K; ssm_out, attn_output Q4_K; in-projections, ffn_gate, ffn_up Q8_0"}


def make_hybrid8b(tmp: str) -> dict:
    import hero_amd

    prompt = np.random.default_rng(HYBRID8B_SEED).integers(0, 151936, HYBRID8B_PROMPT).astype(np.int32)
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else tmp  # the 8.45 GB GGUF, mmapped by the harness
    rd, sha, size, times = run_model_case(tmp, "8b", hero_amd.HYBRID_8B_CONFIG, HYBRID8B_SEED, 1024, True, prompt,
                                          HYBRID8B_STEPS, shm)
    digest = lambda a: hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()  # noqa: E731
    np.savez_compressed(
        os.path.join(HERE, "hybrid8b_model.npz"), prompt=prompt, ids=rd("ids.i32", np.int32),
        top5_ids=rd("top5_ids.i32", np.int32).reshape(-1, 5), top5_logits=rd("top5_logits.f32", np.float32).reshape(-1, 5))
    return {"seed": HYBRID8B_SEED, "ctx": 1024, "prompt_len": HYBRID8B_PROMPT, "decode_steps": HYBRID8B_STEPS,
            "gguf_sha256": sha, "gguf_bytes": size, "reference_times": times,
            "logits_prefill_sha256": digest(rd("logits_prefill.f32", np.float32)),
            "logits_last_sha256": digest(rd("logits_last.f32", np.float32))}


HYBRID8B_2K_PROMPT = 2048
HYBRID8B_2K_STEPS = 64
HYBRID8B_2K_CTX = 4096
# the benchmark's own prompts: batch 1 (seed SEED) and sequences 0 and 15 of
# its 16-sequence batch (seeds SEED + 1 + b)
HYBRID8B_2K_RUNS = {"b1": HYBRID8B_SEED, "seq0": HYBRID8B_SEED + 1, "seq15": HYBRID8B_SEED + 16}


def make_hybrid8b_2k(tmp: str) -> dict:
    """the ~8B model on the benchmark's workload: 2048-token prompts (two
    1024-row prefill chunks), then 64 greedy passes, for the batch-1 prompt and
    two of the batch leg's prompts; about 15 minutes of reference CPU time each"""
    import hero_amd

    shm = "/dev/shm" if os.path.isdir("/dev/shm") else tmp
    gguf = os.path.join(shm, "8b_2k.gguf")
    hero_amd.write_synthetic_gguf(gguf, hero_amd.HYBRID_8B_CONFIG, seed=HYBRID8B_SEED, ctx=HYBRID8B_2K_CTX)
    h = hashlib.sha256()
    with open(gguf, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    digest = lambda a: hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()  # noqa: E731
    out, entry = {}, {"seed": HYBRID8B_SEED, "ctx": HYBRID8B_2K_CTX, "prompt_len": HYBRID8B_2K_PROMPT,
                      "decode_steps": HYBRID8B_2K_STEPS, "gguf_sha256": h.hexdigest(), "gguf_bytes": os.path.getsize(gguf),
                      "runs": {}}
    try:
        for name, seed in HYBRID8B_2K_RUNS.items():
            prompt = np.random.default_rng(seed).integers(0, 151936, HYBRID8B_2K_PROMPT).astype(np.int32)
            prompt.tofile(os.path.join(tmp, f"{name}_prompt.i32"))
            outdir = os.path.join(tmp, f"8b2k_{name}")
            os.makedirs(outdir, exist_ok=True)
            subprocess.run([HARNESS, "model", "8b", gguf, os.path.join(tmp, f"{name}_prompt.i32"), str(HYBRID8B_2K_STEPS), outdir],
                           check=True)
            rd = lambda n, dt: np.fromfile(os.path.join(outdir, n), dtype=dt)  # noqa: E731
            out[f"{name}_prompt_seed"] = np.array([seed], np.int64)
            out[f"{name}_ids"] = rd("ids.i32", np.int32)
            out[f"{name}_top5_ids"] = rd("top5_ids.i32", np.int32).reshape(-1, 5)
            out[f"{name}_top5_logits"] = rd("top5_logits.f32", np.float32).reshape(-1, 5)
            entry["runs"][name] = {"prompt_seed": seed,
                                   "logits_prefill_sha256": digest(rd("logits_prefill.f32", np.float32)),
                                   "logits_last_sha256": digest(rd("logits_last.f32", np.float32)),
                                   "reference_times": open(os.path.join(outdir, "times.txt")).read()}
    finally:
        os.remove(gguf)
    np.savez_compressed(os.path.join(HERE, "hybrid8b_2k_model.npz"), **out)
    return entry


GEMMA4_SEED = 4242
GEMMA4_PROMPT = 600
GEMMA4_STEPS = 32
GEMMA4_HEAD = 8192  # logits kept in full per vector (the rest by sha256)


GEMMA4_SHORT_PROMPT = 16
GEMMA4_SHORT_STEPS = 4


def make_gemma4(tmp: str) -> dict:
    """Gemma 4 E4B (full size: the reference's Gemma classes take no other
    shape): a 600-token prompt and 32 greedy passes, and a short run (16
    tokens, 4 passes) cheap enough to pin the oracle's restatement; a few
    minutes of reference CPU time"""
    from hero_amd.gemma4 import GEMMA4_E4B, write_synthetic_gemma4

    shm = "/dev/shm" if os.path.isdir("/dev/shm") else tmp
    gguf = os.path.join(shm, "gemma4_e4b.gguf")
    write_synthetic_gemma4(gguf, GEMMA4_E4B, seed=GEMMA4_SEED)
    h = hashlib.sha256()
    with open(gguf, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    digest = lambda a: hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()  # noqa: E731
    runs = {"": (GEMMA4_SEED, GEMMA4_PROMPT, GEMMA4_STEPS), "short_": (GEMMA4_SEED + 1, GEMMA4_SHORT_PROMPT, GEMMA4_SHORT_STEPS)}
    out, entry = {}, {"seed": GEMMA4_SEED, "gguf_sha256": h.hexdigest(), "gguf_bytes": os.path.getsize(gguf)}
    try:
        for tag, (seed, plen, steps) in runs.items():
            prompt = np.random.default_rng(seed).integers(0, GEMMA4_E4B.vocab, plen).astype(np.int32)
            prompt.tofile(os.path.join(tmp, f"gemma4_{tag}prompt.i32"))
            outdir = os.path.join(tmp, f"gemma4_{tag}out")
            os.makedirs(outdir, exist_ok=True)
            subprocess.run([HARNESS, "model", "gemma4_e4b", gguf, os.path.join(tmp, f"gemma4_{tag}prompt.i32"), str(steps), outdir], check=True)
            rd = lambda n, dt: np.fromfile(os.path.join(outdir, n), dtype=dt)  # noqa: E731
            prefill, last = rd("logits_prefill.f32", np.float32), rd("logits_last.f32", np.float32)
            out.update({f"{tag}prompt": prompt, f"{tag}ids": rd("ids.i32", np.int32), f"{tag}top5_ids": rd("top5_ids.i32", np.int32).reshape(-1, 5),
                        f"{tag}top5_logits": rd("top5_logits.f32", np.float32).reshape(-1, 5), f"{tag}prefill_head": prefill[:GEMMA4_HEAD],
                        f"{tag}last_head": last[:GEMMA4_HEAD]})
            entry.update({f"{tag}prompt_seed": seed, f"{tag}prompt_len": plen, f"{tag}decode_steps": steps,
                          f"{tag}reference_times": open(os.path.join(outdir, "times.txt")).read(),
                          f"{tag}logits_prefill_sha256": digest(prefill), f"{tag}logits_last_sha256": digest(last)})
    finally:
        os.remove(gguf)
    np.savez_compressed(os.path.join(HERE, "gemma4_e4b_model.npz"), **out)
    return entry


PARTS = {"kernels": make_kernels, "tiny": make_tiny, "window": make_window, "variant": make_variant, "kmix": make_kmix,
         "hybrid8b": make_hybrid8b, "dh256": make_dh256, "q8ffn": make_q8ffn,
         "hybrid8b_2k": make_hybrid8b_2k, "gemma4": make_gemma4}
MANIFEST_KEYS = {"kernels": "kernels", "tiny": "tiny_model", "window": "window", "variant": "tiny_hk4u_model",
                 "kmix": "tiny_kmix_model", "hybrid8b": "hybrid8b_model", "dh256": "tiny_dh256_model",
                 "q8ffn": "tiny_q8ffn_model", "hybrid8b_2k": "hybrid8b_2k_model",
                 "gemma4": "gemma4_e4b_model"}


def main():
    if not os.path.exists(HARNESS):
        sys.exit(f"{HARNESS} missing: build it with `make -C oracle` (needs the reference tree)")
    parts = sys.argv[1:] or list(PARTS)
    path = os.path.join(HERE, "manifest.json")
    manifest = json.load(open(path)) if os.path.exists(path) else {}
    manifest.update({
        "generator": "tests/golden/make_golden.py",
        "reference": "flywithfang/hero nm/src compiled by oracle/Makefile",
        "flags": "g++ -std=c++20 -O3 -march=x86-64-v3 -ffp-contract=off",
    })
    with tempfile.TemporaryDirectory() as tmp:
        for part in parts:
            manifest[MANIFEST_KEYS[part]] = PARTS[part](tmp)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
