"""Pin the oracle to the REFERENCE: every kernel case and the whole tiny Q8_0
model must match the golden vectors that the compiled reference engine wrote
(tests/golden/make_golden.py), bit for bit."""
import numpy as np
import pytest

import oracle


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fp16_encoder_matches_reference(kernels_golden):
    x = kernels_golden["in_fp16_encode"]
    assert np.array_equal(oracle.fp32_to_fp16(x), kernels_golden["out_fp16_encode"])


def test_activation_and_weight_quantizers_match_reference(kernels_golden):
    x = kernels_golden["in_quant"]
    assert oracle.quantize_row_q8_0(x).tobytes() == kernels_golden["out_quant_act"].tobytes()
    assert oracle.quantize_q8_0(x).tobytes() == kernels_golden["out_quant_weight"].tobytes()


def test_matvec_and_matmul_match_reference(kernels_golden):
    wq = kernels_golden["out_gemv_wq"].view(oracle.BLOCK)
    x = kernels_golden["in_gemv_x"].reshape(8, 4096)
    y = oracle.matvec(wq, 64, 4096, x[0])
    assert np.array_equal(bits(y), bits(kernels_golden["out_gemv_y"]))
    Y = oracle.matmul(wq, 64, 4096, x)
    assert np.array_equal(bits(Y).ravel(), bits(kernels_golden["out_gemm_y"]))


def test_q8_K_quantizer_matches_reference(kernels_golden):
    """zero block, a negative maximum (twice), exact .5 ties at scale 1, equal
    magnitudes of both signs (the first sets the sign) in row 1"""
    x = kernels_golden["in_kq_x"].reshape(4, 4096)
    got = np.concatenate([oracle.quantize_row_q8_K(x[r]) for r in range(4)])
    assert got.tobytes() == kernels_golden["out_kq_act"].tobytes()
    blocks = got.reshape(4, 16, 292)
    assert not blocks[1, 0].any()                                   # the zero block
    assert blocks[1, 1, 4 + 7].view(np.int8) == -127                # first element of largest magnitude
    assert blocks[1, 3, 4 + 10].view(np.int8) == -127 and blocks[1, 3, 4 + 20].view(np.int8) == 127


@pytest.mark.parametrize("wtype,name", [(oracle.Q4_K, "kq_w4"), (oracle.Q6_K, "kq_w6")])
def test_kquant_matvec_and_matmul_match_reference(kernels_golden, wtype, name):
    w = kernels_golden[f"in_{name}"]
    x = kernels_golden["in_kq_x"].reshape(4, 4096)
    expect = kernels_golden["out_kq_y" + ("4" if wtype == oracle.Q4_K else "6")].reshape(5, 64)
    Y = oracle.matmul_kquant(wtype, w, 64, 4096, x)
    assert np.array_equal(bits(Y[0]), bits(expect[0]))   # Weight::matvec
    assert np.array_equal(bits(Y), bits(expect[1:]))     # Weight::matmul, 4 rows


def test_kquant_dots_equal_dequantized_sums_in_exact_arithmetic(kernels_golden):
    """Independent of the reference: decode the K-quant weights from their
    bit layout (ggml's published block formats) and the Q8_K activation, form
    the exact dot in float64 from the same per-block fp32 scales, and compare
    with the oracle's fp32 dot to a rounding bound. A wrong nibble, high-bit
    shift, scale or min index moves the result far outside it."""
    x = kernels_golden["in_kq_x"].reshape(4, 4096)[2]
    act = oracle.quantize_row_q8_K(x)
    ad = act[:, :4].copy().view(np.float32).ravel()
    aq = act[:, 4:260].view(np.int8).astype(np.int64)
    f16 = lambda b: b.copy().view(np.float16).astype(np.float32)  # noqa: E731
    for wtype, name in [(oracle.Q4_K, "kq_w4"), (oracle.Q6_K, "kq_w6")]:
        w = kernels_golden[f"in_{name}"].reshape(64, 16, -1)
        for row in range(0, 64, 9):
            exact = 0.0
            for b in range(16):
                blk = w[row, b]
                if wtype == oracle.Q4_K:
                    d, dmin = f16(blk[0:2])[0], f16(blk[2:4])[0]
                    sc_bytes, qs = blk[4:16].astype(np.int64), blk[16:144].astype(np.int64)
                    sc = [(sc_bytes[j] & 63) if j < 4 else ((sc_bytes[j + 4] & 15) | ((sc_bytes[j - 4] >> 6) << 4)) for j in range(8)]
                    mn = [(sc_bytes[j + 4] & 63) if j < 4 else ((sc_bytes[j + 4] >> 4) | ((sc_bytes[j] >> 6) << 4)) for j in range(8)]
                    q = np.concatenate([np.concatenate([qs[32 * c:32 * c + 32] & 15, qs[32 * c:32 * c + 32] >> 4]) for c in range(4)])
                    scale = np.repeat(sc, 32)
                    mins = np.repeat(mn, 32)
                    dd, dm = np.float32(d * ad[b]), np.float32(dmin * ad[b])
                    exact += float(dd) * float((scale * q * aq[b]).sum()) - float(dm) * float((mins * aq[b]).sum())
                else:
                    ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
                    sc = blk[192:208].view(np.int8).astype(np.int64)
                    d = f16(blk[208:210])[0]
                    q = np.empty(256, np.int64)
                    for h in range(2):
                        for e in range(128):
                            low = ql[64 * h + e % 64] & 15 if e < 64 else ql[64 * h + e % 64] >> 4
                            q[128 * h + e] = (low | (((qh[32 * h + e % 32] >> (2 * (e // 32))) & 3) << 4)) - 32
                    exact += float(np.float32(d * ad[b])) * float((np.repeat(sc, 16) * q * aq[b]).sum())
            got = float(oracle.vec_dot_kquant(wtype, w[row].ravel(), act))
            scale_sum = sum(abs(float(v)) for v in [exact]) + 1e-30
            assert abs(got - exact) <= 1e-5 * max(scale_sum, 1.0), (name, row, got, exact)


def test_q5_K_fp32_matvec_and_matmul_match_reference(kernels_golden):
    """Q5_K has no integer-activation kernel: Weight::matvec / ::matmul take the
    fp32 dequant-in-dot form (nm/src/quant.hpp:207-229)"""
    w = kernels_golden["in_kq_w5"]
    x = kernels_golden["in_kq_x"].reshape(4, 4096)
    expect = kernels_golden["out_kq_y5"].reshape(5, 64)
    Y = oracle.linear(oracle.Q5_K, w, 64, 4096, x)
    assert np.array_equal(bits(Y[0]), bits(expect[0]))
    assert np.array_equal(bits(Y), bits(expect[1:]))


@pytest.mark.parametrize("wtype,name", [(oracle.Q4_K, "kq_w4"), (oracle.Q5_K, "kq_w5"), (oracle.Q6_K, "kq_w6")])
def test_kquant_dequant_rows_match_reference(kernels_golden, wtype, name):
    """Weight::dequant_row (the embedding gather) of rows 0 and 37 of random-byte blocks"""
    w = kernels_golden[f"in_{name}"].reshape(64, -1)
    got = np.concatenate([oracle.dequant_rows(wtype, w[r], 1, 4096).ravel() for r in (0, 37)])
    expect = kernels_golden["out_kq_dq" + {oracle.Q4_K: "4", oracle.Q5_K: "5", oracle.Q6_K: "6"}[wtype]]
    assert np.array_equal(bits(got), bits(expect))


def test_q5_K_dot_equals_dequantized_sum_in_float64(kernels_golden):
    """Independent of the reference: the Q5_K fields decoded from ggml's layout
    (fifth bit j of qh[l] for element l of sub-block j) against the oracle's
    fp32 dot, to a rounding bound. A wrong qh bit, nibble or scale index moves
    the result far outside it."""
    x = kernels_golden["in_kq_x"].reshape(4, 4096)[3].astype(np.float64)
    w = kernels_golden["in_kq_w5"].reshape(64, 16, 176)
    f16 = lambda b: float(b.copy().view(np.float16)[0])  # noqa: E731
    for row in range(0, 64, 7):
        exact, mag, block0 = 0.0, 0.0, None
        for b in range(16):
            blk = w[row, b]
            d, dmin = f16(blk[0:2]), f16(blk[2:4])
            sb, qh, qs = blk[4:16].astype(np.int64), blk[16:48].astype(np.int64), blk[48:176].astype(np.int64)
            for j in range(8):
                sc = (sb[j] & 63) if j < 4 else ((sb[j + 4] & 15) | ((sb[j - 4] >> 6) << 4))
                mn = (sb[j + 4] & 63) if j < 4 else ((sb[j + 4] >> 4) | ((sb[j] >> 6) << 4))
                nib = qs[32 * (j // 2):32 * (j // 2) + 32]
                q = (nib & 15 if j % 2 == 0 else nib >> 4) + ((qh >> j) & 1) * 16
                wv = d * sc * q - dmin * mn
                xs = x[256 * b + 32 * j:256 * b + 32 * j + 32]
                exact += float((wv * xs).sum())
                mag += float(np.abs(wv * xs).sum())
            if b == 0:
                block0 = (exact, mag)
        got0 = float(oracle.dot_block_q5_K(w[row, 0], x[:256].astype(np.float32)))  # one block
        assert abs(got0 - block0[0]) <= 4e-6 * block0[1], (row, got0, block0)
        got = float(oracle.linear(oracle.Q5_K, w[row].ravel(), 1, 4096, x.astype(np.float32))[0, 0])  # the row
        assert abs(got - exact) <= 4e-6 * mag, (row, got, exact, mag)


SAMPLER_CFGS = [(0.7, 40, 0.9), (1.0, 1, 1.0), (1.3, 1000, 0.95), (0.5, 0, 1.0), (2.0, 200, 0.5), (0.9, 64, 0.0)]


def test_sampler_matches_reference(kernels_golden):
    """Logits<32000>::sample over 8 rows x 6 configurations (top_k 0 = the
    whole vocabulary, top_p 0 = the first candidate), given the uniform draw
    the reference's generator made"""
    lg = kernels_golden["in_sample_logits"].reshape(8, 32000)
    res = kernels_golden["out_sample"].reshape(8, len(SAMPLER_CFGS), 2)
    for r in range(8):
        for c, (temp, k, p) in enumerate(SAMPLER_CFGS):
            assert oracle.sample_topk(lg[r], k, temp, p, res[r, c, 1]) == int(res[r, c, 0]), (r, c)


def test_sampler_limits():
    """closed forms: top_k 1 and top_p 0 are greedy; u -> 0 picks the first
    kept candidate; a large temperature spreads the draw over the kept set"""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(5000).astype(np.float32)
    best = int(np.argmax(x))
    assert oracle.sample_topk(x, 1, 0.8, 1.0, 0.99) == best
    assert oracle.sample_topk(x, 50, 0.8, 0.0, 0.99) == best
    assert oracle.sample_topk(x, 50, 0.8, 1.0, 0.0) == best
    top = set(np.argsort(-x, kind="stable")[:10].tolist())
    picks = {oracle.sample_topk(x, 10, 1e6, 1.0, u) for u in np.linspace(0, 0.999, 40)}
    assert picks == top


@pytest.mark.parametrize("n", [128, 1024, 4096])
def test_rmsnorm_matches_reference(kernels_golden, n):
    v = kernels_golden[f"in_rms{n}"]
    y = oracle.rmsnorm(v[:n], v[n:])
    assert np.array_equal(bits(y), bits(kernels_golden[f"out_rms{n}"]))


def test_l2_normalize_matches_reference(kernels_golden):
    x = kernels_golden["in_l2"].reshape(16, 128)
    y = np.concatenate([oracle.l2_normalize(r) for r in x])
    assert np.array_equal(bits(y), bits(kernels_golden["out_l2"]))


@pytest.mark.parametrize("name", ["silu", "sigmoid", "softplus"])
def test_scalar_activations_match_reference(kernels_golden, name):
    x = kernels_golden["in_act"]
    y = getattr(oracle, name)(x)
    assert np.array_equal(bits(y), bits(kernels_golden[f"out_{name}"]))


def test_conv_steps_match_reference(kernels_golden):
    taps = kernels_golden["in_conv_taps"].reshape(256, 4)
    xs = kernels_golden["in_conv_x"].reshape(6, 256)
    hist = np.zeros((3, 256), np.float32)
    y = np.concatenate([oracle.conv_step(x, taps, hist) for x in xs])
    assert np.array_equal(bits(y), bits(kernels_golden["out_conv"]))


def test_gated_delta_steps_match_reference(kernels_golden):
    state = kernels_golden["in_delta_state"].reshape(1, 128, 128).copy()
    tok = kernels_golden["in_delta_tok"].reshape(4, 386)
    outs = [oracle.gated_delta_step(state, t[:128], t[128:256], t[256:384], t[384:385], t[385:386], 1) for t in tok]
    assert np.array_equal(bits(np.concatenate(outs).ravel()), bits(kernels_golden["out_delta_out"]))
    assert np.array_equal(bits(state.ravel()), bits(kernels_golden["out_delta_state"]))


def test_rope_matches_reference(kernels_golden):
    x = kernels_golden["in_rope"].reshape(8, 128)
    inv = oracle.rope_inv_freq(128, 1e6, 32)
    positions = [0, 1, 2, 7, 100, 1023, 4095, 65535]
    y = np.concatenate([oracle.rope_apply(r, inv, p) for r, p in zip(x, positions)])
    assert np.array_equal(bits(y), bits(kernels_golden["out_rope"]))


@pytest.mark.parametrize("name,scale", [("attn_scaled", np.float32(1.0) / np.sqrt(np.float32(128.0))), ("attn_unit", 1.0)])
def test_attention_reduction_matches_reference(kernels_golden, name, scale):
    q = kernels_golden["in_attn_q"]
    k = kernels_golden["in_attn_k"].reshape(-1, 128)
    v = kernels_golden["in_attn_v"].reshape(-1, 128)
    out = oracle.attend_decode(q, k, v, 1, 1, 128, 0, np.float32(scale))
    assert np.array_equal(bits(out.ravel()), bits(kernels_golden[f"out_{name}"]))


@pytest.fixture(scope="module")
def tiny_run(tiny_gguf, tiny_golden):
    m = oracle.Model(path=tiny_gguf)
    oracle.set_threads(4)
    prompt = tiny_golden["prompt"]
    steps = len(tiny_golden["ids"]) - 1
    logits_prefill = m.forward_ids(prompt)
    ids = [oracle.argmax(logits_prefill)]
    mid = None
    for i in range(steps):
        logits = m.forward_ids([ids[-1]])
        ids.append(oracle.argmax(logits))
        if i + 1 == steps // 2:
            mid = logits.copy()
    return dict(ids=np.array(ids, np.int32), prefill=logits_prefill, mid=mid, last=logits)


def oracle_argmax(logits):
    return int(oracle.lib.oracle_argmax(logits.ctypes.data, logits.size))


oracle.argmax = oracle_argmax


def test_tiny_model_greedy_ids_match_reference(tiny_run, tiny_golden):
    assert np.array_equal(tiny_run["ids"], tiny_golden["ids"])


@pytest.mark.parametrize("which", ["prefill", "mid", "last"])
def test_tiny_model_logits_match_reference_bitwise(tiny_run, tiny_golden, which):
    assert np.array_equal(bits(tiny_run[which]), bits(tiny_golden[f"logits_{which}"]))


def test_fp16_decoder_is_ieee_half_on_all_inputs():
    """nm/src/core.hpp:34-59 decodes IEEE binary16 exactly: all 65536 codes
    against numpy's float16 -> float32 conversion, bit for bit."""
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _fp16_nearest_ties_away(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits: round to nearest, ties away from zero, overflow and
    NaN to signed infinity -- the rule of nm/src/core.hpp:61-79, computed here
    from the fp16 grid in float64 rather than from the bits."""
    x = np.asarray(x, np.float32)
    sign = (x.view(np.uint32) >> 16).astype(np.uint16) & np.uint16(0x8000)
    v = np.abs(x.astype(np.float64))
    with np.errstate(over="ignore", invalid="ignore"):
        h = v.astype(np.float16)  # nearest-even, used only to find the neighbours
        lo = np.where(h.astype(np.float64) <= v, h, np.nextafter(h, np.float16(-np.inf)))
        lo = np.where(np.isinf(lo), np.float16(65504.0), lo)
        hi = np.nextafter(lo, np.float16(np.inf))
        hi_val = np.where(np.isinf(hi), 65536.0, hi.astype(np.float64))
        d_lo = v - lo.astype(np.float64)
        d_hi = hi_val - v
        pick = np.where(d_hi <= d_lo, hi, lo)
    bits = pick.view(np.uint16)
    bits = np.where(np.isnan(x), np.uint16(0x7C00), bits)
    return (bits | sign).astype(np.uint16)


def test_fp16_encoder_is_nearest_ties_away():
    """The encoder against a closed form on 2^21 random fp32 patterns plus every
    fp16 midpoint (the ties), zeros, infinities and NaN."""
    rng = np.random.default_rng(11)
    rand = rng.integers(0, 2**32, 1 << 21, dtype=np.uint64).astype(np.uint32).view(np.float32)
    grid = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)  # exact in fp32
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65519.99, 65520.0, 2.0**-25, 2.0**-26, 3 * 2.0**-26], np.float32)
    x = np.concatenate([rand, mids, -mids, special])
    got = oracle.fp32_to_fp16(x)
    want = _fp16_nearest_ties_away(x)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(float(x[i]), hex(int(got[i])), hex(int(want[i]))) for i in bad[:5]]


def test_fp16_cache_rounding_is_ieee_nearest_even():
    """The oracle's fp16 cache rounding (F16C) equals numpy's IEEE binary16
    conversion: normals at every scale, subnormals, exact midpoints (ties to
    even), the overflow edge, signed zeros and infinities."""
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 100000).astype(np.float32),
        (np.arange(0, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),   # subnormal midpoints
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),  # normal midpoints in [1, 2)
        np.array([65504, 65519.99, 65520, 7e4, -65520, 0.0, -0.0, np.inf, -np.inf, 6e-8, 2.9e-8, 3.0e-8], np.float32),
    ]).astype(np.float32)
    want = x.astype(np.float16).astype(np.float32)
    got = oracle.round_fp16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- causal and sliding-window visibility (CausalWindow / LocalAttentionCache) ----------
WINDOW_CASES = [("window_full", 0, np.float32(1.0) / np.sqrt(np.float32(128.0))), ("window_w3", 3, np.float32(1.0)),
                ("window_w1024", 1024, np.float32(1.0))]


@pytest.mark.parametrize("name,window,scale", WINDOW_CASES)
def test_window_attention_matches_reference(window_golden, name, window, scale):
    """The oracle's attention over positions 0..t with a window, against the
    reference's own caches (a full append-only cache; rings of 3 and 1024 rows
    that evict) at probes before, at and after the ring fills: bit for bit."""
    k, v, q = window_golden["k"], window_golden["v"], window_golden["q"]
    for i, t in enumerate(window_golden["probes"]):
        out = oracle.attend_decode(q[t], k[: t + 1], v[: t + 1], 4, 2, 128, window, scale)
        assert np.array_equal(bits(out.ravel()), bits(window_golden[name][i])), f"{name} probe {t}"


@pytest.mark.parametrize("name,window", [(c[0], c[1]) for c in WINDOW_CASES])
def test_window_visible_positions_follow_the_reference_rule(window_golden, name, window):
    """The reference's visible rows, mapped back to positions, are the closed
    form the kernels and the oracle use: [max(0, t - W + 1), t] (all of 0..t
    without a window)."""
    for i, t in enumerate(window_golden["probes"]):
        first, end = window_golden[name + "_rows"][i]
        size = t + 1 if window == 0 else min(t + 1, window)  # rows the cache holds after appending position t
        oldest = t + 1 - size
        lo = 0 if window == 0 else max(0, t - window + 1)
        assert (oldest + first, oldest + end) == (lo, t + 1), f"{name} probe {t}"


# ---- Hk != Hv (tiled key heads) and an untied head -------------------------------------
def test_variant_model_matches_reference(variant_gguf, variant_golden):
    """4 key heads tiled over 8 value heads (value head h reads key head h % 4,
    nm/src/qwen35.hpp:172) and a separate output.weight: the oracle's greedy
    ids and its prefill / last logits equal the reference's bit for bit."""
    m = oracle.Model(path=variant_gguf)
    assert (m.Hk, m.Hv, m.tied) == (4, 8, 0)
    prompt = variant_golden["prompt"]
    prefill = m.forward_ids(prompt)
    assert np.array_equal(bits(prefill), bits(variant_golden["logits_prefill"]))
    ids = [oracle.argmax(prefill)]
    for _ in range(len(variant_golden["ids"]) - 1):
        last = m.forward_ids([ids[-1]])
        ids.append(oracle.argmax(last))
    assert np.array_equal(np.array(ids, np.int32), variant_golden["ids"])
    assert np.array_equal(bits(last), bits(variant_golden["logits_last"]))
    m.close()


# ---- 256-wide attention heads (the reference's Qwen 3.5 4B / 9B geometry) ---------------
def test_dh256_model_matches_reference(dh256_gguf, dh256_golden):
    """8 query / 2 K/V heads of 256 channels (Hq * Dh = 2048 != D = 1024),
    rope.dimension_count 64 (partial rotary), RoPE base 1e7, 4 key heads over
    8 value heads and an untied head: the oracle's greedy ids and its prefill /
    last logits equal the reference's bit for bit."""
    m = oracle.Model(path=dh256_gguf)
    prompt = dh256_golden["prompt"]
    prefill = m.forward_ids(prompt)
    assert np.array_equal(bits(prefill), bits(dh256_golden["logits_prefill"]))
    ids = [oracle.argmax(prefill)]
    for _ in range(len(dh256_golden["ids"]) - 1):
        last = m.forward_ids([ids[-1]])
        ids.append(oracle.argmax(last))
    assert np.array_equal(np.array(ids, np.int32), dh256_golden["ids"])
    assert np.array_equal(bits(last), bits(dh256_golden["logits_last"]))
    m.close()


# ---- K-quant tensors: the tensor types of a Q4_K_M checkpoint -----------------------
def test_kquant_model_matches_reference(kmix_gguf, kmix_golden):
    """The tiny shape with a Q6_K embedding (the tied head), Q5_K attn_qkv and
    attn_output (fp32-activation dots), Q6_K ffn_down and attn_v, Q8_0
    ssm_alpha / ssm_beta and Q4_K elsewhere: the oracle's greedy ids and its
    prefill / last logits equal the reference's bit for bit."""
    m = oracle.Model(path=kmix_gguf)
    prompt = kmix_golden["prompt"]
    prefill = m.forward_ids(prompt)
    assert np.array_equal(bits(prefill), bits(kmix_golden["logits_prefill"]))
    ids = [oracle.argmax(prefill)]
    for _ in range(len(kmix_golden["ids"]) - 1):
        last = m.forward_ids([ids[-1]])
        ids.append(oracle.argmax(last))
    assert np.array_equal(np.array(ids, np.int32), kmix_golden["ids"])
    assert np.array_equal(bits(last), bits(kmix_golden["logits_last"]))
    m.close()


def test_q8_ffn_mix_model_matches_reference(q8ffn_gguf, q8ffn_golden):
    """SwiGLU width 3584 with Q8_0 in-projections, gate and up beside a Q6_K
    embedding and down projection and Q4_K output projections: the oracle's
    greedy ids and its prefill / last logits equal the reference's bit for bit."""
    m = oracle.Model(path=q8ffn_gguf)
    prompt = q8ffn_golden["prompt"]
    prefill = m.forward_ids(prompt)
    assert np.array_equal(bits(prefill), bits(q8ffn_golden["logits_prefill"]))
    ids = [oracle.argmax(prefill)]
    for _ in range(len(q8ffn_golden["ids"]) - 1):
        last = m.forward_ids([ids[-1]])
        ids.append(oracle.argmax(last))
    assert np.array_equal(np.array(ids, np.int32), q8ffn_golden["ids"])
    assert np.array_equal(bits(last), bits(q8ffn_golden["logits_last"]))
    m.close()
