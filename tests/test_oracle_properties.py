"""The oracle against what the mathematics fixes, independent of the golden
vectors: the closed forms and invariants the reference's own tests assert
(nm/tests/qwen35_tests.cpp:132-197, nm/tests/property_tests.cpp:137-239,
nm/tests/quant_tests.cpp:53-70), hand-worked attention cases, and float64
brute force of the delta rule and attention. Each check is chosen so that a
plausible slip in the restatement (a dropped term, a swapped operand, a wrong
index or sign) fails it."""
import numpy as np
import pytest

import oracle


def test_conv_step_closed_form():
    """taps [1, 10, 100] on two channels, width 3: y_t = x_{t-2} + 10 x_{t-1} + 100 x_t
    with zero history (qwen35_tests.cpp:132-155)"""
    taps = np.array([[1, 10, 100], [1, 10, 100]], np.float32)
    hist = np.zeros((2, 2), np.float32)
    ys = [oracle.conv_step(np.array([x, 0], np.float32), taps, hist)[0] for x in (1, 2, 3)]
    assert ys == [100.0, 210.0, 321.0]
    fresh = np.zeros((2, 2), np.float32)
    assert oracle.conv_step(np.array([1, 0], np.float32), taps, fresh)[0] == 100.0


def test_delta_rule_is_an_associative_memory():
    """Dk = Dv = 2 (qwen35_tests.cpp:157-186): beta 1 and gate 0 store v along a
    unit k, and a query at k reads v back; an orthogonal query reads nothing;
    gate -4 decays the stored value by exp(-4)."""
    k = np.array([1, 0], np.float32)
    v = np.array([3, -5], np.float32)
    state = np.zeros((1, 2, 2), np.float32)
    out = oracle.gated_delta_step(state, k, k, v, np.float32([0]), np.float32([1]), 1)
    assert np.allclose(out, [[3, -5]], atol=1e-6)
    ortho = np.array([0, 1], np.float32)
    miss = oracle.gated_delta_step(state, ortho, ortho, np.zeros(2, np.float32), np.float32([0]), np.float32([0]), 1)
    assert np.allclose(miss, 0, atol=1e-6)
    decaying = np.zeros((1, 2, 2), np.float32)
    oracle.gated_delta_step(decaying, k, k, v, np.float32([0]), np.float32([1]), 1)
    faded = oracle.gated_delta_step(decaying, k, k, np.zeros(2, np.float32), np.float32([-4]), np.float32([0]), 1)
    assert abs(faded[0, 0] - 3 * np.exp(-4.0)) < 1e-5


def delta_step_f64(S, q, k, v, g, beta):
    """the gated delta rule in float64: S <- exp(g) S; d = beta (v - S^T k);
    S <- S + k d^T; o = S^T q  (S is [Dk][Dv])"""
    S *= np.exp(g)
    d = beta * (v - S.T @ k)
    S += np.outer(k, d)
    return S.T @ q


@pytest.mark.parametrize("hk,hv", [(2, 2), (2, 4)])
def test_delta_rule_equals_float64_brute_force_with_tiled_key_heads(hk, hv):
    """12 tokens of 128x128 heads against float64; value head h uses key head
    h % hk (tiled, nm/src/qwen35.hpp:172), so a grouped mapping h // (hv/hk)
    fails the hk=2, hv=4 case"""
    rng = np.random.default_rng(5 + hv)
    dk = dv = 128
    state = np.zeros((hv, dk, dv), np.float32)
    ref = np.zeros((hv, dk, dv), np.float64)
    for _ in range(12):
        q = rng.standard_normal((hk, dk)).astype(np.float32)
        q /= np.linalg.norm(q, axis=1, keepdims=True) * np.sqrt(dk)
        k = rng.standard_normal((hk, dk)).astype(np.float32)
        k /= np.linalg.norm(k, axis=1, keepdims=True)
        v = rng.standard_normal((hv, dv)).astype(np.float32)
        g = -np.abs(rng.standard_normal(hv)).astype(np.float32)
        beta = rng.uniform(0, 1, hv).astype(np.float32)
        out = oracle.gated_delta_step(state, q.ravel(), k.ravel(), v.ravel(), g, beta, hk)
        for h in range(hv):
            kh = h % hk
            want = delta_step_f64(ref[h], q[kh].astype(np.float64), k[kh].astype(np.float64), v[h].astype(np.float64),
                                  float(g[h]), float(beta[h]))
            assert np.allclose(out[h], want, rtol=1e-4, atol=1e-5), f"head {h}"
    assert np.allclose(state, ref, rtol=1e-4, atol=1e-5)


def test_rope_offset_identity_and_position_zero():
    """(R(p) q) . (R(m) k) depends only on m - p (property_tests.cpp:137-152);
    position 0 is the identity; the unrotated planes (rotary 1/4 of 128) are
    untouched"""
    rng = np.random.default_rng(9)
    inv = oracle.rope_inv_freq(128, 1e6, 32)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    score = lambda p, m: float(np.dot(oracle.rope_apply(q, inv, p).astype(np.float64), oracle.rope_apply(k, inv, m)))  # noqa: E731
    a, b, c = score(3, 1), score(10, 8), score(1000, 998)
    assert abs(a - b) < 1e-3 and abs(b - c) < 1e-3
    assert np.array_equal(oracle.rope_apply(q, inv, 0), q)
    rot = oracle.rope_apply(q, inv, 777)
    untouched = np.r_[16:64, 80:128]  # planes (i, i + 64) rotate for i < 16 only
    assert np.array_equal(rot[untouched], q[untouched])
    assert not np.array_equal(rot[:16], q[:16])


def test_rmsnorm_scale_invariance_and_row_equals_batch():
    """n(x) == n(10 x) (property_tests.cpp:153-167); a matrix of rows is the row
    operation applied to each row (:168-186); the closed form gamma x / rms"""
    g = np.ones(4, np.float32)
    a = np.array([2, 4, 6, 8], np.float32)
    assert np.max(np.abs(oracle.rmsnorm(a, g) - oracle.rmsnorm(10 * a, g))) < 1e-5
    gamma = np.array([1, 2, 3, 4], np.float32)
    rows = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    batch = oracle.rmsnorm(rows, gamma)
    for r in range(2):
        assert np.array_equal(batch[r], oracle.rmsnorm(rows[r], gamma))
    x = np.random.default_rng(1).standard_normal(1024).astype(np.float32)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    assert np.allclose(oracle.rmsnorm(x, np.ones(1024, np.float32)), want, rtol=1e-5, atol=1e-6)


def test_attention_hand_worked_causal_and_window():
    """One K/V head of width 2 (property_tests.cpp:187-223): the query at
    position 0 sees key 0 only; at position 1 both keys with weights from
    softmax(scale q.k); a window of one keeps the current position only."""
    scale = np.float32(1 / np.sqrt(2.0))
    keys = np.array([[1, 0], [0, 1]], np.float32)
    vals = np.array([[10, 0], [30, 0]], np.float32)
    q0, q1 = np.array([1, 0], np.float32), np.array([0, 1], np.float32)
    assert oracle.attend_decode(q0, keys[:1], vals[:1], 1, 1, 2, 0, scale)[0, 0] == 10.0
    w1 = np.exp(scale) / (1 + np.exp(scale))
    got = oracle.attend_decode(q1, keys, vals, 1, 1, 2, 0, scale)[0, 0]
    assert abs(got - ((1 - w1) * 10 + w1 * 30)) < 1e-5
    assert oracle.attend_decode(q1, keys, vals, 1, 1, 2, 1, scale)[0, 0] == 30.0


@pytest.mark.parametrize("window", [0, 1, 5, 64])
def test_attention_equals_float64_brute_force_with_grouped_kv_heads(window):
    """8 query heads over 2 K/V heads (head h reads K/V head h // 4, grouped,
    nm/src/qwen35.hpp:369), 200 keys, against softmax in float64 over the
    positions [t - W + 1, t]"""
    rng = np.random.default_rng(window)
    hq, hkv, dh, ctx = 8, 2, 16, 200
    q = rng.standard_normal(hq * dh).astype(np.float32)
    keys = rng.standard_normal((ctx, hkv * dh)).astype(np.float32)
    vals = rng.standard_normal((ctx, hkv * dh)).astype(np.float32)
    scale = np.float32(0.25)
    got = oracle.attend_decode(q, keys, vals, hq, hkv, dh, window, scale)
    lo = 0 if window == 0 else max(0, ctx - window)
    for h in range(hq):
        g = h // (hq // hkv)
        kk = keys[lo:, g * dh:(g + 1) * dh].astype(np.float64)
        vv = vals[lo:, g * dh:(g + 1) * dh].astype(np.float64)
        s = float(scale) * (kk @ q[h * dh:(h + 1) * dh].astype(np.float64))
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(got[h], p @ vv, rtol=1e-4, atol=1e-5), f"head {h}"


def test_softmax_sums_to_one_and_activations_special_values():
    s = oracle.softmax(np.random.default_rng(2).standard_normal(50).astype(np.float32) * 3)
    assert abs(float(np.sum(s, dtype=np.float64)) - 1) < 1e-5
    assert abs(oracle.softplus(np.float32([0]))[0] - np.log(2)) < 1e-6
    assert oracle.softplus(np.float32([60]))[0] == 60.0  # saturates, never inf
    assert np.allclose(oracle.l2_normalize(np.float32([3, 4])), [0.6, 0.8], atol=1e-6)


def test_weight_quantizer_round_trip_within_one_quantum():
    """|q| <= 127, the block maximum maps to +-127, a zero block gives d = 0 and
    q = 0, and dequantization is within half a step of the input
    (quant_tests.cpp:56-70)"""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(64 * 32) * np.repeat(np.exp(rng.uniform(-6, 3, 64)), 32)).astype(np.float32)
    x[:32] = 0
    blocks = oracle.quantize_q8_0(x)
    q = blocks["qs"].astype(np.int32)
    d = oracle.fp16_to_fp32(blocks["d"])
    assert np.all(np.abs(q) <= 127)
    assert d[0] == 0 and np.all(q[0] == 0)
    xb = x.reshape(64, 32)
    peak = np.argmax(np.abs(xb), axis=1)
    assert np.all(np.abs(q[np.arange(1, 64), peak[1:]]) == 127)
    step = np.abs(xb).max(axis=1) / 127  # the fp32 scale before fp16 rounding
    err = np.abs(q * d[:, None].astype(np.float64) - xb)
    assert np.all(err <= 0.5 * step[:, None] + 127 * np.abs(d - step)[:, None] + 1e-12)
