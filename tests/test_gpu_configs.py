"""The benchmark workloads at their own sizes, against the oracle.

* Q8_0 GEMV / GEMM: K=4096 with N in {4096, 12288, 151936} and K=12288 with
  N=4096, M in {1, 8, 24, 64, 512}: int8 weights uniform in [-127, 127], fp16
  scales |N(0, 0.02)| * 4/127, fp32 N(0, 1) activations quantized on the fly.
  Every kernel form the dispatcher can choose (two skinny forms, the tiled
  kernel at 16/32/64/128 rows per tile) is selected by at least one case.
* Gated delta-net: 16 heads of 128, one decode step for B in {1, 8, 32} from a
  non-zero state, and a 4096-token prefill in the chunked form (chunks of 64)
  against the token-serial form and the oracle's serial recurrence.
* GQA decode attention: 32 query / 8 KV heads of 128 at 1k, 8k and 32k context,
  B in {1, 16} (and 3, for the middle form of the weighted sum), full causal at
  scale 1/sqrt(128) and a sliding window of 1024 at scale 1, over the fp32 cache
  (bit for bit) and the paged fp16 cache (tolerance).

Bars: bit-exact for every integer / byte result and for every fp32 result of
the exact paths (the kernels replay the reference's fp32 operation order); the
chunked delta-net prefill and the paged fp16 attention reorder fp32 sums, and
their tolerances are stated in the tests.
"""
import os
import time

import numpy as np
import pytest

import oracle
from gpu_util import act_to_blocks, bits, check, dev, empty, gdn_reference, host, ptr, quantize_dev, stream, ulp_diff

pytestmark = pytest.mark.gpu

GEMM_SHAPES = [(4096, 4096), (4096, 12288), (4096, 151936), (12288, 4096)]  # (K, N)
GEMM_ROWS = [1, 8, 24, 64, 100, 512]
PLAN_NAMES = {1: "skinny-wave", 2: "skinny-shared", 3: "skinny-lds", 4: "skinny-wave4", 16: "tile16", 32: "tile32", 64: "tile64", 128: "tile128"}


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def lib():
    import torch

    from hero_amd._lib import lib as _lib

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    oracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    return _lib


def gemm_plan(lib, m, n, k):
    import ctypes

    out = ctypes.c_int32()
    check(lib.hero_q8_0_gemm_plan(m, n, k, ctypes.byref(out)))
    return out.value


def test_gemm_shapes_reach_every_kernel_form(lib):
    """the (M, K, N) cases below select every form of hero_q8_0_gemm"""
    seen = {gemm_plan(lib, m, n, k) for (k, n) in GEMM_SHAPES for m in GEMM_ROWS if m > 1}
    say("GEMM forms: " + ", ".join(sorted(PLAN_NAMES[p] for p in seen)))
    assert seen == set(PLAN_NAMES), f"forms not reached: {set(PLAN_NAMES) - seen}"


def microbench_weight(rng, n, k):
    """int8 uniform in [-127, 127] per 32-block with fp16 scale |N(0,0.02)|*4/127"""
    blocks = np.zeros((n, k // 32), oracle.BLOCK)
    blocks["qs"] = rng.integers(-127, 128, size=(n, k // 32, 32), dtype=np.int8)
    scale = (np.abs(rng.standard_normal((n, k // 32), dtype=np.float32)) * np.float32(0.02 * 4 / 127)).astype(np.float32)
    blocks["d"] = oracle.fp32_to_fp16(scale)
    return blocks


@pytest.mark.timeout(900)
@pytest.mark.parametrize("k,n", GEMM_SHAPES)
def test_gemv_gemm_baseline_shapes_match_oracle_bitwise(lib, k, n):
    """Every M of the microbenchmark on one (K, N): the M=1 streaming GEMV and
    the GEMM forms against Weight::matvec / ::matmul restated, bit for bit."""
    from hero_amd._lib import check as _check

    rng = np.random.default_rng(k * 7 + n)
    t0 = time.perf_counter()
    w = microbench_weight(rng, n, k)
    src = dev(w)
    packed = empty(lib.hero_q8_0_packed_bytes(n, k))
    _check(lib.hero_q8_0_pack(ptr(src), ptr(packed), n, k, 0, n, stream()))
    del src
    say(f"[gemm K={k} N={n}] weights ready in {time.perf_counter() - t0:.1f} s")
    for m in GEMM_ROWS:
        x = rng.standard_normal((m, k), dtype=np.float32)
        act = quantize_dev(lib, x)
        y = empty(m * n * 4)
        if m == 1:
            _check(lib.hero_q8_0_gemv(ptr(packed), ptr(act), ptr(y), None, n, k, stream()))
            form = "gemv"
        else:
            _check(lib.hero_q8_0_gemm(ptr(packed), ptr(act), ptr(y), None, m, n, k, stream()))
            form = PLAN_NAMES[gemm_plan(lib, m, n, k)]
        got = host(y, np.float32, (m, n))
        t = time.perf_counter()
        want = oracle.matmul(w, n, k, x)
        same = bits(got) == bits(want)
        say(f"[gemm K={k} N={n}] M={m} {form}: exact {same.mean():.6f} (oracle {time.perf_counter() - t:.1f} s)")
        assert same.all(), f"M={m} ({form}): {np.count_nonzero(~same)} outputs differ, max ulp {ulp_diff(got, want).max()}"


# ---- gated delta-net, 16 heads -----------------------------------------------------------
GDN_H, GDN_DK, GDN_W = 16, 128, 4


def gdn_params(rng, hk, hv):
    cc = 2 * hk * GDN_DK + hv * GDN_DK
    return dict(
        taps=(rng.standard_normal((cc, GDN_W)) * 0.5).astype(np.float32),
        dt=(rng.standard_normal(hv) * 0.1).astype(np.float32),
        decay=(-np.exp(rng.standard_normal(hv) * 0.5)).astype(np.float32),
        gamma=(1 + 0.1 * rng.standard_normal(GDN_DK)).astype(np.float32),
    )


@pytest.mark.timeout(600)
@pytest.mark.parametrize("B", [1, 8, 32])
def test_gdn_decode_16_heads_matches_oracle(lib, B):
    """One decode step of B sequences from a non-zero state and conv ring
    (position 64: the ring holds positions 61-63), all 16 heads: output,
    quantized output and the new state bit for bit."""
    from hero_amd._lib import GdnDecodeArgs

    rng = np.random.default_rng(1000 + B)
    hk = hv = GDN_H
    dk = GDN_DK
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    p = gdn_params(rng, hk, hv)
    eps = np.float32(1e-6)
    pos = 64
    state0 = (rng.standard_normal((B, hv, dk, dk), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    ring = (rng.standard_normal((B, GDN_W, cc), dtype=np.float32) * np.float32(0.7)).astype(np.float32)
    proj = (rng.standard_normal((B, stride), dtype=np.float32) * np.float32(0.7)).astype(np.float32)
    d_taps, d_dt, d_decay, d_gamma = dev(p["taps"]), dev(p["dt"]), dev(p["decay"]), dev(p["gamma"])
    d_hist, d_state = dev(ring), dev(state0)
    d_proj, d_pos = dev(proj), dev(np.full(B, pos, np.int32))
    act = empty(lib.hero_q8_0_act_bytes(B, hv * dk))
    out = empty(B * hv * dk * 4)
    a = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + hv * dk, cc + hv * dk + hv, ptr(d_taps), ptr(d_hist), ptr(d_state),
                      ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(act), ptr(out), B, hk, hv, dk, dk, GDN_W)
    check(lib.hero_gdn_decode(a, stream()))
    got = host(out, np.float32, (B, hv * dk))
    gstate = host(d_state, np.float32, (B, hv, dk, dk))
    blocks = act_to_blocks(host(act, np.uint8), B, hv * dk)
    for b in range(B):
        hist = np.stack([ring[b, (pos - GDN_W + 1 + i) % GDN_W] for i in range(GDN_W - 1)])  # oldest first
        st = state0[b].copy()
        expect = gdn_reference(proj[b], p["taps"], hist, st, p["dt"], p["decay"], p["gamma"], eps, hk, hv, pos)
        assert np.array_equal(bits(got[b]), bits(expect)), f"seq {b}: max ulp {ulp_diff(got[b], expect).max()}"
        assert blocks[b].tobytes() == oracle.quantize_row_q8_0(expect).tobytes(), f"seq {b} quantized output"
        assert np.array_equal(bits(gstate[b]), bits(st)), f"seq {b} state"
    say(f"[gdn decode H=16 B={B}] output, quantized output and state bit-exact")
    # the column-split form from the same state: raw outputs, then the head
    # norm + gate + quantize kernel; everything equal bit for bit
    d_hist2, d_state2 = dev(ring), dev(state0)
    o_raw, act2, out2 = empty(B * hv * dk * 4), empty(lib.hero_q8_0_act_bytes(B, hv * dk)), empty(B * hv * dk * 4)
    a2 = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + hv * dk, cc + hv * dk + hv, ptr(d_taps), ptr(d_hist2), ptr(d_state2),
                       ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(act2), ptr(out2), B, hk, hv, dk, dk, GDN_W)
    check(lib.hero_gdn_decode_cols(a2, ptr(o_raw), None, stream()))
    check(lib.hero_gdn_norm_gate(ptr(o_raw), a2, stream()))
    assert np.array_equal(bits(host(out2, np.float32, (B, hv * dk))), bits(got))
    assert np.array_equal(host(act2, np.uint8), host(act, np.uint8))
    assert np.array_equal(bits(host(d_state2, np.float32, (B, hv, dk, dk))), bits(gstate))
    assert np.array_equal(host(d_hist2, np.uint8), host(d_hist, np.uint8))
    say(f"[gdn decode H=16 B={B}] column-split form: the same outputs, state and ring")


@pytest.mark.timeout(900)
def test_gdn_chunked_prefill_4096_tokens(lib):
    """The 4096-token prefill of one sequence (16 heads, zero initial state) in
    the chunked form (64 chunks of 64 tokens) against the token-serial form,
    which must equal the oracle's serial recurrence bit for bit.

    Stated bound for the chunked form (a reordering of fp32 sums inside each
    chunk, carried across 64 chunks): every output and final-state value within
    rtol 1e-3 + atol 1e-4 * max|value| of the serial result."""
    from hero_amd._lib import GdnDecodeArgs

    rng = np.random.default_rng(4096)
    T, hk, hv, dk = 4096, GDN_H, GDN_H, GDN_DK
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    p = gdn_params(rng, hk, hv)
    eps = np.float32(1e-6)
    proj = (rng.standard_normal((T, stride), dtype=np.float32) * np.float32(0.7)).astype(np.float32)
    d_taps, d_dt, d_decay, d_gamma = dev(p["taps"]), dev(p["dt"]), dev(p["decay"]), dev(p["gamma"])
    d_proj, d_pos = dev(proj), dev(np.array([0], np.int32))
    wbytes = lib.hero_gdn_prefill_work_bytes(T, hk, hv)
    results = {}
    for name, fn in (("serial", lib.hero_gdn_prefill), ("chunked", lib.hero_gdn_prefill_chunked)):
        d_hist, d_state = empty(GDN_W * cc * 4), empty(hv * dk * dk * 4)
        work, act, out = empty(wbytes), empty(lib.hero_q8_0_act_bytes(T, hv * dk)), empty(T * hv * dk * 4)
        a = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + hv * dk, cc + hv * dk + hv, ptr(d_taps), ptr(d_hist), ptr(d_state),
                          ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(act), ptr(out), T, hk, hv, dk, dk, GDN_W)
        t = time.perf_counter()
        check(fn(a, ptr(work), wbytes, stream()))
        results[name] = (host(out, np.float32, (T, hv * dk)).copy(), host(d_state, np.float32, (hv, dk, dk)).copy())
        say(f"[gdn prefill T=4096] {name} form done in {time.perf_counter() - t:.2f} s")
    (o_ser, s_ser), (o_chk, s_chk) = results["serial"], results["chunked"]
    # the serial form against the oracle, token by token
    t = time.perf_counter()
    hist = np.zeros((GDN_W - 1, cc), np.float32)
    state = np.zeros((hv, dk, dk), np.float32)
    for i in range(T):
        expect = gdn_reference(proj[i], p["taps"], hist, state, p["dt"], p["decay"], p["gamma"], eps, hk, hv, i)
        assert np.array_equal(bits(o_ser[i]), bits(expect)), f"token {i}: max ulp {ulp_diff(o_ser[i], expect).max()}"
    assert np.array_equal(bits(s_ser), bits(state)), "final state"
    say(f"[gdn prefill T=4096] serial form equals the oracle bit for bit ({time.perf_counter() - t:.1f} s)")
    so, ss = np.abs(o_ser).max(), np.abs(s_ser).max()
    dev_o = np.abs(o_chk - o_ser).max() / so
    dev_s = np.abs(s_chk - s_ser).max() / ss
    say(f"[gdn prefill T=4096] chunked vs serial: max|d|/max = {dev_o:.3g} (outputs), {dev_s:.3g} (state)")
    np.testing.assert_allclose(o_chk, o_ser, rtol=1e-3, atol=1e-4 * so)
    np.testing.assert_allclose(s_chk, s_ser, rtol=1e-3, atol=1e-4 * ss)


# ---- GQA decode attention, 32 q / 8 kv heads -------------------------------------------------
ATT_HQ, ATT_HKV, ATT_DH = 32, 8, 128
VARIANTS = [(0, np.float32(1.0) / np.sqrt(np.float32(ATT_DH))), (1024, np.float32(1.0))]  # (window, score scale)


def attn_inputs(rng, B, ctx):
    """cached rows 0..ctx-2 (N(0,1)/sqrt(128)) and the projections of the token
    at position ctx-1, so that ctx keys are visible without a window"""
    kw = ATT_HKV * ATT_DH
    qw = ATT_HQ * ATT_DH
    s = np.float32(1.0 / np.sqrt(128.0))
    pos = ctx - 1
    keys = rng.standard_normal((B, pos, kw), dtype=np.float32) * s
    vals = rng.standard_normal((B, pos, kw), dtype=np.float32) * s
    proj = rng.standard_normal((B, 2 * qw + 2 * kw), dtype=np.float32) * s
    qg = (1 + 0.1 * rng.standard_normal(ATT_DH)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(ATT_DH)).astype(np.float32)
    return pos, keys, vals, proj, qg, kg


def attn_expect(proj_b, keys_b, vals_b, qg, kg, inv, pos, window, scale, fp16):
    """the oracle: q/k RMSNorm + RoPE, append, attend, sigmoid gate"""
    dh, hq, hkv = ATT_DH, ATT_HQ, ATT_HKV
    qw, kw = hq * dh, hkv * dh
    eps = np.float32(1e-6)
    q = np.stack([proj_b[h * 2 * dh: h * 2 * dh + dh] for h in range(hq)])
    g = np.concatenate([proj_b[h * 2 * dh + dh: h * 2 * dh + 2 * dh] for h in range(hq)])
    q = oracle.rope_apply(oracle.rmsnorm(q, qg, eps), inv, pos)
    k = oracle.rope_apply(oracle.rmsnorm(proj_b[2 * qw: 2 * qw + kw].reshape(hkv, dh), kg, eps), inv, pos).reshape(1, kw)
    v = proj_b[2 * qw + kw:].reshape(1, kw)
    if fp16:
        k, v = oracle.round_fp16(k), oracle.round_fp16(v)
    kk = np.concatenate([keys_b, k])
    vv = np.concatenate([vals_b, v])
    att = oracle.attend_decode(q.reshape(-1), kk, vv, hq, hkv, dh, window, scale).reshape(-1)
    return (att * oracle.sigmoid(g)).astype(np.float32)


# (1, 70000), (2, 66000): contexts past 65536 positions (the reference's CTX is 262144)
ATTN_CASES = [(1, 1024), (16, 1024), (1, 8192), (16, 8192), (1, 32768), (16, 32768), (3, 9000), (1, 70000), (2, 66000)]


@pytest.mark.timeout(900)
@pytest.mark.parametrize("B,ctx", ATTN_CASES)
def test_attn_baseline_sizes_match_oracle(lib, B, ctx):
    """32q/8kv attention decode at the benchmark's contexts, full causal
    (scale 1/sqrt(128)) and sliding window 1024 (scale 1):
    * fp32 cache: bit for bit against the oracle. Above 4096 visible keys the
      softmax total runs in 4095-key chunks; B=1 takes the fused softmax +
      weighted-sum pipeline up to 4096 keys, B=3 the shallow-ring weighted sum,
      B=16 the many-sequence form.
    * paged fp16 cache (pages of 64 positions in a shuffled pool): against the
      oracle over the same fp16-rounded K/V; the split-K merge reorders the
      softmax sums, so outputs agree within rtol 1e-4 + atol 1e-4 * max|out|,
      and the quantized output equals the quantization of the kernel's own
      fp32 output."""
    from hero_amd._lib import AttnDecodeArgs, AttnPagedArgs

    rng = np.random.default_rng(B * 100003 + ctx)
    dh, hq, hkv = ATT_DH, ATT_HQ, ATT_HKV
    qw, kw = hq * dh, hkv * dh
    t0 = time.perf_counter()
    pos, keys, vals, proj, qg, kg = attn_inputs(rng, B, ctx)
    inv = oracle.rope_inv_freq(dh, 1e6, 32)
    d_cs = dev(oracle.rope_table(dh, 1e6, 32, ctx))
    d_qg, d_kg = dev(qg), dev(kg)
    d_proj, d_pos = dev(proj), dev(np.full(B, pos, np.int32))
    stride = 2 * qw + 2 * kw
    eps = np.float32(1e-6)
    act = empty(lib.hero_q8_0_act_bytes(B, qw))
    out = empty(B * qw * 4)
    d_qr = empty(B * hq * dh * 4)
    # fp32 cache: K channel-major [B][Hkv][Dh][ctx], V [B][ctx][Hkv*Dh]
    kc = np.zeros((B, hkv, dh, ctx), np.float32)
    kc[:, :, :, :pos] = keys.reshape(B, pos, hkv, dh).transpose(0, 2, 3, 1)
    d_kc = dev(kc)
    del kc
    vc = np.zeros((B, ctx, kw), np.float32)
    vc[:, :pos] = vals
    d_vc = dev(vc)
    del vc
    d_sc = empty(B * hq * ctx * 4)
    say(f"[attn B={B} ctx={ctx}] inputs ready in {time.perf_counter() - t0:.1f} s")
    for window, scale in VARIANTS:
        a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), ptr(d_kc), ptr(d_vc),
                           ctx, ptr(d_pos), ptr(d_sc), ptr(d_qr), scale, window, ptr(act), ptr(out), B, hq, hkv, dh)
        check(lib.hero_attn_decode(a, stream()))
        got = host(out, np.float32, (B, qw))
        blocks = act_to_blocks(host(act, np.uint8), B, qw)
        for b in range(B):
            expect = attn_expect(proj[b], keys[b], vals[b], qg, kg, inv, pos, window, scale, False)
            assert np.array_equal(bits(got[b]), bits(expect)), f"fp32 window={window} seq {b}: max ulp {ulp_diff(got[b], expect).max()}"
            assert blocks[b].tobytes() == oracle.quantize_row_q8_0(expect).tobytes()
        say(f"[attn B={B} ctx={ctx}] fp32 cache, window={window}: bit-exact")
    del d_kc, d_vc, d_sc
    # paged fp16 cache
    page = 64
    max_pages = (ctx + page - 1) // page
    table = rng.permutation(B * max_pages).astype(np.int32).reshape(B, max_pages)
    pool = np.zeros((B * max_pages, 2, hkv, page, dh), np.float16)
    for which, src in ((0, keys), (1, vals)):
        padded = np.zeros((B, max_pages * page, hkv, dh), np.float16)
        padded[:, :pos] = src.reshape(B, pos, hkv, dh).astype(np.float16)
        pool[table.reshape(-1), which] = padded.reshape(B, max_pages, page, hkv, dh).transpose(0, 1, 3, 2, 4).reshape(B * max_pages, hkv, page, dh)
        del padded
    d_pages, d_table = dev(pool), dev(table)
    del pool
    keys16 = keys.astype(np.float16).astype(np.float32)
    vals16 = vals.astype(np.float16).astype(np.float32)
    for window, scale in VARIANTS:
        wbytes = lib.hero_attn_paged_work_bytes(max_pages * page, window, B, hq, hkv, dh)
        d_work = empty(wbytes)
        a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), None, None,
                           0, ptr(d_pos), None, ptr(d_qr), scale, window, ptr(act), ptr(out), B, hq, hkv, dh)
        pa = AttnPagedArgs(a, ptr(d_pages), ptr(d_table), page, max_pages, ptr(d_work), wbytes)
        check(lib.hero_attn_decode_paged(pa, stream()))
        got = host(out, np.float32, (B, qw))
        blocks = act_to_blocks(host(act, np.uint8), B, qw)
        worst = 0.0
        for b in range(B):
            expect = attn_expect(proj[b], keys16[b], vals16[b], qg, kg, inv, pos, window, scale, True)
            tol = 1e-4 * np.abs(expect).max()
            np.testing.assert_allclose(got[b], expect, rtol=1e-4, atol=tol, err_msg=f"fp16 window={window} seq {b}")
            worst = max(worst, float(np.abs(got[b] - expect).max() / np.abs(expect).max()))
            assert blocks[b].tobytes() == oracle.quantize_row_q8_0(got[b]).tobytes()
        say(f"[attn B={B} ctx={ctx}] paged fp16 cache, window={window}: max|d|/max = {worst:.3g}")


def q8_round_trip(x):
    """rows of 128-value heads through quantize_row_q8_0 (the reference's
    activation quantizer) and back as d * q: the values a Q8_0 cache holds;
    also returns the int8 quants and fp16 scale bits, [rows][128], [rows][4]"""
    flat = np.ascontiguousarray(x, np.float32).reshape(-1, ATT_DH)
    blocks = oracle.quantize_row_q8_0(flat.reshape(-1))
    d16 = np.ascontiguousarray(blocks["d"]).view(np.uint16).reshape(-1)
    q = np.ascontiguousarray(blocks["qs"]).view(np.int8).reshape(-1, 32)
    deq = (oracle.fp16_to_fp32(d16).astype(np.float32)[:, None] * q.astype(np.float32)).astype(np.float32)
    return deq.reshape(x.shape), q.reshape(flat.shape[0], ATT_DH), d16.reshape(flat.shape[0], 4)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("B,ctx", [(1, 8192), (16, 1024), (3, 9000)])
def test_attn_q8_pages_match_oracle(lib, B, ctx):
    """32q/8kv attention decode over a Q8_0 paged cache (pages of 64 positions
    in a shuffled pool; int8 rows and fp16 block scales per page): against the
    oracle over the same Q8_0 round-tripped K/V, full causal and window 1024,
    within rtol 1e-4 + atol 1e-4 * max|out| (the split-K merge reorders the
    softmax sums); the row the kernel appends equals the oracle's quantization
    of the new key and value."""
    from hero_amd._lib import AttnDecodeArgs, AttnPagedArgs

    rng = np.random.default_rng(B * 7919 + ctx)
    dh, hq, hkv = ATT_DH, ATT_HQ, ATT_HKV
    qw, kw = hq * dh, hkv * dh
    pos, keys, vals, proj, qg, kg = attn_inputs(rng, B, ctx)
    inv = oracle.rope_inv_freq(dh, 1e6, 32)
    d_cs = dev(oracle.rope_table(dh, 1e6, 32, ctx))
    d_qg, d_kg = dev(qg), dev(kg)
    d_proj, d_pos = dev(proj), dev(np.full(B, pos, np.int32))
    stride = 2 * qw + 2 * kw
    eps = np.float32(1e-6)
    act = empty(lib.hero_q8_0_act_bytes(B, qw))
    out = empty(B * qw * 4)
    d_qr = empty(B * hq * dh * 4)
    page = 64
    max_pages = (ctx + page - 1) // page
    page_bytes = lib.hero_attn_page_bytes(hkv, dh, page, 1)
    assert page_bytes == 2 * hkv * page * (dh + 8)
    table = rng.permutation(B * max_pages).astype(np.int32).reshape(B, max_pages)
    pool = np.zeros((B * max_pages, page_bytes), np.uint8)
    qpart = pool[:, :2 * hkv * page * dh].reshape(-1, 2, hkv, page, dh)
    spart = pool[:, 2 * hkv * page * dh:].view(np.uint16).reshape(-1, 2, hkv, page, 4)
    deq = {}
    for which, src in ((0, keys), (1, vals)):
        d, q, sc = q8_round_trip(src.reshape(B, pos, hkv, dh))
        deq[which] = d.reshape(B, pos, kw)
        qp = np.zeros((B, max_pages * page, hkv, dh), np.int8)
        sp = np.zeros((B, max_pages * page, hkv, 4), np.uint16)
        qp[:, :pos] = q.reshape(B, pos, hkv, dh)
        sp[:, :pos] = sc.reshape(B, pos, hkv, 4)
        qpart[table.reshape(-1), which] = qp.reshape(B, max_pages, page, hkv, dh).transpose(0, 1, 3, 2, 4).reshape(-1, hkv, page, dh).view(np.uint8)
        spart[table.reshape(-1), which] = sp.reshape(B, max_pages, page, hkv, 4).transpose(0, 1, 3, 2, 4).reshape(-1, hkv, page, 4)
        del qp, sp
    d_pages, d_table = dev(pool), dev(table)
    for window, scale in VARIANTS:
        wbytes = lib.hero_attn_paged_work_bytes(max_pages * page, window, B, hq, hkv, dh)
        d_work = empty(wbytes)
        a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), None, None,
                           0, ptr(d_pos), None, ptr(d_qr), scale, window, ptr(act), ptr(out), B, hq, hkv, dh)
        pa = AttnPagedArgs(a, ptr(d_pages), ptr(d_table), page, max_pages, ptr(d_work), wbytes, 1)
        check(lib.hero_attn_decode_paged(pa, stream()))
        got = host(out, np.float32, (B, qw))
        worst = 0.0
        for b in range(B):
            # the oracle appends the new row through the same round trip
            qv = proj[b, 2 * qw:].reshape(2, hkv, dh)
            k_new = oracle.rope_apply(oracle.rmsnorm(qv[0], kg, eps), inv, pos).reshape(1, kw)
            k_new, _, _ = q8_round_trip(k_new)
            v_new, _, _ = q8_round_trip(qv[1].reshape(1, kw))
            qh = np.stack([proj[b, h * 2 * dh: h * 2 * dh + dh] for h in range(hq)])
            g = np.concatenate([proj[b, h * 2 * dh + dh: h * 2 * dh + 2 * dh] for h in range(hq)])
            q = oracle.rope_apply(oracle.rmsnorm(qh, qg, eps), inv, pos)
            kk = np.concatenate([deq[0][b], k_new])
            vv = np.concatenate([deq[1][b], v_new])
            expect = (oracle.attend_decode(q.reshape(-1), kk, vv, hq, hkv, dh, window, scale).reshape(-1) * oracle.sigmoid(g)).astype(np.float32)
            tol = 1e-4 * np.abs(expect).max()
            np.testing.assert_allclose(got[b], expect, rtol=1e-4, atol=tol, err_msg=f"q8 window={window} seq {b}")
            worst = max(worst, float(np.abs(got[b] - expect).max() / np.abs(expect).max()))
        say(f"[attn B={B} ctx={ctx}] paged Q8_0 cache, window={window}: max|d|/max = {worst:.3g}")
    # the appended row (position pos) of sequence 0, K and V: the oracle's quantization
    pool_after = host(d_pages, np.uint8).reshape(B * max_pages, page_bytes)
    pg = table[0, pos // page]
    qa = pool_after[:, :2 * hkv * page * dh].reshape(-1, 2, hkv, page, dh)[pg, :, :, pos % page].view(np.int8)
    sa = pool_after[:, 2 * hkv * page * dh:].copy().view(np.uint16).reshape(-1, 2, hkv, page, 4)[pg, :, :, pos % page]
    qv = proj[0, 2 * qw:].reshape(2, hkv, dh)
    k_new = oracle.rope_apply(oracle.rmsnorm(qv[0], kg, eps), inv, pos)
    for which, row in ((0, k_new), (1, qv[1])):
        _, q, sc = q8_round_trip(row.reshape(1, kw))
        assert np.array_equal(qa[which], q.reshape(hkv, dh)), which
        assert np.array_equal(sa[which], sc.reshape(hkv, 4)), which
