"""GPU kernels through the C ABI against the oracle and the reference's golden
vectors. Integer and byte results (quantized activations, int32 block sums,
argmax) must be bit-exact, and so must every fp32 result: each kernel replays
the reference's fp32 operation order, and the device's expf / log1pf return
exactly glibc's values (hero/libm.hpp), which the first test checks."""
import numpy as np
import pytest

import oracle
from gpu_util import act_to_blocks, bits, check, dev, empty, gdn_reference, host, pack_weight, ptr, quantize_dev, stream, ulp_diff

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from hero_amd._lib import lib as _lib

    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return _lib


# ---- scalar functions --------------------------------------------------------------
def math_inputs():
    rng = np.random.default_rng(42)
    stride = np.arange(0, 2 ** 32, 4099, dtype=np.uint64).astype(np.uint32).view(np.float32)
    hexes = ["0x1.04845ep+5", "-0x1.f8cbb2p+5", "0x1.a827aep-2", "0x1.a827b4p-2", "0x1.6a09e6p+125"]  # glibc != correctly rounded
    hard = np.array([float.fromhex(h) for h in hexes] + [88.0, 88.72283, 88.7229, -103.97, -103.98, -87.3, -1.0, -0.99999994,
                                                        20.0, 20.000002, 1e-30, -1e-30, np.inf, -np.inf], np.float32)
    dense = np.concatenate([rng.uniform(-30, 30, 1 << 20), rng.standard_normal(1 << 18) * 3]).astype(np.float32)
    x = np.concatenate([stride, hard, dense])
    return x[~np.isnan(x)]


def test_device_exp_log1p_equal_glibc_and_activations_equal_oracle(lib):
    x = math_inputs()
    out = empty(5 * x.size * 4)
    xd = dev(x)
    check(lib.hero_math_eval(ptr(xd), ptr(out), x.size, stream()))
    got = host(out, np.float32, (5, x.size))
    same = lambda a, b: bool(np.all((bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b))))  # noqa: E731
    assert same(got[0], oracle.expf(x)), "expf differs from glibc"
    assert same(got[1], oracle.log1pf(x)), "log1pf differs from glibc"
    assert same(got[2], oracle.silu(x)), "silu differs from the reference form x/(1+exp(-x))"
    assert same(got[3], oracle.sigmoid(x))
    assert same(got[4], oracle.softplus(x))


# ---- quantization --------------------------------------------------------------
def test_quantize_matches_reference_golden(lib, kernels_golden):
    x = kernels_golden["in_quant"].reshape(1, -1)
    act = host(quantize_dev(lib, x), np.uint8)
    assert act_to_blocks(act, 1, x.shape[1]).tobytes() == kernels_golden["out_quant_act"].tobytes()


@pytest.mark.parametrize("k", [1024, 2816, 4096, 12288])
def test_quantize_matches_oracle(lib, k):
    rng = np.random.default_rng(k)
    x = (rng.standard_normal((3, k)) * np.exp(rng.uniform(-10, 6, (3, 1)))).astype(np.float32)
    x[0, :32] = 0
    act = host(quantize_dev(lib, x), np.uint8)
    got = act_to_blocks(act, 3, k)
    for r in range(3):
        assert got[r].tobytes() == oracle.quantize_row_q8_0(x[r]).tobytes()


# ---- GEMV -----------------------------------------------------------------------
def test_gemv_matches_reference_golden(lib, kernels_golden):
    wq = kernels_golden["out_gemv_wq"].view(oracle.BLOCK)
    x = kernels_golden["in_gemv_x"].reshape(8, 4096)
    packed = pack_weight(lib, wq, 64, 4096)
    golden = [kernels_golden["out_gemv_y"]] + list(kernels_golden["out_gemm_y"].reshape(8, 64))
    for r in range(8):
        act = quantize_dev(lib, x[r:r + 1])
        y = empty(64 * 4)
        check(lib.hero_q8_0_gemv(ptr(packed), ptr(act), ptr(y), None, 64, 4096, stream()))
        assert np.array_equal(bits(host(y, np.float32)), bits(golden[r + 1] if r else golden[0])), f"row {r}"


# K % 4096 == 0 takes the streaming kernel (incl. N not a multiple of 8 and
# fewer rows than workgroups); other K the general one
GEMV_SHAPES = [(4096, 4096), (16448, 4096), (4096, 12288), (4100, 4096), (33, 8192), (1003, 12288), (96, 4096),
               (10240, 1024), (5632, 1024), (1024, 2816), (32000, 1024), (64, 256)]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_matches_oracle_bitwise(lib, n, k):
    rng = np.random.default_rng(n * 7 + k)
    w = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((1, k)).astype(np.float32)
    packed = pack_weight(lib, w, n, k)
    act = quantize_dev(lib, x)
    y = empty(n * 4)
    check(lib.hero_q8_0_gemv(ptr(packed), ptr(act), ptr(y), None, n, k, stream()))
    expect = oracle.matvec(w, n, k, x[0])
    assert np.array_equal(bits(host(y, np.float32)), bits(expect))
    # residual epilogue: y = r + W x, one fp32 add (nm/src/qwen35.hpp:321)
    r = rng.standard_normal(n).astype(np.float32)
    rd = dev(r)
    check(lib.hero_q8_0_gemv(ptr(packed), ptr(act), ptr(y), ptr(rd), n, k, stream()))
    assert np.array_equal(bits(host(y, np.float32)), bits(r + expect))


@pytest.mark.parametrize("n,k", [(4096, 4096), (16448, 4096), (33, 4096), (1000, 1024)])
def test_rmsnorm_gemv_matches_oracle_bitwise(lib, n, k):
    """RMSNorm + quantize + matvec; K == 4096 runs as one launch with the norm
    in the GEMV prologue, other K through the act scratch."""
    rng = np.random.default_rng(n + 3 * k)
    w = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed = pack_weight(lib, w, n, k)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    gd = dev(g)
    scratch = empty(lib.hero_q8_0_act_bytes(1, k))
    y = empty(n * 4)
    rows = [rng.standard_normal(k) * 3] + ([_hard_rows(k)[i] for i in (1, 5, 6, 8, 9)] if k == 4096 else [])
    for i, row in enumerate(rows):
        x = np.asarray(row, np.float32)
        xd = dev(x)
        r = rng.standard_normal(n).astype(np.float32)
        rd = dev(r)
        check(lib.hero_rmsnorm_q8_0_gemv(ptr(packed), ptr(xd), ptr(gd), np.float32(1e-6), ptr(y), ptr(rd), n, k, ptr(scratch), stream()))
        expect = r + oracle.matvec(w, n, k, oracle.rmsnorm(x[None, :], g)[0])
        assert np.array_equal(bits(host(y, np.float32)), bits(expect)), f"row {i}"


@pytest.mark.parametrize("n,k", [(4096, 12288), (1003, 4096), (64, 8192), (1024, 2816)])
def test_swiglu_gemv_matches_oracle_bitwise(lib, n, k):
    """silu(gate) * up + quantize + matvec (the down projection)."""
    rng = np.random.default_rng(n + 5 * k)
    w = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed = pack_weight(lib, w, n, k)
    gu = (rng.standard_normal(2 * k) * 1.5).astype(np.float32)
    gud = dev(gu)
    scratch = empty(lib.hero_q8_0_act_bytes(1, k))
    y = empty(n * 4)
    check(lib.hero_swiglu_q8_0_gemv(ptr(packed), ptr(gud), ptr(y), None, n, k, ptr(scratch), stream()))
    expect = oracle.matvec(w, n, k, oracle.silu(gu[:k]) * gu[k:])
    assert np.array_equal(bits(host(y, np.float32)), bits(expect))


@pytest.mark.parametrize("ff", [12288, 96])
def test_rmsnorm_gate_up_swiglu_matches_oracle_bytes(lib, ff):
    """RMSNorm -> [gate|up] GEMV -> silu(gate)*up -> quantize in one launch
    (gate and up packed in alternating 32-row chunks) against the oracle's
    separate steps, byte for byte."""
    k = 4096
    rng = np.random.default_rng(ff)
    wg = oracle.quantize_q8_0((rng.standard_normal((ff, k)) * 0.02).astype(np.float32))
    wu = oracle.quantize_q8_0((rng.standard_normal((ff, k)) * 0.02).astype(np.float32))
    packed = empty(lib.hero_q8_0_packed_bytes(2 * ff, k))
    srcg, srcu = dev(wg), dev(wu)
    check(lib.hero_q8_0_pack_interleaved(ptr(srcg), ptr(packed), 2 * ff, k, 0, ff, 32, stream()))
    check(lib.hero_q8_0_pack_interleaved(ptr(srcu), ptr(packed), 2 * ff, k, 32, ff, 32, stream()))
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    xd, gd = dev(x), dev(g)
    act = empty(lib.hero_q8_0_act_bytes(1, ff))
    check(lib.hero_rmsnorm_q8_0_gemv_swiglu(ptr(packed), ptr(xd), ptr(gd), np.float32(1e-6), ptr(act), ff, k, stream()))
    xn = oracle.rmsnorm(x[None, :], g)[0]
    gate = oracle.matvec(wg, ff, k, xn)
    up = oracle.matvec(wu, ff, k, xn)
    want = oracle.quantize_row_q8_0(oracle.silu(gate) * up)
    got = act_to_blocks(host(act, np.uint8), 1, ff)[0]
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096), (64, 1000, 1024), (5, 96, 12288), (130, 4100, 4096), (33, 64, 2816), (1, 64, 256),
                                   # the skinny path (M <= 16): ragged 16-row groups, a partial round
                                   # (768 = 24 blocks), fewer rows than one group, the largest K
                                   (2, 4100, 4096), (8, 33, 12288), (16, 1003, 768), (13, 12288, 4096), (3, 7, 256), (16, 40, 16384),
                                   # its tall forms (at least two 16-row groups per CU): a wave per range (8200
                                   # rows with a ragged last group, K = 12288), and from four groups per CU at
                                   # K = 4096 the activations in shared memory with 6 (16448, 24576) and 8
                                   # (40000) waves per workgroup
                                   (16, 8200, 4096), (7, 9000, 12288), (5, 16448, 4096), (16, 24576, 4096), (11, 40000, 4096)])
def test_gemm_matches_oracle_bitwise(lib, m, n, k):
    """M-row GEMM on int8 MFMA: every element equals the reference's matmul
    (per-row vec_dot in block order), with and without the residual."""
    rng = np.random.default_rng(m * 31 + n + k)
    w = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed = pack_weight(lib, w, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    act = quantize_dev(lib, x)
    y = empty(m * n * 4)
    check(lib.hero_q8_0_gemm(ptr(packed), ptr(act), ptr(y), None, m, n, k, stream()))
    expect = oracle.matmul(w, n, k, x)
    got = host(y, np.float32, (m, n))
    assert np.array_equal(bits(got), bits(expect))
    r = rng.standard_normal((m, n)).astype(np.float32)
    rd = dev(r)
    check(lib.hero_q8_0_gemm(ptr(packed), ptr(act), ptr(y), ptr(rd), m, n, k, stream()))
    assert np.array_equal(bits(host(y, np.float32, (m, n))), bits(r + expect))


# scales in fp16's subnormal range (and rows whose scale rounds to 0): every
# GEMM form must turn them into fp32 and form d_x * d_w with no flush to zero;
# (512, 8192) selects the 128-row tile, (70, 4100) a smaller one, (9, 4100)
# the skinny form
@pytest.mark.parametrize("m,n,k", [(512, 8192, 1024), (70, 4100, 2048), (9, 4100, 1024)])
def test_gemm_subnormal_scales_match_oracle_bitwise(lib, m, n, k):
    rng = np.random.default_rng(m + n + k + 5)
    wscale = np.where(rng.random((n, 1)) < 0.3, 1e-3, 1.0) * np.where(rng.random((n, 1)) < 0.05, 1e-6, 1.0)
    w = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02 * wscale).astype(np.float32))
    d = w["d"].view(np.float16).astype(np.float32)
    assert np.any((d > 0) & (d < 6.1e-5)), "some weight scales are subnormal fp16"
    packed = pack_weight(lib, w, n, k)
    xscale = rng.choice([1.0, 3e-5, 1e-7, 1e3], size=(m, 1))
    x = (rng.standard_normal((m, k)) * xscale).astype(np.float32)
    act = quantize_dev(lib, x)
    y = empty(m * n * 4)
    check(lib.hero_q8_0_gemm(ptr(packed), ptr(act), ptr(y), None, m, n, k, stream()))
    expect = oracle.matmul(w, n, k, x)
    got = host(y, np.float32, (m, n))
    bad = np.flatnonzero(bits(got).ravel() != bits(expect).ravel())
    assert bad.size == 0, f"{bad.size} outputs differ, first {bad[:5]}: {got.ravel()[bad[:3]]} vs {expect.ravel()[bad[:3]]}"


def test_block_sums_are_exact(lib):
    n, k = 257 * 2, 4096
    rng = np.random.default_rng(3)
    w = np.zeros(n * k // 32, oracle.BLOCK)
    w["qs"] = rng.integers(-127, 128, (n * k // 32, 32))
    w["d"] = np.float16(0.01).view(np.uint16)
    x = rng.standard_normal((1, k)).astype(np.float32) * 3
    x[0, :32] = 127.0  # extreme block: |sumi| up to 32*127*127
    w["qs"][0] = 127
    packed = pack_weight(lib, w, n, k)
    act = quantize_dev(lib, x)
    out = empty(n * (k // 32) * 4)
    check(lib.hero_q8_0_block_sums(ptr(packed), ptr(act), ptr(out), n, k, stream()))
    xb = oracle.quantize_row_q8_0(x[0])
    assert np.array_equal(host(out, np.int32).reshape(n, -1), oracle.block_sums(w, n, k, xb))
    # brute force over the int8 values
    brute = np.einsum("nbj,bj->nb", w["qs"].reshape(n, k // 32, 32).astype(np.int64), xb["qs"].astype(np.int64))
    assert np.array_equal(host(out, np.int32).reshape(n, -1), brute)


# ---- RMSNorm + quantize, SwiGLU + quantize -------------------------------------------
@pytest.mark.parametrize("d", [1024, 4096])
def test_rmsnorm_quant_matches_oracle(lib, d):
    rng = np.random.default_rng(d)
    m = 3
    x = (rng.standard_normal((m, d)) * 2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    xd, gd = dev(x), dev(g)
    y = empty(m * d * 4)
    act = empty(lib.hero_q8_0_act_bytes(m, d))
    check(lib.hero_rmsnorm_quant(ptr(xd), ptr(gd), np.float32(1e-6), ptr(y), ptr(act), m, d, stream()))
    expect = oracle.rmsnorm(x, g)
    assert np.array_equal(bits(host(y, np.float32, (m, d))), bits(expect))
    blocks = act_to_blocks(host(act, np.uint8), m, d)
    for r in range(m):
        assert blocks[r].tobytes() == oracle.quantize_row_q8_0(expect[r]).tobytes()


def _hard_rows(d: int) -> np.ndarray:
    """Rows whose sums of squares stress the exact parallel sum: ties, zeros,
    subnormal and near-overflow squares, outliers, many binade crossings."""
    rng = np.random.default_rng(d + 1)
    i = np.arange(d, dtype=np.float64)
    rows = [
        rng.standard_normal(d) * 2,
        rng.standard_normal(d) * 1e-21,                       # subnormal squares
        rng.standard_normal(d) * 3e17,                        # squares near 1e36
        np.where(rng.random(d) < 0.5, 0.0, rng.standard_normal(d)),
        np.where(i < d // 2, 0.0, rng.standard_normal(d)),    # leading zeros
        np.ones(d),                                           # exact integer sums
        rng.integers(-4, 5, d) * 0.5,                         # many ties
        rng.standard_normal(d) * np.where(rng.random(d) < 0.01, 1e3, 1.0),
        np.exp2(i / 300.0) * np.sign(rng.standard_normal(d)), # growing terms
        np.zeros(d),
        np.full(d, 2.0 ** 60),                                # sum overflows to inf
    ]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("d", [4096, 1024, 2080])
def test_rmsnorm_exact_on_hard_rows(lib, d):
    x = _hard_rows(d)
    m = x.shape[0]
    g = np.ones(d, np.float32)
    y = empty(m * d * 4)
    xd, gd = dev(x), dev(g)
    check(lib.hero_rmsnorm_quant(ptr(xd), ptr(gd), np.float32(1e-6), ptr(y), None, m, d, stream()))
    got = host(y, np.float32, (m, d))
    expect = oracle.rmsnorm(x, g)
    for r in range(m):
        assert np.array_equal(bits(got[r]), bits(expect[r])), f"row {r}"


def test_rmsnorm_matches_reference_golden(lib, kernels_golden):
    for n in (1024, 4096):
        v = kernels_golden[f"in_rms{n}"]
        xd, gd = dev(v[:n]), dev(v[n:])
        y = empty(n * 4)
        check(lib.hero_rmsnorm_quant(ptr(xd), ptr(gd), np.float32(1e-6), ptr(y), None, 1, n, stream()))
        assert np.array_equal(bits(host(y, np.float32)), bits(kernels_golden[f"out_rms{n}"]))


def test_swiglu_quant_matches_oracle(lib):
    rng = np.random.default_rng(11)
    m, ff = 2, 12288
    gu = (rng.standard_normal((m, 2 * ff)) * 1.5).astype(np.float32)
    act = empty(lib.hero_q8_0_act_bytes(m, ff))
    gud = dev(gu)
    check(lib.hero_swiglu_quant(ptr(gud), ptr(act), m, ff, stream()))
    got = act_to_blocks(host(act, np.uint8), m, ff)
    for r in range(m):
        g = oracle.silu(gu[r, :ff]) * gu[r, ff:]
        assert got[r].tobytes() == oracle.quantize_row_q8_0(g).tobytes()


# ---- embedding, argmax ------------------------------------------------------------
def test_embed_matches_oracle(lib):
    rng = np.random.default_rng(5)
    v, d = 1000, 1024
    w = oracle.quantize_q8_0((rng.standard_normal((v, d)) * 0.02).astype(np.float32))
    packed = pack_weight(lib, w, v, d)
    ids = np.array([0, 999, 5, 5, 123], np.int32)
    out = empty(len(ids) * d * 4)
    idd = dev(ids)
    check(lib.hero_q8_0_embed(ptr(packed), v, d, ptr(idd), len(ids), ptr(out), stream()))
    got = host(out, np.float32, (len(ids), d))
    wb = w.reshape(v, d // 32)
    for i, t in enumerate(ids):
        d16 = wb[t]["d"].view(np.float16).astype(np.float32)
        expect = (np.repeat(d16, 32) * wb[t]["qs"].reshape(-1).astype(np.float32)).astype(np.float32)
        assert np.array_equal(bits(got[i]), bits(expect))


def test_argmax_ties_go_to_lowest_index(lib):
    rng = np.random.default_rng(9)
    m, n = 4, 151936
    logits = rng.standard_normal((m, n)).astype(np.float32)
    logits[1, [70000, 5, 150000]] = 50.0          # tie: lowest index wins
    logits[2, :] = -1.0
    logits[2, 100] = 0.0
    logits[2, 50] = -0.0                          # -0 == +0: lowest index wins
    logits[3, n - 1] = 99.0                       # last element
    out = empty(m * 4)
    scratch = empty(m * 128 * 8)
    ld = dev(logits)
    check(lib.hero_argmax(ptr(ld), m, n, ptr(out), ptr(scratch), stream()))
    got = host(out, np.int32)
    assert list(got) == [int(np.argmax(r)) for r in logits]
    assert list(got[1:]) == [5, 50, n - 1]


# ---- gated delta-net decode ---------------------------------------------------------
@pytest.mark.parametrize("hk,hv", [(8, 8), (4, 8)])
def test_gdn_decode_matches_oracle(lib, hk, hv):
    from hero_amd._lib import GdnDecodeArgs

    rng = np.random.default_rng(hk * 100 + hv)
    B, dk, W, steps = 2, 128, 4, 6
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    taps = (rng.standard_normal((cc, W)) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(hv) * 0.1).astype(np.float32)
    decay = (-np.exp(rng.standard_normal(hv) * 0.5)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(dk)).astype(np.float32)
    eps = np.float32(1e-6)
    d_taps, d_dt, d_decay, d_gamma = dev(taps), dev(dt), dev(decay), dev(gamma)
    d_hist = empty(B * W * cc * 4)
    d_state = empty(B * hv * dk * dk * 4)
    o_hist = [np.zeros((W - 1, cc), np.float32) for _ in range(B)]
    o_state = [np.zeros((hv, dk, dk), np.float32) for _ in range(B)]
    act = empty(lib.hero_q8_0_act_bytes(B, hv * dk))
    out = empty(B * hv * dk * 4)
    for step in range(steps):
        proj = (rng.standard_normal((B, stride)) * 0.7).astype(np.float32)
        pos = np.array([step, step], np.int32)
        d_proj, d_pos = dev(proj), dev(pos)
        a = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + hv * dk, cc + hv * dk + hv, ptr(d_taps), ptr(d_hist), ptr(d_state),
                          ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(act), ptr(out), B, hk, hv, dk, dk, W)
        check(lib.hero_gdn_decode(a, stream()))
        got = host(out, np.float32, (B, hv * dk))
        got_blocks = act_to_blocks(host(act, np.uint8), B, hv * dk)
        for b in range(B):
            expect = gdn_reference(proj[b], taps, o_hist[b], o_state[b], dt, decay, gamma, eps, hk, hv, step)
            assert np.array_equal(bits(got[b]), bits(expect)), f"step {step} seq {b}: max ulp {ulp_diff(got[b], expect).max()}"
            assert got_blocks[b].tobytes() == oracle.quantize_row_q8_0(expect).tobytes()
        gstate = host(d_state, np.float32, (B, hv, dk, dk))
        for b in range(B):
            assert np.array_equal(bits(gstate[b]), bits(o_state[b])), f"state after step {step} seq {b}"


@pytest.mark.parametrize("hk,hv,W", [(4, 8, 4), (32, 32, 4), (2, 4, 3)])
def test_gdn_decode_column_split_equals_fused_kernel(lib, hk, hv, W):
    """The column-split decode (8 workgroups per head) followed by the head
    norm + gate, or by the head-gated output projection (32 heads: the GEMV
    prologue form), over 3 steps from zero state: outputs, quantized outputs,
    the W_o product, state and ring equal the one-workgroup-per-head kernel's
    bit for bit (tiled key heads with hk < hv)."""
    from hero_amd._lib import GdnDecodeArgs

    rng = np.random.default_rng(hk * 7 + hv + W)
    B, dk = 2, 128
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    taps = (rng.standard_normal((cc, W)) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(hv) * 0.1).astype(np.float32)
    decay = (-np.exp(rng.standard_normal(hv) * 0.5)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(dk)).astype(np.float32)
    eps = np.float32(1e-6)
    d_taps, d_dt, d_decay, d_gamma = dev(taps), dev(dt), dev(decay), dev(gamma)
    width = hv * dk
    if width == 4096:
        wo = np.zeros((1000, width // 32), oracle.BLOCK)
        wo["qs"] = rng.integers(-127, 128, (1000, width // 32, 32), dtype=np.int8)
        wo["d"] = oracle.fp32_to_fp16(np.abs(rng.standard_normal((1000, width // 32))).astype(np.float32) * np.float32(1e-3))
        packed = pack_weight(lib, wo, 1000, width)
        resid = dev(rng.standard_normal(1000).astype(np.float32))
    bufs = {}
    for name in ("fused", "split"):
        bufs[name] = dict(hist=empty(B * W * cc * 4), state=empty(B * hv * dk * dk * 4), act=empty(lib.hero_q8_0_act_bytes(B, width)),
                          out=empty(B * width * 4), o_raw=empty(B * width * 4), gates=empty(B * width * 4), y=empty(1000 * 4))
    for step in range(3):
        proj = (rng.standard_normal((B, stride)) * 0.7).astype(np.float32)
        d_proj, d_pos = dev(proj), dev(np.array([step, step + 5], np.int32))
        res = {}
        for name, bf in bufs.items():
            a = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + width, cc + width + hv, ptr(d_taps), ptr(bf["hist"]), ptr(bf["state"]),
                              ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(bf["act"]), ptr(bf["out"]), B, hk, hv, dk, dk, W)
            if name == "fused":
                check(lib.hero_gdn_decode(a, stream()))
            else:
                check(lib.hero_gdn_decode_cols(a, ptr(bf["o_raw"]), ptr(bf["gates"]), stream()))
                check(lib.hero_gdn_norm_gate(ptr(bf["o_raw"]), a, stream()))
            res[name] = [host(bf[k], np.uint8).copy() for k in ("out", "act", "state", "hist")]
        for i, what in enumerate(("output", "quantized output", "state", "ring")):
            assert np.array_equal(res["fused"][i], res["split"][i]), f"step {step}: {what}"
        if width == 4096:  # sequence 0 through W_o: plain GEMV on the fused act vs the head-gated prologue
            fb, sb = bufs["fused"], bufs["split"]
            a_all = host(fb["act"], np.uint8)  # [B*K int8][B*K/32 fp32]: sequence 0's row as a 1-row act
            act0 = dev(np.concatenate([a_all[:width], a_all[B * width: B * width + width // 32 * 4]]))
            check(lib.hero_q8_0_gemv(ptr(packed), ptr(act0), ptr(fb["y"]), ptr(resid), 1000, width, stream()))
            check(lib.hero_headgate_q8_0_gemv(ptr(packed), ptr(sb["o_raw"]), ptr(sb["gates"]), ptr(d_gamma), eps, ptr(sb["y"]), ptr(resid),
                                              1000, width, stream()))
            assert np.array_equal(host(fb["y"], np.uint32), host(sb["y"], np.uint32)), f"step {step}: W_o product"


@pytest.mark.parametrize("W,chunks", [(4, [2, 7, 1, 3, 5, 40, 17]), (3, [1, 1, 6, 2, 33]), (1, [3, 1, 4, 16])])
def test_gdn_prefill_chunks_match_oracle(lib, W, chunks):
    """Delta-net prefill in ragged chunks (shorter and longer than the conv
    window, single tokens through the decode entry point in between): every
    output row, its Q8_0 blocks and the state after each chunk equal the
    oracle's token-serial recurrence bit for bit."""
    from hero_amd._lib import GdnDecodeArgs

    hk, hv, dk = 2, 4, 128
    rng = np.random.default_rng(1000 + W)
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    taps = (rng.standard_normal((cc, W)) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(hv) * 0.1).astype(np.float32)
    decay = (-np.exp(rng.standard_normal(hv) * 0.5)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(dk)).astype(np.float32)
    eps = np.float32(1e-6)
    d_taps, d_dt, d_decay, d_gamma = dev(taps), dev(dt), dev(decay), dev(gamma)
    d_hist = empty(W * cc * 4)
    d_state = empty(hv * dk * dk * 4)
    o_hist = np.zeros((max(W - 1, 0), cc), np.float32)
    o_state = np.zeros((hv, dk, dk), np.float32)
    tmax = max(chunks)
    act = empty(lib.hero_q8_0_act_bytes(tmax, hv * dk))
    out = empty(tmax * hv * dk * 4)
    work_bytes = lib.hero_gdn_prefill_work_bytes(tmax, hk, hv)
    work = empty(work_bytes)
    pos = 0
    for i, T in enumerate(chunks):
        proj = (rng.standard_normal((T, stride)) * 0.7).astype(np.float32)
        d_proj, d_pos = dev(proj), dev(np.array([pos], np.int32))
        a = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + hv * dk, cc + hv * dk + hv, ptr(d_taps), ptr(d_hist), ptr(d_state),
                          ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(act), ptr(out), T, hk, hv, dk, dk, W)
        if T == 1 and i % 2:
            check(lib.hero_gdn_decode(a, stream()))
        else:
            check(lib.hero_gdn_prefill(a, ptr(work), work_bytes, stream()))
        got = host(out, np.float32, (tmax, hv * dk))[:T]
        got_blocks = act_to_blocks(host(act, np.uint8)[: T * hv * dk + T * hv * dk // 32 * 4], T, hv * dk)
        for t in range(T):
            expect = gdn_reference(proj[t], taps, o_hist, o_state, dt, decay, gamma, eps, hk, hv, pos + t)
            assert np.array_equal(bits(got[t]), bits(expect)), f"chunk {i} row {t}: max ulp {ulp_diff(got[t], expect).max()}"
            assert got_blocks[t].tobytes() == oracle.quantize_row_q8_0(expect).tobytes(), f"chunk {i} row {t} blocks"
        gstate = host(d_state, np.float32, (hv, dk, dk))
        assert np.array_equal(bits(gstate), bits(o_state)), f"state after chunk {i}"
        pos += T


@pytest.mark.parametrize("T,hk,hv", [(70, 2, 4), (300, 4, 4)])
def test_gdn_chunked_prefill_matches_serial(lib, T, hk, hv):
    """The chunked (WY) delta-net prefill against the token-serial one (which
    is bit-exact with the oracle) and, for the shorter case, the oracle's own
    serial recurrence: outputs and the final state within fp32 rounding-order
    tolerance, over a partial last chunk and several chunks, from a non-zero
    state and a non-empty conv ring (a first chunk of 37 tokens)."""
    from hero_amd._lib import GdnDecodeArgs

    rng = np.random.default_rng(T + hk)
    dk, W = 128, 4
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    taps = (rng.standard_normal((cc, W)) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(hv) * 0.1).astype(np.float32)
    decay = (-np.exp(rng.standard_normal(hv) * 0.5)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(dk)).astype(np.float32)
    eps = np.float32(1e-6)
    d_taps, d_dt, d_decay, d_gamma = dev(taps), dev(dt), dev(decay), dev(gamma)
    warm = (rng.standard_normal((37, stride)) * 0.7).astype(np.float32)
    proj = (rng.standard_normal((T, stride)) * 0.7).astype(np.float32)
    wbytes = lib.hero_gdn_prefill_work_bytes(T, hk, hv)
    results = []
    for entry in (lib.hero_gdn_prefill, lib.hero_gdn_prefill_chunked):
        d_hist = empty(W * cc * 4)
        d_state = empty(hv * dk * dk * 4)
        work = empty(wbytes)
        act = empty(lib.hero_q8_0_act_bytes(T, hv * dk))
        out = empty(T * hv * dk * 4)
        for rows, pos0, fn in ((warm, 0, lib.hero_gdn_prefill), (proj, 37, entry)):
            d_proj, d_pos = dev(rows), dev(np.array([pos0], np.int32))
            n = rows.shape[0]
            a = GdnDecodeArgs(ptr(d_proj), stride, cc, cc + hv * dk, cc + hv * dk + hv, ptr(d_taps), ptr(d_hist), ptr(d_state),
                              ptr(d_dt), ptr(d_decay), ptr(d_gamma), eps, ptr(d_pos), ptr(act), ptr(out), n, hk, hv, dk, dk, W)
            check(fn(a, ptr(work), wbytes, stream()))
        results.append((host(out, np.float32, (T, hv * dk)).copy(), host(d_state, np.float32, (hv, dk, dk)).copy()))
    (o_ser, s_ser), (o_chk, s_chk) = results
    scale_o, scale_s = np.abs(o_ser).max(), np.abs(s_ser).max()
    np.testing.assert_allclose(o_chk, o_ser, rtol=1e-3, atol=1e-4 * scale_o)
    np.testing.assert_allclose(s_chk, s_ser, rtol=1e-3, atol=1e-4 * scale_s)
    if T <= 100:  # the oracle's serial recurrence, token by token
        hist = np.zeros((W - 1, cc), np.float32)
        state = np.zeros((hv, dk, dk), np.float32)
        for t in range(37):
            gdn_reference(warm[t], taps, hist, state, dt, decay, gamma, eps, hk, hv, t)
        for t in range(T):
            expect = gdn_reference(proj[t], taps, hist, state, dt, decay, gamma, eps, hk, hv, 37 + t)
            np.testing.assert_allclose(o_chk[t], expect, rtol=1e-3, atol=1e-4 * scale_o)


# ---- attention decode ------------------------------------------------------------------
@pytest.mark.parametrize("window", [0, 3])
def test_attn_decode_matches_oracle(lib, window):
    from hero_amd._lib import AttnDecodeArgs

    rng = np.random.default_rng(17 + window)
    B, hq, hkv, dh, steps, max_ctx = 2, 8, 2, 128, 7, 16
    qw, kw = hq * dh, hkv * dh
    stride = 2 * qw + 2 * kw
    qg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    eps = np.float32(1e-6)
    scale = np.float32(1.0) / np.sqrt(np.float32(dh))
    inv = oracle.rope_inv_freq(dh, 1e6, dh // 4)
    d_cs = dev(oracle.rope_table(dh, 1e6, dh // 4, max_ctx))  # the reference's own cos/sin values
    d_kc, d_vc = empty(B * max_ctx * kw * 4), empty(B * max_ctx * kw * 4)
    d_sc = empty(B * hq * max_ctx * 4)
    d_qr = empty(B * hq * dh * 4)
    act = empty(lib.hero_q8_0_act_bytes(B, qw))
    out = empty(B * qw * 4)
    keys = [np.zeros((0, kw), np.float32) for _ in range(B)]
    vals = [np.zeros((0, kw), np.float32) for _ in range(B)]
    d_qg, d_kg = dev(qg), dev(kg)  # kept alive while the kernels read them
    for step in range(steps):
        proj = (rng.standard_normal((B, stride))).astype(np.float32)
        d_proj, d_pos = dev(proj), dev(np.array([step, step], np.int32))
        a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), ptr(d_kc), ptr(d_vc),
                           max_ctx, ptr(d_pos), ptr(d_sc), ptr(d_qr), scale, window, ptr(act), ptr(out), B, hq, hkv, dh)
        check(lib.hero_attn_decode(a, stream()))
        got = host(out, np.float32, (B, qw))
        for b in range(B):
            p = proj[b]
            q = np.stack([p[h * 2 * dh: h * 2 * dh + dh] for h in range(hq)])
            g = np.concatenate([p[h * 2 * dh + dh: h * 2 * dh + 2 * dh] for h in range(hq)])
            q = oracle.rope_apply(oracle.rmsnorm(q, qg, eps), inv, step)
            k = oracle.rope_apply(oracle.rmsnorm(p[2 * qw: 2 * qw + kw].reshape(hkv, dh), kg, eps), inv, step)
            keys[b] = np.concatenate([keys[b], k.reshape(1, kw)])
            vals[b] = np.concatenate([vals[b], p[2 * qw + kw:].reshape(1, kw)])
            att = oracle.attend_decode(q.reshape(-1), keys[b], vals[b], hq, hkv, dh, window, scale).reshape(-1)
            expect = (att * oracle.sigmoid(g)).astype(np.float32)
            assert np.array_equal(bits(got[b]), bits(expect)), f"step {step} seq {b}: max ulp {ulp_diff(got[b], expect).max()}"
        blocks = act_to_blocks(host(act, np.uint8), B, qw)
        for b in range(B):
            assert blocks[b].tobytes() == oracle.quantize_row_q8_0(got[b]).tobytes()


# long contexts over pre-filled caches: several tiles of the weighted sum
# (64 rows each, a ring of 6), score tiles of 256 keys, GQA groups of 1, 4 and
# 6 (score head chunks of 4 and 2), a sliding window, and enough sequences x
# heads to take the many-sequence form of the weighted sum (B * Hq * 4 > 512),
# whose workgroups serve up to four heads of a group (6 = one of 4, one of 2)
# 256-wide heads (the reference's Qwen 3.5 4B / 9B attention) take the per-row
# kernels at every B: one and two sequences, a window, many sequences
@pytest.mark.parametrize("B,hq,hkv,pos,window,dh", [(2, 8, 2, 700, 0, 128), (1, 6, 1, 1500, 0, 128), (2, 4, 4, 450, 300, 128),
                                                    (5, 32, 8, 333, 0, 128), (12, 12, 2, 260, 0, 128), (1, 16, 4, 1500, 0, 256),
                                                    (2, 8, 2, 450, 300, 256), (16, 16, 4, 333, 0, 256), (3, 8, 2, 4200, 0, 256)])
def test_attn_decode_long_context_matches_oracle(lib, B, hq, hkv, pos, window, dh):
    from hero_amd._lib import AttnDecodeArgs

    rng = np.random.default_rng(pos + hq)
    max_ctx = pos + 9
    qw, kw = hq * dh, hkv * dh
    stride = 2 * qw + 2 * kw
    qg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    eps = np.float32(1e-6)
    scale = np.float32(1.0) / np.sqrt(np.float32(dh)) if window == 0 else np.float32(1.0)
    inv = oracle.rope_inv_freq(dh, 1e6, 32)
    d_cs = dev(oracle.rope_table(dh, 1e6, 32, max_ctx))
    # cached rows 0 .. pos-1: K channel-major [B][Hkv][Dh][max_ctx], V [B][max_ctx][Hkv*Dh]
    keys = (rng.standard_normal((B, pos, kw)) * 0.5).astype(np.float32)
    vals = rng.standard_normal((B, pos, kw)).astype(np.float32)
    kc = np.zeros((B, hkv, dh, max_ctx), np.float32)
    kc[:, :, :, :pos] = keys.reshape(B, pos, hkv, dh).transpose(0, 2, 3, 1)
    vc = np.zeros((B, max_ctx, kw), np.float32)
    vc[:, :pos] = vals
    d_kc, d_vc = dev(kc), dev(vc)
    d_sc = empty(B * hq * max_ctx * 4)
    d_qr = empty(B * hq * dh * 4)
    act = empty(lib.hero_q8_0_act_bytes(B, qw))
    out = empty(B * qw * 4)
    proj = rng.standard_normal((B, stride)).astype(np.float32)
    d_proj, d_pos = dev(proj), dev(np.full(B, pos, np.int32))
    d_qg, d_kg = dev(qg), dev(kg)
    a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), ptr(d_kc), ptr(d_vc),
                       max_ctx, ptr(d_pos), ptr(d_sc), ptr(d_qr), scale, window, ptr(act), ptr(out), B, hq, hkv, dh)
    check(lib.hero_attn_decode(a, stream()))
    got = host(out, np.float32, (B, qw))
    for b in range(B):
        p = proj[b]
        q = np.stack([p[h * 2 * dh: h * 2 * dh + dh] for h in range(hq)])
        g = np.concatenate([p[h * 2 * dh + dh: h * 2 * dh + 2 * dh] for h in range(hq)])
        q = oracle.rope_apply(oracle.rmsnorm(q, qg, eps), inv, pos)
        k = oracle.rope_apply(oracle.rmsnorm(p[2 * qw: 2 * qw + kw].reshape(hkv, dh), kg, eps), inv, pos)
        kk = np.concatenate([keys[b], k.reshape(1, kw)])
        vv = np.concatenate([vals[b], p[2 * qw + kw:].reshape(1, kw)])
        att = oracle.attend_decode(q.reshape(-1), kk, vv, hq, hkv, dh, window, scale).reshape(-1)
        expect = (att * oracle.sigmoid(g)).astype(np.float32)
        assert np.array_equal(bits(got[b]), bits(expect)), f"seq {b}: max ulp {ulp_diff(got[b], expect).max()}"
    blocks = act_to_blocks(host(act, np.uint8), B, qw)
    for b in range(B):
        assert blocks[b].tobytes() == oracle.quantize_row_q8_0(got[b]).tobytes()


# a prefill chunk: M consecutive tokens of one sequence after p0 cached rows,
# all sharing cache 0 (the reference appends the whole batch, then reduces
# each row over its visible rows). max_ctx % 4 == 0 with no window takes the
# register softmax and the row-block weighted sum (blocks of 8 rows: 37 and
# 603 rows leave a partial last block; group 6 makes head chunks of 4 and 2;
# p0 = 4100 gives rows of more than 4096 keys, the chunked softmax);
# max_ctx % 4 != 0 and the window take the per-row kernels.
@pytest.mark.parametrize("M,p0,hq,hkv,max_ctx,window,dh", [(37, 0, 8, 2, 40, 0, 128), (603, 70, 32, 8, 676, 0, 128), (20, 33, 6, 1, 56, 0, 128),
                                                           (64, 4100, 8, 2, 4168, 0, 128), (10, 5, 4, 1, 17, 0, 128), (24, 9, 8, 2, 36, 7, 128),
                                                           (300, 40, 16, 4, 344, 0, 256), (12, 3, 8, 2, 17, 0, 256)])
def test_attn_prefill_rows_match_oracle(lib, M, p0, hq, hkv, max_ctx, window, dh):
    from hero_amd._lib import AttnDecodeArgs

    rng = np.random.default_rng(M + p0 + hq)
    qw, kw = hq * dh, hkv * dh
    stride = 2 * qw + 2 * kw
    qg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    eps = np.float32(1e-6)
    scale = np.float32(1.0) / np.sqrt(np.float32(dh)) if window == 0 else np.float32(1.0)
    inv = oracle.rope_inv_freq(dh, 1e6, 32)
    d_cs = dev(oracle.rope_table(dh, 1e6, 32, max_ctx))
    keys = (rng.standard_normal((p0, kw)) * 0.5).astype(np.float32)
    vals = rng.standard_normal((p0, kw)).astype(np.float32)
    kc = np.zeros((hkv, dh, max_ctx), np.float32)
    kc[:, :, :p0] = keys.reshape(p0, hkv, dh).transpose(1, 2, 0)
    vc = np.zeros((max_ctx, kw), np.float32)
    vc[:p0] = vals
    d_kc, d_vc = dev(kc), dev(vc)
    d_sc = empty(M * hq * max_ctx * 4)
    d_qr = empty(M * hq * dh * 4)
    act = empty(lib.hero_q8_0_act_bytes(M, qw))
    out = empty(M * qw * 4)
    proj = rng.standard_normal((M, stride)).astype(np.float32)
    d_proj, d_pos = dev(proj), dev(np.arange(p0, p0 + M, dtype=np.int32))
    d_qg, d_kg = dev(qg), dev(kg)
    a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), ptr(d_kc), ptr(d_vc),
                       max_ctx, ptr(d_pos), ptr(d_sc), ptr(d_qr), scale, window, ptr(act), ptr(out), M, hq, hkv, dh)
    check(lib.hero_attn_prefill(a, stream()))
    got = host(out, np.float32, (M, qw))
    # every row's key and value appended first, then each row reduced
    kk, vv = [keys], [vals]
    qs, gs = [], []
    for b in range(M):
        p = proj[b]
        q = np.stack([p[h * 2 * dh: h * 2 * dh + dh] for h in range(hq)])
        gs.append(np.concatenate([p[h * 2 * dh + dh: h * 2 * dh + 2 * dh] for h in range(hq)]))
        qs.append(oracle.rope_apply(oracle.rmsnorm(q, qg, eps), inv, p0 + b))
        kk.append(oracle.rope_apply(oracle.rmsnorm(p[2 * qw: 2 * qw + kw].reshape(hkv, dh), kg, eps), inv, p0 + b).reshape(1, kw))
        vv.append(p[2 * qw + kw:].reshape(1, kw))
    kk, vv = np.concatenate(kk), np.concatenate(vv)
    assert np.array_equal(bits(host(d_kc, np.float32, (hkv, dh, max_ctx))[:, :, :p0 + M]), bits(kk.reshape(-1, hkv, dh).transpose(1, 2, 0)))
    for b in range(M):
        att = oracle.attend_decode(qs[b].reshape(-1), kk[:p0 + b + 1], vv[:p0 + b + 1], hq, hkv, dh, window, scale).reshape(-1)
        expect = (att * oracle.sigmoid(gs[b])).astype(np.float32)
        assert np.array_equal(bits(got[b]), bits(expect)), f"row {b}: max ulp {ulp_diff(got[b], expect).max()}"
    blocks = act_to_blocks(host(act, np.uint8), M, qw)
    for b in range(M):
        assert blocks[b].tobytes() == oracle.quantize_row_q8_0(got[b]).tobytes(), f"row {b}"


@pytest.mark.parametrize("hq,window,page,dh", [(8, 0, 16, 128), (8, 50, 16, 128), (16, 0, 16, 128), (8, 0, 64, 128), (8, 50, 64, 128),
                                                (8, 70, 64, 128), (16, 0, 64, 128), (8, 0, 64, 256), (8, 70, 64, 256), (16, 50, 64, 256)])
def test_attn_paged_fp16_matches_oracle_over_fp16_kv(lib, hq, window, page, dh):
    """Split-K attention over the paged fp16 cache: pages of 16 positions (the
    per-key kernel: several pages per tile) or 64 (the page-streaming kernel:
    splits that start and end inside a page) in a shuffled pool, contexts up to
    300 (several splits), 4 and 8 query heads per KV head, full and windowed
    (windows of 50 and 70: splits not aligned to pages), heads of 128 and of
    256 channels (the reference's Qwen 3.5 4B / 9B width). The oracle
    attends over the same K/V rounded to fp16 (its storage), sequentially; the
    split kernel sums dot products by channel quarters with fused multiply-adds
    and merges the split softmax in another order, so the outputs agree within
    rtol 1e-4 + atol 1e-4 * max|out| (measured: a few 1e-6 absolute), and the
    quantized W_o input is the quantization of the kernel's own output."""
    from hero_amd._lib import AttnDecodeArgs, AttnPagedArgs

    rng = np.random.default_rng(23 + hq + window + page + dh)
    B, hkv, steps = 2, 2, 300
    max_pages = (320 + page - 1) // page
    max_ctx = page * max_pages
    qw, kw = hq * dh, hkv * dh
    stride = 2 * qw + 2 * kw
    qg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(dh)).astype(np.float32)
    eps = np.float32(1e-6)
    scale = np.float32(1.0) / np.sqrt(np.float32(dh)) if window == 0 else np.float32(1.0)
    inv = oracle.rope_inv_freq(dh, 1e6, 32)
    d_cs = dev(oracle.rope_table(dh, 1e6, 32, max_ctx))
    table = rng.permutation(B * max_pages).astype(np.int32).reshape(B, max_pages)
    d_table = dev(table)
    d_pages = empty(B * max_pages * 2 * hkv * page * dh * 2)
    wbytes = lib.hero_attn_paged_work_bytes(max_ctx, window, B, hq, hkv, dh)
    d_work = empty(wbytes)
    d_qr = empty(B * qw * 4)
    act = empty(lib.hero_q8_0_act_bytes(B, qw))
    out = empty(B * qw * 4)
    keys = [np.zeros((0, kw), np.float32) for _ in range(B)]
    vals = [np.zeros((0, kw), np.float32) for _ in range(B)]
    d_qg, d_kg = dev(qg), dev(kg)
    checked = 0
    for step in range(steps):
        proj = (rng.standard_normal((B, stride))).astype(np.float32)
        d_proj, d_pos = dev(proj), dev(np.array([step, step], np.int32))
        a = AttnDecodeArgs(ptr(d_proj), stride, 2 * qw, 2 * qw + kw, ptr(d_qg), ptr(d_kg), eps, ptr(d_cs), None, None,
                           0, ptr(d_pos), None, ptr(d_qr), scale, window, ptr(act), ptr(out), B, hq, hkv, dh)
        pa = AttnPagedArgs(a, ptr(d_pages), ptr(d_table), page, max_pages, ptr(d_work), wbytes)
        check(lib.hero_attn_decode_paged(pa, stream()))
        last = step in (0, 1, 63, 64, 65, 130, 200) or step == steps - 1
        for b in range(B):
            p = proj[b]
            k = oracle.rope_apply(oracle.rmsnorm(p[2 * qw: 2 * qw + kw].reshape(hkv, dh), kg, eps), inv, step)
            keys[b] = np.concatenate([keys[b], oracle.round_fp16(k.reshape(1, kw))])
            vals[b] = np.concatenate([vals[b], oracle.round_fp16(p[2 * qw + kw:].reshape(1, kw))])
        if not last:
            continue
        got = host(out, np.float32, (B, qw))
        blocks = act_to_blocks(host(act, np.uint8), B, qw)
        for b in range(B):
            p = proj[b]
            q = np.stack([p[h * 2 * dh: h * 2 * dh + dh] for h in range(hq)])
            g = np.concatenate([p[h * 2 * dh + dh: h * 2 * dh + 2 * dh] for h in range(hq)])
            q = oracle.rope_apply(oracle.rmsnorm(q, qg, eps), inv, step)
            att = oracle.attend_decode(q.reshape(-1), keys[b], vals[b], hq, hkv, dh, window, scale).reshape(-1)
            expect = (att * oracle.sigmoid(g)).astype(np.float32)
            np.testing.assert_allclose(got[b], expect, rtol=1e-4, atol=1e-4 * np.abs(expect).max(), err_msg=f"step {step} seq {b}")
            want = oracle.quantize_row_q8_0(got[b])
            assert blocks[b].tobytes() == want.tobytes()  # the kernel quantizes its own output exactly
            checked += 1
    assert checked == 16


# ---- K-quant weights (Q4_K / Q6_K against Q8_K activations) -------------------
def kquant_weights(rng, wtype, n, k):
    """random GGUF Q4_K / Q6_K blocks: random quants and scales, sane fp16 d"""
    nb = n * (k // 256)
    f16 = lambda a: np.asarray(a, np.float16).view(np.uint8).reshape(-1, 2)  # noqa: E731
    if wtype == oracle.Q4_K:
        w = np.concatenate([f16(rng.uniform(0.2, 2.0, nb) * 1e-2), f16(rng.uniform(0.0, 2.0, nb) * 1e-2),
                            rng.integers(0, 256, (nb, 140)).astype(np.uint8)], axis=1)
    else:
        w = np.concatenate([rng.integers(0, 256, (nb, 208)).astype(np.uint8), f16(rng.uniform(0.2, 2.0, nb) * 1e-3)], axis=1)
    return np.ascontiguousarray(w, np.uint8)


def kquant_pack_dev(lib, wtype, w, n, k):
    """a GGUF K-quant tensor on the device in its packed form"""
    raw = dev(np.ascontiguousarray(w, np.uint8))
    packed = empty(lib.hero_kquant_packed_bytes(wtype, n, k))
    check(lib.hero_kquant_pack(wtype, ptr(raw), ptr(packed), n, k, stream()))
    return packed


def kquant_dev(lib, wtype, w, x, n, k):
    m = x.shape[0]
    xd, wd = dev(x.astype(np.float32)), kquant_pack_dev(lib, wtype, w, n, k)
    act = empty(lib.hero_q8_K_act_bytes(m, k))
    check(lib.hero_q8_K_quantize(ptr(xd), ptr(act), m, k, stream()))
    y = empty(m * n * 4)
    check(lib.hero_kquant_gemm(wtype, ptr(wd), ptr(act), ptr(y), m, n, k, stream()))
    return host(act, np.uint8), host(y, np.float32).reshape(m, n)


def test_q8_K_quantizer_and_kquant_products_match_reference_golden(lib, kernels_golden):
    """the reference's own outputs: Q8_K blocks of 4 crafted rows, and
    Weight<4096,64>::matvec / ::matmul over raw Q4_K and Q6_K blocks"""
    x = kernels_golden["in_kq_x"].reshape(4, 4096)
    for wtype, name, out in [(oracle.Q4_K, "kq_w4", "kq_y4"), (oracle.Q6_K, "kq_w6", "kq_y6")]:
        act, y = kquant_dev(lib, wtype, kernels_golden[f"in_{name}"], x, 64, 4096)
        golden_act = kernels_golden["out_kq_act"]
        assert act[:golden_act.size].tobytes() == golden_act.tobytes()
        expect = kernels_golden[f"out_{out}"].reshape(5, 64)
        assert np.array_equal(bits(y[0]), bits(expect[0]))
        assert np.array_equal(bits(y), bits(expect[1:])), name


# K = 4096 / 12288 (the model's widths), 1024 and 2816 (blocks per row 4 and
# 11: Q6_K rows start off 16-byte boundaries), row counts not a multiple of a
# workgroup's rows, several activation rows
@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 12288, 4096), (2, 4096, 12288), (3, 1001, 1024), (1, 517, 2816), (16, 300, 4096)])
def test_kquant_gemm_matches_oracle_bitwise(lib, wtype, m, n, k):
    rng = np.random.default_rng(wtype * 1000 + m * 100 + n + k)
    w = kquant_weights(rng, wtype, n, k)
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-3, 3, (m, 1)))).astype(np.float32)
    act, y = kquant_dev(lib, wtype, w, x, n, k)
    expect_act = np.concatenate([oracle.quantize_row_q8_K(x[r]) for r in range(m)])
    assert act[:expect_act.size].tobytes() == expect_act.tobytes()
    # the regrouped copy after the blocks: per sub-block j, dword 8j + l holds
    # the int8 at 32j + l, +8, +16, +24
    off = (expect_act.size + 15) // 16 * 16
    q = expect_act[:, 4:260].reshape(-1, 8, 4, 8)             # [block][j][rep][l]
    regrouped = np.ascontiguousarray(q.transpose(0, 1, 3, 2))  # [block][j][l][rep]
    assert act[off:off + regrouped.size].tobytes() == regrouped.tobytes()
    expect = oracle.matmul_kquant(wtype, w, n, k, x)
    bad = np.flatnonzero(bits(y).ravel() != bits(expect).ravel())
    assert bad.size == 0, f"{bad.size} outputs differ, first {bad[:5]}: {y.ravel()[bad[:3]]} vs {expect.ravel()[bad[:3]]}"


# many activation rows (the prefill form: rows split over workgroups, each
# workgroup's weights reused across its rows) and the LM-head shape
@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("m,n,k", [(130, 256, 1024), (37, 1024, 2816), (64, 8192, 4096)])
def test_kquant_gemm_many_rows_matches_oracle_bitwise(lib, wtype, m, n, k):
    rng = np.random.default_rng(wtype * 7 + m + n + k)
    w = kquant_weights(rng, wtype, n, k)
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-3, 3, (m, 1)))).astype(np.float32)
    _, y = kquant_dev(lib, wtype, w, x, n, k)
    expect = oracle.matmul_kquant(wtype, w, n, k, x)
    bad = np.flatnonzero(bits(y).ravel() != bits(expect).ravel())
    assert bad.size == 0, f"{bad.size} outputs differ, first {bad[:5]}"


def q5k_weights(rng, n, k):
    nb = n * (k // 256)
    f16 = lambda a: np.asarray(a, np.float16).view(np.uint8).reshape(-1, 2)  # noqa: E731
    w = np.concatenate([f16(rng.uniform(0.2, 2.0, nb) * 1e-2), f16(rng.uniform(0.0, 2.0, nb) * 1e-2),
                        rng.integers(0, 256, (nb, 172)).astype(np.uint8)], axis=1)
    return np.ascontiguousarray(w, np.uint8)


def q5k_dev(lib, w, x, n, k):
    m = x.shape[0]
    wd, xd = kquant_pack_dev(lib, 13, w, n, k), dev(np.ascontiguousarray(x, np.float32))
    y = empty(m * n * 4)
    check(lib.hero_q5_K_gemm(ptr(wd), ptr(xd), ptr(y), m, n, k, stream()))
    return host(y, np.float32).reshape(m, n)


def test_q5_K_gemm_matches_reference_golden(lib, kernels_golden):
    """Weight<4096,64>::matvec / ::matmul over random Q5_K blocks: the
    reference's fp32-activation dequant-in-dot results"""
    x = kernels_golden["in_kq_x"].reshape(4, 4096)
    y = q5k_dev(lib, kernels_golden["in_kq_w5"], x, 64, 4096)
    expect = kernels_golden["out_kq_y5"].reshape(5, 64)
    assert np.array_equal(bits(y[0]), bits(expect[0]))
    assert np.array_equal(bits(y), bits(expect[1:]))


# the row-tile forms: 1 (decode), 4 (k <= 4096), 2 (k 8192), 1 (k 12288)
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 12288, 1024), (3, 1001, 1024), (130, 512, 4096), (9, 300, 8192),
                                   (5, 256, 12288), (17, 517, 2816)])
def test_q5_K_gemm_matches_oracle_bitwise(lib, m, n, k):
    rng = np.random.default_rng(m * 31 + n + k)
    w = q5k_weights(rng, n, k)
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-3, 3, (m, 1)))).astype(np.float32)
    y = q5k_dev(lib, w, x, n, k)
    expect = oracle.linear(oracle.Q5_K, w, n, k, x)
    bad = np.flatnonzero(bits(y).ravel() != bits(expect).ravel())
    assert bad.size == 0, f"{bad.size} outputs differ, first {bad[:5]}"


@pytest.mark.parametrize("wtype,name", [(12, "kq_w4"), (13, "kq_w5"), (14, "kq_w6")])
def test_kquant_dequant_rows_match_reference_golden(lib, kernels_golden, wtype, name):
    """Weight::dequant_row of rows 0 and 37 (the embedding gather), the
    reference's own values; plus rows of a random tensor against the oracle
    and an out-of-range id, which gives zeros"""
    w = kernels_golden[f"in_{name}"]
    wd = kquant_pack_dev(lib, wtype, w, 64, 4096)
    ids = dev(np.array([0, 37, 63, 64], np.int32))
    out = empty(4 * 4096 * 4)
    check(lib.hero_kquant_dequant_rows(wtype, ptr(wd), 64, 4096, ptr(ids), 4, ptr(out), stream()))
    got = host(out, np.float32).reshape(4, 4096)
    expect = kernels_golden["out_kq_dq" + {12: "4", 13: "5", 14: "6"}[wtype]].reshape(2, 4096)
    assert np.array_equal(bits(got[:2]), bits(expect))
    assert np.array_equal(bits(got[2]), bits(oracle.dequant_rows(wtype, np.ascontiguousarray(w).reshape(64, -1)[63], 1, 4096)[0]))
    assert not got[3].any()


def test_kquant_pack_permutes_the_tensor_bytes(lib):
    """the packed tensor holds the GGUF tensor's bytes, permuted, and zeros in
    its padding slots (40 rows of 4 blocks: one tile of 64 rows, 4 waves)"""
    rng = np.random.default_rng(5)
    for wtype in (12, 13, 14):
        w = q5k_weights(rng, 40, 1024) if wtype == 13 else kquant_weights(rng, wtype, 40, 1024)
        got = host(kquant_pack_dev(lib, wtype, w, 40, 1024), np.uint8)
        assert got.size == lib.hero_kquant_packed_bytes(wtype, 40, 1024)
        expect = np.concatenate([w.ravel(), np.zeros(got.size - w.size, np.uint8)])
        assert np.array_equal(np.sort(got), np.sort(expect)), wtype


# ---- top-k / top-p sampling -------------------------------------------------------------
def sample_dev(lib, logits_dev, v, k, temp, p, u):
    out = empty(8)
    check(lib.hero_sample_topk(ptr(logits_dev), v, k, temp, p, float(u), ptr(out), stream()))
    return int(host(out, np.int32)[0])


def sample_any_dev(lib, logits_dev, v, k, temp, p, u):
    wbytes = lib.hero_sample_work_bytes(v)
    assert wbytes > 0
    work, out = empty(wbytes), empty(8)
    check(lib.hero_sample(ptr(logits_dev), v, k, temp, p, float(u), ptr(work), wbytes, ptr(out), stream()))
    return int(host(out, np.int32)[0])


def test_sampler_matches_reference_golden(lib, kernels_golden):
    """Logits<32000>::sample, the reference's own picks; top_k 0 (the whole
    vocabulary) through the sorted form, every configuration through it too"""
    cfgs = [(0.7, 40, 0.9), (1.0, 1, 1.0), (1.3, 1000, 0.95), (0.5, 0, 1.0), (2.0, 200, 0.5), (0.9, 64, 0.0)]
    lg = kernels_golden["in_sample_logits"].reshape(8, 32000)
    res = kernels_golden["out_sample"].reshape(8, len(cfgs), 2)
    for r in range(8):
        d = dev(lg[r])
        for c, (temp, k, p) in enumerate(cfgs):
            if k > 0:
                assert sample_dev(lib, d, 32000, k, temp, p, res[r, c, 1]) == int(res[r, c, 0]), (r, c)
            assert sample_any_dev(lib, d, 32000, k, temp, p, res[r, c, 1]) == int(res[r, c, 0]), (r, c)


# the whole vocabulary (top_k 0) and k past the one-workgroup form, over the
# model's vocabulary: top_p cuts that stop in the first chunk of 4095 sorted
# logits, in a later one, and never (1.0); heavy ties (ids ascending)
@pytest.mark.parametrize("k,temp,p", [(0, 1.0, 1.0), (0, 0.7, 0.9), (0, 2.5, 0.999), (0, 0.3, 0.0), (5000, 1.2, 0.95), (151936, 1.0, 1.0)])
def test_sampler_whole_vocabulary_matches_oracle(lib, k, temp, p):
    rng = np.random.default_rng(k + int(temp * 10))
    v = 151936
    rows = [rng.standard_normal(v).astype(np.float32) * 2,
            np.round(rng.standard_normal(v) * 3).astype(np.float32)]  # heavy ties
    for x in rows:
        d = dev(x)
        for u in (0.0, 0.25, 0.5, 0.999):
            assert sample_any_dev(lib, d, v, k, temp, p, u) == oracle.sample_topk(x, k, temp, p, u), (k, temp, p, u)


# the model's vocabulary, k up to the device limit, top_p cuts, and a row of
# many equal logits (ties ordered by ascending id, as in the oracle)
@pytest.mark.parametrize("k,temp,p", [(1, 1.0, 1.0), (7, 0.6, 0.8), (40, 0.7, 0.9), (256, 1.5, 0.99), (1000, 1.0, 0.5), (1024, 3.0, 1.0)])
def test_sampler_matches_oracle(lib, k, temp, p):
    rng = np.random.default_rng(k)
    v = 151936
    rows = [rng.standard_normal(v).astype(np.float32) * 4,
            np.round(rng.standard_normal(v) * 8).astype(np.float32)]  # heavy ties
    for x in rows:
        d = dev(x)
        for u in (0.0, 0.123, 0.5, 0.987654):
            assert sample_dev(lib, d, v, k, temp, p, u) == oracle.sample_topk(x, k, temp, p, u), (k, temp, p, u)


@pytest.mark.parametrize("v,k", [(100, 1024), (1, 1), (1023, 500), (5000, 1024)])
def test_sampler_small_vocabularies(lib, v, k):
    """fewer logits than lanes (top_k above V means V), a single logit, and a
    vocabulary where k reaches past the lane-maximum bound"""
    rng = np.random.default_rng(v + k)
    x = (rng.standard_normal(v) * 3).astype(np.float32)
    d = dev(x)
    for u in (0.0, 0.31, 0.999):
        assert sample_dev(lib, d, v, k, 0.8, 0.95, u) == oracle.sample_topk(x, k, 0.8, 0.95, u), (v, k, u)
