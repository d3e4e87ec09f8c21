"""hero_amd.microbench -- the kernel microbenchmarks of the hot path on one GPU.

    python -m hero_amd.microbench [--suite hbm,gemv,kquant,gdn,attn] [--out results.md]

Suites (synthetic, seeded inputs; every launch goes through the C ABI):

hbm    the read ceiling: a kernel that only reads (hero_read_probe) over
       18 MB .. 2 GB fresh regions, 512 / 2048 / 8192 workgroups.
mall   the batch-1 GEMV of the decode step's shapes over cold weights and
       right after another kernel read the same weights (warm last-level
       cache), to price a prefetch into that cache.
kquant Q4_K / Q5_K / Q6_K products over packed random blocks, (K, N) as in
       gemv, M in {1, 16, 512}.

gemv   Q8_0 matvec / matmul. W is N x K int8 uniform in [-127, 127] with fp16
       block scales |N(0, 0.02)| * 4/127; activations are N(0, 1) rows
       quantized to Q8_0 beforehand. (K, N) in {(4096, 4096), (4096, 12288),
       (4096, 151936), (12288, 4096)} x M in {1, 8, 64, 512}: M = 1 runs the
       streaming GEMV, M > 1 the int8-MFMA GEMM. Enough distinct weight copies
       (>= 512 MB) rotate to keep the 256 MB last-level cache cold.
gdn    the fused delta-net layer body (conv + SiLU, L2 norms, gates, the delta
       rule on the fp32 state, head norm, gate, quantize) with 16 heads of
       128 x 128: one decode step at B in {1, 8, 32} from a state warmed by 64
       steps, and the prefill of 4096 tokens: the bit-exact token-serial scan
       and the chunked (WY) form with chunks of 64.
gemma4 the Gemma 4 E4B decode step (seeded synthetic 7.9 GB Q8_0 model): a
       --gemma4-ctx-token prompt, then 32 greedy passes replayed as one
       hipGraph each; ms per pass and the weight bytes a pass reads (every
       layer and the tied head, one per-layer-table row) per second.
attn   gated GQA decode (32 q / 8 kv heads of 128) at context {1k, 8k, 32k} x
       B {1, 16}: full causal (scale 1/sqrt(128)) and a 1024 sliding window
       (scale 1), over the fp32 cache (the reference's precision, bit-exact
       kernels) and over the paged fp16 and Q8_0 caches (split-K kernels).

Each case is captured once as a hipGraph (one pass over its inputs) and
replayed; the time per launch is the replay time divided by the launches,
so it includes the graph's inter-kernel gaps (about 1.7 us each) and is an
upper bound on the kernel's own duration (rocprofv3 --kernel-trace --stats
gives the latter). Algorithmic bytes follow the unit of work of each kernel:
GEMV/GEMM weights + scales + activations + outputs; delta-net state read and
write plus its per-token inputs and outputs; attention the visible K and V
rows plus q and the output.
"""
from __future__ import annotations

import argparse
import json
import math
import sys

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
CALIBRATION_BYTES = 512 << 20  # one known-size device-to-device copy (read and written once)
CALIBRATION_COPIES = 3


def _torch():
    import torch

    return torch


def _stream() -> int:
    return _torch().cuda.current_stream().cuda_stream


def _p(t) -> int:
    return t.data_ptr()


def _bytes(n: int):
    t = _torch()
    return t.empty(int(n), dtype=t.uint8, device="cuda")


DIRECT = 0  # --direct N: run each case N times as plain launches (no graph), for counter collection


def _time_graph(body, launches: int, replays: int, budget_s: float = 1.0) -> float:
    """seconds per launch of `body` (which makes `launches` launches), from
    hipGraph replays timed with events on the replay stream; at most
    `replays` replays and about `budget_s` seconds of them. With DIRECT set,
    `body` instead runs DIRECT times as plain launches (what a per-dispatch
    counter collection profiles)."""
    t = _torch()
    if DIRECT:
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(DIRECT):
            body()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / (DIRECT * launches)
    body()  # warm: code objects, caches
    t.cuda.synchronize()
    g = t.cuda.CUDAGraph()
    s = t.cuda.Stream()
    s.wait_stream(t.cuda.current_stream())
    with t.cuda.stream(s):
        with t.cuda.graph(g, stream=s):
            body()
    t.cuda.synchronize()
    e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    e1.synchronize()
    once = e0.elapsed_time(e1) * 1e-3
    n = max(1, min(replays, int(budget_s / max(once, 1e-9))))
    e0.record()
    for _ in range(n):
        g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / (n * launches)


# ---- Q8_0 GEMV / GEMM ----------------------------------------------------------------------
GEMV_SHAPES = [(4096, 4096), (4096, 12288), (4096, 151936), (12288, 4096)]
GEMV_BATCHES = [1, 8, 64, 512]


def _q8_weight_copies(lib, n: int, k: int, copies: int, gen):
    """`copies` packed Q8_0 weights of the benchmark distribution"""
    from ._lib import check

    t = _torch()
    nb = n * (k // 32)
    out = []
    for _ in range(copies):
        qs = t.randint(-127, 128, (nb, 32), dtype=t.int8, device="cuda", generator=gen)
        d = (t.randn(nb, device="cuda", generator=gen).abs() * (0.02 * 4 / 127)).half()
        blocks = t.cat([d.view(t.uint8).view(nb, 2), qs.view(t.uint8)], dim=1).contiguous()
        packed = _bytes(lib.hero_q8_0_packed_bytes(n, k))
        check(lib.hero_q8_0_pack(_p(blocks), _p(packed), n, k, 0, n, _stream()))
        del blocks, qs, d
        out.append(packed)
    t.cuda.synchronize()
    return out


def bench_gemv(lib, replays: int = 20, batches=GEMV_BATCHES):
    from ._lib import check

    t = _torch()
    gen = t.Generator(device="cuda")
    gen.manual_seed(1234)
    rows = []
    for k, n in GEMV_SHAPES:
        wbytes = n * k * 34 // 32
        copies = max(1, math.ceil(512e6 / wbytes))
        weights = _q8_weight_copies(lib, n, k, copies, gen)
        for m in batches:
            x = t.randn(m, k, device="cuda", generator=gen)
            act = _bytes(lib.hero_q8_0_act_bytes(m, k))
            check(lib.hero_q8_0_quantize(_p(x), _p(act), m, k, _stream()))
            y = t.empty(m, n, device="cuda")

            def body():
                for w in weights:
                    if m == 1:
                        check(lib.hero_q8_0_gemv(_p(w), _p(act), _p(y), None, n, k, _stream()))
                    else:
                        check(lib.hero_q8_0_gemm(_p(w), _p(act), _p(y), None, m, n, k, _stream()))

            def norm_body():
                # the decode step's form: RMSNorm + quantize of x fused as the GEMV's prologue
                for w in weights:
                    check(lib.hero_rmsnorm_q8_0_gemv(_p(w), _p(x), _p(gamma), 1e-6, _p(y), None, n, k, _p(act), _stream()))

            variants = [("gemv_q8_stream" if m == 1 else "gemm_q8 (int8 MFMA)", body)]
            if m == 1 and k == 4096:
                gamma = 1.0 + 0.1 * t.randn(k, device="cuda", generator=gen)
                variants.append(("gemv_q8_stream, RMSNorm prologue", norm_body))
            for name, fn in variants:
                sec = _time_graph(fn, len(weights), replays)
                nbytes = wbytes + m * k * 4 + m * n * 4  # the unit of work: weights + fp32 x in + fp32 y out
                ops = 2.0 * m * n * k
                rows.append({
                    "suite": "gemv", "kernel": name,
                    "K": k, "N": n, "M": m, "copies": copies, "us": sec * 1e6,
                    "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS,
                    "TOPS": ops / sec / 1e12, "int8_frac": ops / sec / 1e12 / INT8_PEAK_TOPS,
                })
                print(json.dumps(rows[-1]), flush=True)
            del act, y, x
        del weights
        t.cuda.empty_cache()
    return rows


# ---- K-quant GEMV / GEMM (Q4_K, Q6_K against Q8_K rows; Q5_K against fp32 rows) ---------------------
KQUANT_SHAPES = [(4096, 4096), (4096, 12288), (12288, 4096)]
KQUANT_BATCHES = (1, 16, 512)


def bench_kquant(lib, replays: int = 20, batches=KQUANT_BATCHES):
    """packed K-quant weights (hero_kquant_pack of random GGUF blocks with sane
    fp16 scales); algorithmic bytes = weights + activation rows as read (Q8_K
    blocks and their regrouped copy, or fp32) + outputs"""
    from ._lib import check

    t = _torch()
    gen = t.Generator(device="cuda")
    gen.manual_seed(4321)
    rows = []
    for wtype, name, bb in ((12, "Q4_K", 144), (13, "Q5_K", 176), (14, "Q6_K", 210)):
        for k, n in KQUANT_SHAPES:
            nb = n * (k // 256)
            wbytes = nb * bb
            copies = max(1, math.ceil(512e6 / wbytes))
            weights = []
            for _ in range(copies):
                w = t.randint(0, 256, (nb, bb), dtype=t.uint8, device="cuda", generator=gen)
                d = (t.rand(nb, device="cuda", generator=gen) * 0.01 + 0.002).half().view(t.uint8).view(nb, 2)
                if wtype in (12, 13):
                    w[:, 0:2] = d
                    w[:, 2:4] = d
                else:
                    w[:, 208:210] = d
                packed = _bytes(lib.hero_kquant_packed_bytes(wtype, n, k))
                check(lib.hero_kquant_pack(wtype, _p(w), _p(packed), n, k, _stream()))
                weights.append(packed)
                del w
            for m in batches:
                x = t.randn(m, k, device="cuda", generator=gen)
                y = t.empty(m, n, device="cuda")
                if wtype == 13:
                    act_bytes = m * k * 4

                    def body():
                        for w in weights:
                            check(lib.hero_q5_K_gemm(_p(w), _p(x), _p(y), m, n, k, _stream()))
                else:
                    act = _bytes(lib.hero_q8_K_act_bytes(m, k))
                    act_bytes = lib.hero_q8_K_act_bytes(m, k)
                    check(lib.hero_q8_K_quantize(_p(x), _p(act), m, k, _stream()))

                    def body():
                        for w in weights:
                            check(lib.hero_kquant_gemm(wtype, _p(w), _p(act), _p(y), m, n, k, _stream()))

                sec = _time_graph(body, len(weights), replays if m < 512 else 3)
                nbytes = wbytes + act_bytes + m * n * 4
                rows.append({"suite": "kquant", "kernel": f"kquant {name}", "K": k, "N": n, "M": m, "copies": copies,
                             "us": sec * 1e6, "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS,
                             "Gweight/s": m * n * k / sec / 1e9})
                print(json.dumps(rows[-1]), flush=True)
                del y, x
            del weights
            t.cuda.empty_cache()
    return rows


# ---- plain HBM read (the ceiling) ------------------------------------------------------------
HBM_READ_SIZES_MB = (18, 54, 107, 622, 2048)


def bench_hbm(lib, replays: int = 20):
    """hero_read_probe: contiguous shares, 16-byte loads, 8 in flight per lane.
    Timed like the kernels (hipGraph replays, so each launch includes the
    graph's inter-kernel gap): a replay reads up to 32 distinct regions of a
    4 GiB buffer back to back, more bytes than the 256 MB MALL holds, so every
    launch reads cold data."""
    from ._lib import check

    t = _torch()
    total = 4 << 30
    buf = t.empty(total, dtype=t.uint8, device="cuda").fill_(1)
    out = t.zeros(4, dtype=t.int32, device="cuda")
    rows = []
    for mb in HBM_READ_SIZES_MB:
        nbytes = mb << 20
        copies = max(1, min(32, total // nbytes - 1))
        for wg in (512, 2048, 8192):
            def body():
                for c in range(copies):
                    check(lib.hero_read_probe(buf.data_ptr() + c * nbytes, nbytes, wg, _p(out), _stream()))

            sec = _time_graph(body, copies, replays)
            rows.append({"suite": "hbm", "kernel": "read_probe", "MB": mb, "workgroups": wg, "copies": copies, "us": sec * 1e6,
                         "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS})
            print(json.dumps(rows[-1]), flush=True)
    del buf
    t.cuda.empty_cache()
    return rows


# ---- GEMV over weights another kernel has just read (warm last-level cache) ------------------------
MALL_SHAPES = [(4096, 4096), (12288, 4096), (4096, 16448), (4096, 24576)]  # (K, N): the decode step's GEMVs


def bench_mall(lib, replays: int = 20):
    """A batch-1 GEMV over cold weights (rotating copies, >= 512 MB, more than
    the 256 MB last-level cache holds) against the same GEMV right after a
    kernel that read its weights (hero_read_probe over the packed matrix, 512
    workgroups, or the same GEMV run once before). warm = time(reader, GEMV)
    - time(reader alone), per copy; all timed as graph replays, so each launch
    includes the graph's inter-kernel gap."""
    from ._lib import check

    t = _torch()
    gen = t.Generator(device="cuda")
    gen.manual_seed(4321)
    out = t.zeros(4, dtype=t.int32, device="cuda")
    rows = []
    for k, n in MALL_SHAPES:
        wbytes = lib.hero_q8_0_packed_bytes(n, k)
        copies = max(2, math.ceil(600e6 / wbytes))
        weights = _q8_weight_copies(lib, n, k, copies, gen)
        x = t.randn(1, k, device="cuda", generator=gen)
        act = _bytes(lib.hero_q8_0_act_bytes(1, k))
        check(lib.hero_q8_0_quantize(_p(x), _p(act), 1, k, _stream()))
        y = t.empty(1, n, device="cuda")

        def gemv(w):
            check(lib.hero_q8_0_gemv(_p(w), _p(act), _p(y), None, n, k, _stream()))

        def probe(w):
            check(lib.hero_read_probe(_p(w), wbytes, 512, _p(out), _stream()))

        def xcd_prefetch(w):
            check(lib.hero_q8_0_gemv_prefetch(_p(w), n, k, _stream()))

        cold = _time_graph(lambda: [gemv(w) for w in weights], len(weights), replays)
        probe_only = _time_graph(lambda: [probe(w) for w in weights], len(weights), replays)
        pair = _time_graph(lambda: [(probe(w), gemv(w)) for w in weights], len(weights), replays)
        twice = _time_graph(lambda: [(gemv(w), gemv(w)) for w in weights], len(weights), replays)
        cases = [("cold", cold), ("after read_probe", pair - probe_only), ("after the same GEMV", twice - cold),
                 ("read_probe alone (cold)", probe_only)]
        if k == 4096:
            pf_only = _time_graph(lambda: [xcd_prefetch(w) for w in weights], len(weights), replays)
            pf_pair = _time_graph(lambda: [(xcd_prefetch(w), gemv(w)) for w in weights], len(weights), replays)
            cases += [("after the XCD-matched prefetch", pf_pair - pf_only), ("XCD-matched prefetch alone (cold)", pf_only)]
        for name, sec in cases:
            kernel = "gemv_q8_stream" if "alone" not in name else "read_probe" if "read_probe" in name else "gemv_prefetch"
            rows.append({"suite": "mall", "kernel": kernel,
                         "K": k, "N": n, "MB": wbytes / 1e6, "weights": name, "copies": copies, "us": sec * 1e6,
                         "GB/s": wbytes / sec / 1e9, "hbm_frac": wbytes / sec / 1e9 / HBM_PEAK_GBS,
                         "vs_cold": cold / sec})
            print(json.dumps(rows[-1]), flush=True)
        del weights, act, y, x
        t.cuda.empty_cache()
    return rows


# ---- gated delta-net -----------------------------------------------------------------------------
def _gdn_case(lib, hk: int, hv: int, B: int, W: int, gen):
    from ._lib import GdnDecodeArgs

    t = _torch()
    dk = 128
    cc = 2 * hk * dk + hv * dk
    stride = cc + hv * dk + 2 * hv
    bufs = {
        "taps": (t.randn(cc, W, device="cuda", generator=gen) * 0.5),
        "dt": t.randn(hv, device="cuda", generator=gen) * 0.1,
        "decay": -t.exp(t.randn(hv, device="cuda", generator=gen) * 0.5),
        "gamma": 1 + 0.1 * t.randn(dk, device="cuda", generator=gen),
        "hist": t.zeros(B * W * cc, device="cuda"),
        "state": t.zeros(B * hv * dk * dk, device="cuda"),
        "proj": t.randn(B, stride, device="cuda", generator=gen),
        "act": _bytes(lib.hero_q8_0_act_bytes(B, hv * dk)),
        "pos": t.zeros(B, dtype=t.int32, device="cuda"),
    }
    a = GdnDecodeArgs(_p(bufs["proj"]), stride, cc, cc + hv * dk, cc + hv * dk + hv, _p(bufs["taps"]), _p(bufs["hist"]),
                      _p(bufs["state"]), _p(bufs["dt"]), _p(bufs["decay"]), _p(bufs["gamma"]), 1e-6, _p(bufs["pos"]),
                      _p(bufs["act"]), None, B, hk, hv, dk, dk, W)
    return a, bufs


def bench_gdn(lib, replays: int = 50):
    from ._lib import check

    t = _torch()
    gen = t.Generator(device="cuda")
    gen.manual_seed(4321)
    rows = []
    H, W, dk = 16, 4, 128
    for B in (1, 8, 32):
        # state copies enough that a replay reads the states cold (>= 512 MB,
        # more than the 256 MB last-level cache)
        copies = max(1, min(64, math.ceil(512e6 / (B * H * dk * dk * 4))))
        cases = [_gdn_case(lib, H, H, B, W, gen) for _ in range(copies)]
        for a, bufs in cases:
            for step in range(64):  # a seeded non-zero state
                bufs["pos"].fill_(step)
                check(lib.hero_gdn_decode(a, _stream()))
            bufs["pos"].fill_(64)
        o_raw = t.empty(B * H * dk, device="cuda")
        gates = t.empty(B * H * dk, device="cuda")

        def fused():
            for a, _ in cases:
                check(lib.hero_gdn_decode(a, _stream()))

        def cols():
            for a, _ in cases:
                check(lib.hero_gdn_decode_cols(a, _p(o_raw), _p(gates), _stream()))

        def cols_norm():
            for a, _ in cases:
                check(lib.hero_gdn_decode_cols(a, _p(o_raw), None, _stream()))
                check(lib.hero_gdn_norm_gate(_p(o_raw), a, _stream()))

        nbytes = B * H * dk * dk * 4 * 2 + B * H * (3 * 128 + 2) * 4 + B * H * 128 * 4
        for name, fn, launches in (("gdn_decode (fused layer body)", fused, 1),
                                   ("gdn_decode_cols (column split; the head norm and gate in the next GEMV's prologue)", cols, 1),
                                   ("gdn_decode_cols + gdn_norm_gate", cols_norm, 2)):
            sec = _time_graph(fn, len(cases), replays)  # per layer body (both launches of the last form)
            rows.append({"suite": "gdn", "kernel": name, "mode": "decode", "H": H, "B": B, "copies": copies,
                         "us": sec * 1e6, "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS})
            print(json.dumps(rows[-1]), flush=True)
        del cases
    T = 4096
    a, bufs = _gdn_case(lib, H, H, T, W, gen)
    wb = lib.hero_gdn_prefill_work_bytes(T, H, H)
    work = _bytes(wb)

    serial_flops = 7.0 * T * H * dk * dk
    C = 64
    chunk_flops = (T / C) * H * (6 * C * dk * dk + 8 * C * C * dk + C ** 3 / 3)  # the chunked form's unit of work
    for name, fn, flops in (("gdn_prefill (prep + token-serial scan + out, bit-exact)", lib.hero_gdn_prefill, serial_flops),
                            ("gdn_prefill_chunked (prep + chunked WY form, chunk 64 + out)", lib.hero_gdn_prefill_chunked, chunk_flops)):
        def prefill():
            bufs["state"].zero_()
            bufs["hist"].zero_()
            check(fn(a, _p(work), wb, _stream()))

        prefill()
        t.cuda.synchronize()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        reps = 5
        e0.record()
        for _ in range(reps):
            prefill()
        e1.record()
        e1.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / reps
        rows.append({"suite": "gdn", "kernel": name, "mode": "prefill", "H": H, "T": T, "us": sec * 1e6, "tok/s": T / sec,
                     "GFLOP/s": flops / sec / 1e9})
        print(json.dumps(rows[-1]), flush=True)
    return rows


# ---- GQA decode attention ------------------------------------------------------------------------
ATTN_CTX = (1024, 8192, 32768)
ATTN_BATCH = (1, 16)
ATTN_CACHES = ("fp32", "fp16", "q8")


ATTN_VARIANTS = ("full", "swa1024")


def bench_attn(lib, replays: int = 20, contexts=ATTN_CTX, batches=ATTN_BATCH, caches_run=ATTN_CACHES, variants=ATTN_VARIANTS):
    from ._lib import AttnDecodeArgs, AttnPagedArgs, check

    t = _torch()
    gen = t.Generator(device="cuda")
    gen.manual_seed(999)
    rows = []
    hq, hkv, dh = 32, 8, 128
    qw, kw = hq * dh, hkv * dh
    stride = 2 * qw + 2 * kw
    for ctx in contexts:
        for B in batches:
            cache_bytes = B * ctx * kw * 4 * 2
            copies = max(1, min(16, math.ceil(512e6 / cache_bytes)))
            scale = 1.0 / math.sqrt(dh)
            caches = []
            for _ in range(copies if "fp32" in caches_run else 0):
                kc = t.randn(B * ctx * kw, device="cuda", generator=gen) * scale
                vc = t.randn(B * ctx * kw, device="cuda", generator=gen) * scale
                caches.append((kc, vc))
            proj = t.randn(B, stride, device="cuda", generator=gen) * scale
            gq, gk = t.ones(dh, device="cuda"), t.ones(dh, device="cuda")
            cs = t.zeros(ctx, dh // 2, 2, device="cuda")
            cs[..., 0] = 1.0
            pos = t.full((B,), ctx - 1, dtype=t.int32, device="cuda")
            scores = t.empty(B * hq * ctx, device="cuda")
            qrot = t.empty(B * qw, device="cuda")
            act = _bytes(lib.hero_q8_0_act_bytes(B, qw))
            for name, window, sc in [v for v in (("full", 0, scale), ("swa1024", 1024, 1.0)) if v[0] in variants] if caches else ():
                args = [AttnDecodeArgs(_p(proj), stride, 2 * qw, 2 * qw + kw, _p(gq), _p(gk), 1e-6, _p(cs), _p(kc), _p(vc), ctx,
                                       _p(pos), _p(scores), _p(qrot), sc, window, _p(act), None, B, hq, hkv, dh)
                        for kc, vc in caches]

                def body():
                    for a in args:
                        check(lib.hero_attn_decode(a, _stream()))

                sec = _time_graph(body, len(args), replays)
                l_eff = ctx if window == 0 else min(ctx, window)
                nbytes = B * l_eff * kw * 4 * 2 + B * (qw + 2 * kw + qw) * 4
                rows.append({"suite": "attn", "kernel": "attn_decode (prep + scores + softmax + pv), fp32 K/V",
                             "variant": name, "ctx": ctx, "B": B, "copies": copies, "us": sec * 1e6,
                             "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS})
                print(json.dumps(rows[-1]), flush=True)
            del caches, scores
            t.cuda.empty_cache()
            # the same over the paged fp16 cache (pages of 64 positions, split-K)
            page = 64
            max_pages = ctx // page
            pages = [(t.randn(B * max_pages * 2 * hkv * page * dh, device="cuda", generator=gen) * scale).half()
                      for _ in range(max(1, min(16, math.ceil(512e6 / (cache_bytes // 2)))) if "fp16" in caches_run else 0)]
            table = t.arange(B * max_pages, dtype=t.int32, device="cuda")
            for name, window, sc in [v for v in (("full", 0, scale), ("swa1024", 1024, 1.0)) if v[0] in variants] if pages else ():
                wbytes = lib.hero_attn_paged_work_bytes(ctx, window, B, hq, hkv, dh)
                work = _bytes(wbytes)
                args = []
                for pg in pages:
                    a = AttnDecodeArgs(_p(proj), stride, 2 * qw, 2 * qw + kw, _p(gq), _p(gk), 1e-6, _p(cs), None, None, 0,
                                       _p(pos), None, _p(qrot), sc, window, _p(act), None, B, hq, hkv, dh)
                    args.append(AttnPagedArgs(a, _p(pg), _p(table), page, max_pages, _p(work), wbytes))

                def body():
                    for pa in args:
                        check(lib.hero_attn_decode_paged(pa, _stream()))

                sec = _time_graph(body, len(args), replays)
                l_eff = ctx if window == 0 else min(ctx, window)
                nbytes = B * l_eff * kw * 2 * 2 + B * (qw + 2 * kw + qw) * 4
                rows.append({"suite": "attn", "kernel": "attn_decode_paged (prep + split-K + combine), fp16 K/V",
                             "variant": name, "ctx": ctx, "B": B, "copies": len(pages), "us": sec * 1e6,
                             "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS})
                print(json.dumps(rows[-1]), flush=True)
                del work
            del pages
            t.cuda.empty_cache()
            # the same over Q8_0 pages: int8 rows (random) and fp16 block
            # scales of the inputs' size (|N(0,1)|/sqrt(128) max / 127)
            pb = lib.hero_attn_page_bytes(hkv, dh, page, 1)
            pages8 = []
            for _ in range(max(1, min(16, math.ceil(512e6 / (B * max_pages * pb)))) if "q8" in caches_run else 0):
                pg = t.randint(-127, 128, (B * max_pages, pb), dtype=t.int8, device="cuda", generator=gen).view(t.uint8)
                q_bytes = 2 * hkv * page * dh
                d = t.full((B * max_pages, (pb - q_bytes) // 2), 3.0 * scale / 127.0, device="cuda").half()
                pg[:, q_bytes:] = d.view(t.uint8)
                pages8.append(pg.contiguous())
            for name, window, sc in [v for v in (("full", 0, scale), ("swa1024", 1024, 1.0)) if v[0] in variants] if pages8 else ():
                wbytes = lib.hero_attn_paged_work_bytes(ctx, window, B, hq, hkv, dh)
                work = _bytes(wbytes)
                args = []
                for pg in pages8:
                    a = AttnDecodeArgs(_p(proj), stride, 2 * qw, 2 * qw + kw, _p(gq), _p(gk), 1e-6, _p(cs), None, None, 0,
                                       _p(pos), None, _p(qrot), sc, window, _p(act), None, B, hq, hkv, dh)
                    args.append(AttnPagedArgs(a, _p(pg), _p(table), page, max_pages, _p(work), wbytes, 1))

                def body():
                    for pa in args:
                        check(lib.hero_attn_decode_paged(pa, _stream()))

                sec = _time_graph(body, len(args), replays)
                l_eff = ctx if window == 0 else min(ctx, window)
                nbytes = B * l_eff * kw * 2 * (1 + 2 / 32) + B * (qw + 2 * kw + qw) * 4
                rows.append({"suite": "attn", "kernel": "attn_decode_paged (prep + split-K + combine), Q8_0 K/V",
                             "variant": name, "ctx": ctx, "B": B, "copies": len(pages8), "us": sec * 1e6,
                             "GB/s": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS})
                print(json.dumps(rows[-1]), flush=True)
                del work
            del pages8
            t.cuda.empty_cache()
    return rows


def bench_gemma4(lib, ctx: int = 600, passes: int = 32):
    import time

    import numpy as np

    from .gemma4 import GEMMA4_E4B, Gemma4Model, synthetic_gemma4_image

    shape = GEMMA4_E4B
    image = synthetic_gemma4_image(shape, seed=4242)
    model = Gemma4Model.open_image(image)
    del image
    d = model.dims
    pl = d.per_layer_input * d.layers
    table = lambda n, k: n * k + (n + 7) // 8 * 8 * (k // 32) * 2  # noqa: E731  packed Q8_0 bytes
    step_bytes = d.device_bytes - table(d.vocab, pl) + pl * 17 // 16
    prompt = np.random.default_rng(4242).integers(0, d.vocab, ctx).astype(np.int32)
    state = model.new_state(ctx + passes + 1)
    t = time.perf_counter()
    first = model.forward(state, prompt, want_logits=False)
    prompt_s = time.perf_counter() - t
    model.decode_greedy(state, first, passes)
    sec = model.last_decode_seconds()
    ms = sec * 1e3 / passes
    gbs = step_bytes / (sec / passes) / 1e9
    print(f"gemma4 e4b decode at context {ctx}: {ms:.3f} ms/pass, {1e3 / ms:.1f} tok/s, {gbs:.0f} GB/s of weights", file=sys.stderr)
    model.close()
    return [{"suite": "gemma4", "model": "gemma4-e4b (synthetic Q8_0)", "context": ctx, "passes": passes, "prompt_s (token by token)": prompt_s,
             "ms_per_pass": ms, "tok_s": 1e3 / ms, "weight_MB_per_pass": step_bytes / 1e6, "weight_GBps": gbs, "frac_8TBps": gbs / 8000.0}]


def _markdown(rows) -> str:
    out = []
    for suite in ("hbm", "mall", "gemv", "kquant", "gdn", "attn", "gemma4"):
        rs = [r for r in rows if r["suite"] == suite]
        if not rs:
            continue
        keys = [k for k in rs[0] if k != "suite"]
        for r in rs[1:]:
            keys += [k for k in r if k not in keys and k != "suite"]
        out.append(f"### {suite}\n")
        out.append("| " + " | ".join(keys) + " |")
        out.append("|" + "---|" * len(keys))
        for r in rs:
            cells = []
            for k in keys:
                v = r.get(k, "")
                cells.append(f"{v:.4g}" if isinstance(v, float) else str(v))
            out.append("| " + " | ".join(cells) + " |")
        out.append("")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--suite", default="gemv,gdn,attn")
    ap.add_argument("--out", default=None, help="write a markdown table here")
    ap.add_argument("--gemv-batches", default=",".join(map(str, GEMV_BATCHES)), help="activation rows M of the gemv suite")
    ap.add_argument("--attn-ctx", default=",".join(map(str, ATTN_CTX)), help="contexts of the attn suite")
    ap.add_argument("--attn-batch", default=",".join(map(str, ATTN_BATCH)), help="batches of the attn suite")
    ap.add_argument("--attn-cache", default=",".join(ATTN_CACHES), help="caches of the attn suite: fp32, fp16 (paged), q8 (paged)")
    ap.add_argument("--attn-variant", default=",".join(ATTN_VARIANTS), help="variants of the attn suite: full, swa1024")
    ap.add_argument("--gemma4-ctx", type=int, default=600, help="prompt tokens before the gemma4 suite's decode passes")
    ap.add_argument("--direct", type=int, default=0, help="run each case this many times as plain launches instead of graph replays")
    ap.add_argument("--calibrate", action="store_true",
                    help="first copy 512 MiB device to device three times: the known-size dispatches hero_amd.traffic calibrates "
                         "FETCH_SIZE / WRITE_SIZE with")
    args = ap.parse_args(argv)
    t = _torch()
    if not t.cuda.is_available():
        print("microbench: needs a GPU", file=sys.stderr)
        return 2
    from ._lib import lib

    global DIRECT
    DIRECT = args.direct
    if args.calibrate:
        src = t.empty(CALIBRATION_BYTES, dtype=t.uint8, device="cuda").fill_(1)
        dst = t.empty_like(src)
        for _ in range(CALIBRATION_COPIES):
            dst.copy_(src)
        t.cuda.synchronize()
        del src, dst

    rows = []
    suites = args.suite.split(",")
    if "gemv" in suites:
        rows += bench_gemv(lib, batches=[int(v) for v in args.gemv_batches.split(",")])
    if "hbm" in suites:
        rows += bench_hbm(lib)
    if "mall" in suites:
        rows += bench_mall(lib)
    if "kquant" in suites:
        rows += bench_kquant(lib)
    if "gdn" in suites:
        rows += bench_gdn(lib)
    if "attn" in suites:
        rows += bench_attn(lib, contexts=[int(v) for v in args.attn_ctx.split(",")], batches=[int(v) for v in args.attn_batch.split(",")],
                           caches_run=args.attn_cache.split(","), variants=args.attn_variant.split(","))
    if "gemma4" in suites:
        rows += bench_gemma4(lib, ctx=args.gemma4_ctx)
    md = _markdown(rows)
    if args.out:
        with open(args.out, "w") as f:
            f.write(md + "\n")
    print(md, file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
