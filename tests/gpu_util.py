"""Device-memory plumbing for the GPU tests: torch allocates, the C ABI computes."""
from __future__ import annotations

import numpy as np

import oracle


def torch():
    import torch as _t

    return _t


def dev(a: np.ndarray):
    """numpy -> device tensor (same bytes)"""
    t = torch()
    a = np.ascontiguousarray(a)
    return t.from_numpy(a.view(np.uint8).reshape(-1).copy()).to("cuda")


def empty(nbytes: int):
    return torch().zeros(int(nbytes), dtype=torch().uint8, device="cuda")


def host(t, dtype, shape=None) -> np.ndarray:
    torch().cuda.synchronize()
    a = t.cpu().numpy().view(dtype)
    return a.reshape(shape) if shape is not None else a


def ptr(t) -> int:
    return t.data_ptr()


def stream() -> int:
    return torch().cuda.current_stream().cuda_stream


def pack_weight(lib, blocks: np.ndarray, n: int, k: int):
    """oracle Q8_0 blocks [n][k/32] -> packed device weight"""
    from hero_amd._lib import check

    src = dev(blocks)
    packed = empty(lib.hero_q8_0_packed_bytes(n, k))
    check(lib.hero_q8_0_pack(ptr(src), ptr(packed), n, k, 0, n, stream()))
    return packed


def act_to_blocks(act: np.ndarray, m: int, k: int) -> np.ndarray:
    """device act layout [m*k int8][m*k/32 fp32] -> Q8_0 blocks [m][k/32]"""
    qs = act[: m * k].view(np.int8).reshape(m, k // 32, 32)
    d = act[m * k: m * k + m * (k // 32) * 4].view(np.float32).reshape(m, k // 32)
    out = np.zeros((m, k // 32), oracle.BLOCK)
    out["qs"] = qs
    out["d"] = d.astype(np.float16).view(np.uint16)  # exact: d is an fp16 value
    assert np.array_equal(out["d"].view(np.float16).astype(np.float32), d)
    return out


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ulp_diff(a, b) -> np.ndarray:
    """|a - b| in units of fp32 ulps (sign-magnitude ordering)"""
    def key(x):
        u = bits(x).astype(np.int64)
        return np.where(u & 0x80000000, 0x80000000 - u, u)

    return np.abs(key(a) - key(b))


def check(rc):
    from hero_amd._lib import check as _check

    _check(rc)


def quantize_dev(lib, x: np.ndarray):
    m, k = x.shape
    xd = dev(x.astype(np.float32))
    act = empty(lib.hero_q8_0_act_bytes(m, k))
    check(lib.hero_q8_0_quantize(ptr(xd), ptr(act), m, k, stream()))
    return act


def gdn_reference(proj, taps, hist, state, dt, decay, gamma, eps, hk, hv, pos):
    """one token through the oracle's pieces, in mix_tokens order (qwen35.hpp:420-462)"""
    dk = 128
    kw, cc = hk * dk, 2 * hk * dk + hv * dk
    stream_ = oracle.silu(oracle.conv_step(proj[:cc], taps, hist))
    q = np.concatenate([oracle.l2_normalize(stream_[i * dk:(i + 1) * dk]) for i in range(hk)])
    qs = np.float32(1.0) / np.sqrt(np.float32(dk))
    q = (q * qs).astype(np.float32)
    k = np.concatenate([oracle.l2_normalize(stream_[kw + i * dk: kw + (i + 1) * dk]) for i in range(hk)])
    v = stream_[2 * kw:]
    beta = oracle.sigmoid(proj[cc + hv * dk: cc + hv * dk + hv])
    alpha = proj[cc + hv * dk + hv: cc + hv * dk + 2 * hv]
    gate = (decay * oracle.softplus((alpha + dt).astype(np.float32))).astype(np.float32)
    o = oracle.gated_delta_step(state, q, k, v, gate, beta, hk)
    o = oracle.rmsnorm(o, gamma, eps).reshape(-1)
    z = proj[cc: cc + hv * dk]
    return (o * oracle.silu(z)).astype(np.float32)
