"""The oracle: a CPU restatement of the reference engine's Q8_0 Qwen 3.5 hybrid
path (oracle.cpp, built into liboracle.so by oracle/Makefile).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may use it, and only as the checker or the
timed CPU baseline -- never as part of the product path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_size_t, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_HARNESS = os.path.join(HERE, "_ref", "ref_harness")

_sigs = {
    "oracle_last_error": (c_char_p, []),
    "oracle_set_threads": (None, [c_size_t]),
    "oracle_threads": (c_size_t, []),
    "oracle_fp16_to_fp32": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_fp32_to_fp16": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_quantize_row_q8_0": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_quantize_q8_0": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_vec_dot_q8_0": (c_float, [c_size_t, c_void_p, c_void_p]),
    "oracle_block_sums_q8_0": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "oracle_matvec_q8_0": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "oracle_sample_topk": (c_int32, [c_void_p, c_size_t, c_size_t, c_float, c_float, c_float]),
    "oracle_quantize_row_q8_K": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_vec_dot_kquant": (c_float, [c_int, c_void_p, c_void_p, c_size_t]),
    "oracle_matmul_kquant": (None, [c_int, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p]),
    "oracle_dot_block_q5_K": (c_float, [c_void_p, c_void_p]),
    "oracle_linear_rows": (c_int, [c_int, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p]),
    "oracle_dequant_rows": (c_int, [c_int, c_void_p, c_size_t, c_size_t, c_void_p]),
    "oracle_matmul_q8_0": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p]),
    "oracle_rmsnorm_rows": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_float]),
    "oracle_l2_normalize": (None, [c_void_p, c_void_p, c_size_t, c_float]),
    "oracle_silu": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_sigmoid": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_softplus": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_softmax": (None, [c_void_p, c_size_t]),
    "oracle_expf": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_log1pf": (None, [c_void_p, c_void_p, c_size_t]),
    "oracle_conv_step": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t]),
    "oracle_gated_delta_step": (None, [c_void_p] * 7 + [c_size_t] * 4),
    "oracle_rope_inv_freq": (None, [c_size_t, c_double, c_size_t, c_void_p]),
    "oracle_rope_table": (None, [c_size_t, c_double, c_size_t, c_size_t, c_void_p]),
    "oracle_rope_apply": (None, [c_void_p, c_size_t, c_void_p, c_size_t, c_size_t]),
    "oracle_attend_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_size_t, c_size_t, c_float, c_void_p]),
    "oracle_model_set_kv_fp16": (None, [c_void_p, c_int]),
    "oracle_model_set_kv_q8": (None, [c_void_p, c_int]),
    "oracle_round_fp16": (None, [c_void_p, c_size_t, c_void_p]),
    "oracle_model_open": (c_void_p, [c_char_p]),
    "oracle_model_open_image": (c_void_p, [c_void_p, c_size_t]),
    "oracle_model_close": (None, [c_void_p]),
    "oracle_model_dims": (None, [c_void_p, c_void_p]),
    "oracle_model_reset": (None, [c_void_p]),
    "oracle_model_tokens": (c_size_t, [c_void_p]),
    "oracle_model_embed": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "oracle_model_forward": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "oracle_model_forward_ids": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "oracle_argmax": (c_int32, [c_void_p, c_size_t]),
    "oracle_model_greedy": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, POINTER(c_double), POINTER(c_double)]),
    "oracle_gemma4_open": (c_void_p, [c_char_p]),
    "oracle_gemma4_open_image": (c_void_p, [c_void_p, c_size_t]),
    "oracle_gemma4_close": (None, [c_void_p]),
    "oracle_gemma4_dims": (None, [c_void_p, c_void_p]),
    "oracle_gemma4_reset": (None, [c_void_p]),
    "oracle_gemma4_tokens": (c_size_t, [c_void_p]),
    "oracle_gemma4_kv_source": (c_size_t, [c_void_p, c_size_t]),
    "oracle_gemma4_embed": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "oracle_gemma4_forward": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "oracle_gemma_math": (None, [c_void_p, c_void_p, c_size_t, c_float]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run make -C oracle")
    lib = ctypes.CDLL(LIB_PATH)
    for n, (r, a) in _sigs.items():
        f = getattr(lib, n)
        f.restype = r
        f.argtypes = a
    return lib


lib = _load()
BLOCK = np.dtype([("d", "<u2"), ("qs", "i1", 32)])  # Q8_0 block, 34 bytes


def _p(a):
    return a.ctypes.data if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib.oracle_set_threads(n)


def threads() -> int:
    return int(lib.oracle_threads())


def fp16_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib.oracle_fp16_to_fp32(_p(h), _p(out), h.size)
    return out


def fp32_to_fp16(f):
    f = _f32(f)
    out = np.empty(f.shape, np.uint16)
    lib.oracle_fp32_to_fp16(_p(f), _p(out), f.size)
    return out


def quantize_row_q8_0(x):
    """activation quantizer (roundf) -> Q8_0 blocks [K/32]"""
    x = _f32(x).ravel()
    out = np.zeros(x.size // 32, BLOCK)
    lib.oracle_quantize_row_q8_0(_p(x), _p(out), x.size)
    return out


def quantize_q8_0(x):
    """weight quantizer (lround) -> Q8_0 blocks, row-major"""
    x = _f32(x)
    out = np.zeros(x.size // 32, BLOCK)
    lib.oracle_quantize_q8_0(_p(x), _p(out), x.size)
    return out


def vec_dot_q8_0(w_blocks, x_blocks) -> np.float32:
    return np.float32(lib.oracle_vec_dot_q8_0(w_blocks.size * 32, _p(w_blocks), _p(x_blocks)))


def block_sums(w_blocks, n, k, x_blocks):
    out = np.empty((n, k // 32), np.int32)
    lib.oracle_block_sums_q8_0(_p(w_blocks), n, k, _p(x_blocks), _p(out))
    return out


def matvec(w_blocks, n, k, x):
    x = _f32(x)
    y = np.empty(n, np.float32)
    lib.oracle_matvec_q8_0(_p(w_blocks), n, k, _p(x), _p(y))
    return y


def matmul(w_blocks, n, k, X):
    X = _f32(X)
    t = X.shape[0]
    Y = np.empty((t, n), np.float32)
    lib.oracle_matmul_q8_0(_p(w_blocks), n, k, _p(X), t, _p(Y))
    return Y


def sample_topk(logits, top_k, temp, top_p, u) -> int:
    """Logits::sample (temp > 0) given the uniform draw u in [0, 1)"""
    x = _f32(logits).ravel()
    return int(lib.oracle_sample_topk(_p(x), x.size, int(top_k), float(temp), float(top_p), float(u)))


# ---- K-quants (GGUF types 12 = Q4_K, 14 = Q6_K; activations as Q8_K) ----------
Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
KBLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210}


def row_bytes(wtype, k):
    return k // 32 * 34 if wtype == Q8_0 else k // 256 * KBLOCK_BYTES[wtype]
Q8K_BYTES = 292


def quantize_row_q8_K(x):
    """K-quant activation quantizer -> raw Q8_K blocks, uint8 [K/256, 292]"""
    x = _f32(x).ravel()
    out = np.zeros((x.size // 256, Q8K_BYTES), np.uint8)
    lib.oracle_quantize_row_q8_K(_p(x), _p(out), x.size)
    return out


def vec_dot_kquant(wtype, w_row, x_blocks) -> np.float32:
    """one row of raw Q4_K/Q6_K blocks against raw Q8_K blocks"""
    w_row = np.ascontiguousarray(w_row, np.uint8)
    x_blocks = np.ascontiguousarray(x_blocks, np.uint8)
    return np.float32(lib.oracle_vec_dot_kquant(wtype, _p(w_row), _p(x_blocks), x_blocks.size // Q8K_BYTES * 256))


def matmul_kquant(wtype, w, n, k, X):
    """Weight::matvec/matmul for a raw Q4_K/Q6_K tensor [n rows of k/256 blocks]"""
    w = np.ascontiguousarray(w, np.uint8)
    assert w.size == n * (k // 256) * KBLOCK_BYTES[wtype]
    X = _f32(X).reshape(-1, k)
    Y = np.empty((X.shape[0], n), np.float32)
    lib.oracle_matmul_kquant(wtype, _p(w), n, k, _p(X), X.shape[0], _p(Y))
    return Y


def dot_block_q5_K(block, x) -> np.float32:
    """fp32-activation dot of one raw Q5_K block (176 bytes) with 256 floats"""
    block = np.ascontiguousarray(block, np.uint8)
    x = _f32(x).ravel()
    assert block.size == 176 and x.size == 256
    return np.float32(lib.oracle_dot_block_q5_K(_p(block), _p(x)))


def linear(wtype, w, n, k, X):
    """Weight::matmul of a raw tensor of any linear type (Q8_0 as stored in the
    GGUF, Q4_K, Q5_K, Q6_K): Y[T, n]"""
    w = np.ascontiguousarray(w, np.uint8)
    assert w.size == n * row_bytes(wtype, k)
    X = _f32(X).reshape(-1, k)
    Y = np.empty((X.shape[0], n), np.float32)
    if lib.oracle_linear_rows(wtype, _p(w), n, k, _p(X), X.shape[0], _p(Y)) != 0:
        raise ValueError(f"linear: unsupported type {wtype}")
    return Y


def dequant_rows(wtype, w, rows, k):
    """rows of a raw tensor dequantized to fp32 (the embedding gather)"""
    w = np.ascontiguousarray(w, np.uint8)
    assert w.size >= rows * row_bytes(wtype, k)
    out = np.empty((rows, k), np.float32)
    if lib.oracle_dequant_rows(wtype, _p(w), rows, k, _p(out)) != 0:
        raise ValueError(f"dequant: unsupported type {wtype}")
    return out


def rmsnorm(x, gamma, eps=1e-6):
    x = _f32(x).copy()
    g = _f32(gamma)
    rows = x.size // g.size
    lib.oracle_rmsnorm_rows(_p(x), _p(g), rows, g.size, eps)
    return x


def l2_normalize(x, eps=1e-6):
    x = _f32(x)
    out = np.empty_like(x)
    lib.oracle_l2_normalize(_p(x), _p(out), x.size, eps)
    return out


def _map(fn, x):
    x = _f32(x)
    out = np.empty_like(x)
    fn(_p(x), _p(out), x.size)
    return out


def silu(x):
    return _map(lib.oracle_silu, x)


def sigmoid(x):
    return _map(lib.oracle_sigmoid, x)


def softplus(x):
    return _map(lib.oracle_softplus, x)


def expf(x):
    return _map(lib.oracle_expf, x)


def log1pf(x):
    return _map(lib.oracle_log1pf, x)


def softmax(v):
    v = _f32(v).copy()
    lib.oracle_softmax(_p(v), v.size)
    return v


def conv_step(x, taps, history):
    """one causal conv step; history [(W-1)][C] oldest first is updated in place"""
    x = _f32(x)
    taps = _f32(taps)
    c, w = taps.shape
    out = np.empty(c, np.float32)
    lib.oracle_conv_step(_p(x), _p(taps), _p(history), _p(out), c, w)
    return out


def gated_delta_step(state, q, k, v, gate, beta, key_heads):
    """all heads of one token; state [H][Dk][Dv] updated in place"""
    h, dk, dv = state.shape
    out = np.empty((h, dv), np.float32)
    q, k, v = _f32(q), _f32(k), _f32(v)
    gate, beta = _f32(gate), _f32(beta)
    lib.oracle_gated_delta_step(_p(state), _p(q), _p(k), _p(v), _p(gate), _p(beta), _p(out), h, key_heads, dk, dv)
    return out


def rope_inv_freq(head_dim, base, rotary_dims):
    out = np.empty(head_dim // 2, np.float32)
    lib.oracle_rope_inv_freq(head_dim, base, rotary_dims, _p(out))
    return out


def rope_table(head_dim, base, rotary_dims, positions):
    out = np.empty((positions, head_dim // 2, 2), np.float32)
    lib.oracle_rope_table(head_dim, base, rotary_dims, positions, _p(out))
    return out


def rope_apply(heads, inv_freq, position):
    heads = _f32(heads).copy()
    hd = inv_freq.size * 2
    lib.oracle_rope_apply(_p(heads), heads.size // hd, _p(_f32(inv_freq)), hd, position)
    return heads


def round_fp16(x):
    """IEEE fp16 round-to-nearest-even of fp32 values (the fp16 cache's storage)"""
    x = _f32(x)
    out = np.empty_like(x)
    lib.oracle_round_fp16(_p(x), x.size, _p(out))
    return out


def attend_decode(q, keys, values, hq, hkv, head_dim, window, scale):
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    ctx = keys.shape[0]
    out = np.empty((hq, head_dim), np.float32)
    if lib.oracle_attend_decode(_p(q), _p(keys), _p(values), ctx, hq, hkv, head_dim, window, scale, _p(out)) != 0:
        raise RuntimeError(lib.oracle_last_error().decode())
    return out


class Model:
    """The oracle's Qwen 3.5 model over a GGUF file or an in-memory image."""

    def __init__(self, path: str | None = None, image: np.ndarray | None = None):
        if path is not None:
            self._h = lib.oracle_model_open(path.encode())
        else:
            self._image = image
            self._h = lib.oracle_model_open_image(_p(image), image.nbytes)
        if not self._h:
            raise RuntimeError(lib.oracle_last_error().decode())
        dims = np.zeros(15, np.uint64)
        lib.oracle_model_dims(self._h, _p(dims))
        (self.V, self.D, self.L, self.CTX, self.Hq, self.Hkv, self.head_dim, self.rotary_dims,
         self.Dk, self.Dv, self.Hk, self.Hv, self.conv_width, self.FF, self.tied) = (int(v) for v in dims)

    def close(self):
        if self._h:
            lib.oracle_model_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib.oracle_model_reset(self._h)

    def set_kv_fp16(self, on: bool) -> None:
        """store attention K/V rounded to fp16 (the GPU's fp16 paged cache)"""
        lib.oracle_model_set_kv_fp16(self._h, 1 if on else 0)

    def set_kv_q8(self, on: bool) -> None:
        """keep attention K/V rows as their Q8_0 round trip (the GPU's Q8_0 pages)"""
        lib.oracle_model_set_kv_q8(self._h, 1 if on else 0)

    def tokens(self) -> int:
        return int(lib.oracle_model_tokens(self._h))

    def embed(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((len(ids), self.D), np.float32)
        if lib.oracle_model_embed(self._h, _p(ids), len(ids), _p(out)) != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        return out

    def forward(self, rows):
        rows = _f32(rows).reshape(-1, self.D)
        logits = np.empty(self.V, np.float32)
        if lib.oracle_model_forward(self._h, _p(rows), rows.shape[0], _p(logits)) != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        return logits

    def forward_ids(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.empty(self.V, np.float32)
        if lib.oracle_model_forward_ids(self._h, _p(ids), len(ids), _p(logits)) != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        return logits

    def greedy(self, prompt, steps):
        """prefill + `steps` decode passes; returns (ids[steps+1], last logits, prefill s, decode s)"""
        prompt = np.ascontiguousarray(prompt, np.int32)
        ids = np.empty(steps + 1, np.int32)
        logits = np.empty(self.V, np.float32)
        pf, dc = c_double(), c_double()
        if lib.oracle_model_greedy(self._h, _p(prompt), len(prompt), steps, _p(ids), _p(logits), ctypes.byref(pf), ctypes.byref(dc)) != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        return ids, logits, pf.value, dc.value


def gemma_math(x, cap: float = 30.0):
    """(gelu_pytorch_tanh(x), cap * tanh(x / cap)) with glibc's tanhf"""
    x = _f32(x)
    out = np.empty(2 * x.size, np.float32)
    lib.oracle_gemma_math(_p(x), _p(out), x.size, cap)
    return out[0::2].copy(), out[1::2].copy()


class Gemma4:
    """The oracle's Gemma 4 text model (E4B schema) over a GGUF file or an
    in-memory image; forward runs the reference's batched form."""

    def __init__(self, path: str | None = None, image: np.ndarray | None = None):
        if path is not None:
            self._h = lib.oracle_gemma4_open(path.encode())
        else:
            self._image = image
            self._h = lib.oracle_gemma4_open_image(_p(image), image.nbytes)
        if not self._h:
            raise RuntimeError(lib.oracle_last_error().decode())
        dims = np.zeros(6, np.uint64)
        lib.oracle_gemma4_dims(self._h, _p(dims))
        self.V, self.D, self.L, self.window, self.shared, self.P = (int(v) for v in dims)

    def close(self):
        if self._h:
            lib.oracle_gemma4_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib.oracle_gemma4_reset(self._h)

    def tokens(self) -> int:
        return int(lib.oracle_gemma4_tokens(self._h))

    def kv_source(self, layer: int) -> int:
        return int(lib.oracle_gemma4_kv_source(self._h, layer))

    def embed(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((len(ids), self.D), np.float32)
        if lib.oracle_gemma4_embed(self._h, _p(ids), len(ids), _p(out)) != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        return out

    def forward(self, ids):
        """soft-capped logits of the last of the T ids"""
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.empty(self.V, np.float32)
        if lib.oracle_gemma4_forward(self._h, _p(ids), len(ids), _p(logits)) != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        return logits

    def greedy(self, prompt, steps: int):
        """prefill (batched) + `steps` single-token passes: (ids[steps+1], last logits)"""
        logits = self.forward(prompt)
        ids = [int(np.argmax(logits))]
        for _ in range(steps):
            logits = self.forward([ids[-1]])
            ids.append(int(np.argmax(logits)))
        return np.array(ids, np.int32), logits
