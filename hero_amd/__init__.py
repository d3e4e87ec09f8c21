"""hero_amd -- MI355X (gfx950) decode/prefill path for Q8_0 Qwen 3.5-style hybrid models.

The Python surface mirrors the reference engine's model contract
(nm/src/transformer.hpp:70-78) over the C ABI in include/hero_model.h:

    model = Qwen35Model.open("model.gguf")       # qwen35_loader::load<C>
    rows = model.embed(ids)                      # Qwen35Model::embed -> [T, D] fp32
    state = model.new_state(max_tokens)          # Qwen35State<C>
    logits = model.forward(state, rows=rows)     # Qwen35Model::forward -> Logits
    logits.argmax()                              # Logits::argmax, ties to the lowest id
    cache = PrefixCache(model); cache.evaluate(sequence)   # PrefixCache::evaluate

Everything runs through libhero_amd.so on the GPU; importing raises if the
library is not built.
"""
from __future__ import annotations

import ctypes
import itertools
from ctypes import byref, c_int32, c_void_p
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import ContextExhausted, HeroError, ModelDims, SynthConfig, check, lib

__all__ = [
    "ContextExhausted", "HeroError", "Logits", "Qwen35Model", "PrefixState", "PrefixCache",
    "EmbeddedSequence", "BatchState", "TINY_CONFIG", "HYBRID_8B_CONFIG", "synth_config", "write_synthetic_gguf",
    "synthetic_gguf_image", "lib",
]


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class Logits:
    """One score per vocabulary entry (nm/src/logits.hpp:46-66)."""

    def __init__(self, values: np.ndarray):
        self.values = values

    def argmax(self) -> int:
        # np.argmax returns the first maximum: ties go to the lowest id
        return int(np.argmax(self.values))

    def __len__(self):
        return len(self.values)


def _kv_flags(kv_fp16: bool, kv_q8: bool) -> int:
    return (_lib.HERO_STATE_KV_FP16 if kv_fp16 else 0) | (_lib.HERO_STATE_KV_Q8_0 if kv_q8 else 0)


class PrefixState:
    """Device-resident carried state of one sequence (nm/src/qwen35.hpp:206-241).
    kv_fp16 / kv_q8 keep the attention cache as fp16 / Q8_0 pages (split-K
    attention); gdn_chunked runs the delta-net prefill in its chunked form."""

    def __init__(self, model: "Qwen35Model", max_tokens: int, kv_fp16: bool = False, gdn_chunked: bool = False, kv_q8: bool = False):
        h = c_void_p()
        flags = _kv_flags(kv_fp16, kv_q8) | (_lib.HERO_STATE_GDN_CHUNKED if gdn_chunked else 0)
        if flags:
            check(lib.hero_batch_state_create(model._h, max_tokens, 1, flags, byref(h)))
        else:
            check(lib.hero_state_create(model._h, max_tokens, byref(h)))
        self._h = h
        self.model = model
        self.max_tokens = max_tokens

    def tokens(self) -> int:
        return int(lib.hero_state_tokens(self._h))

    def reset(self) -> None:
        check(lib.hero_state_reset(self._h))

    def close(self) -> None:
        if self._h:
            lib.hero_state_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BatchState:
    """`batch` independent sequences in one device state, decoded together
    (no counterpart in the reference, which carries one sequence per state)."""

    def __init__(self, model: "Qwen35Model", max_tokens: int, batch: int, kv_fp16: bool = False, kv_q8: bool = False):
        h = c_void_p()
        check(lib.hero_batch_state_create(model._h, max_tokens, batch, _kv_flags(kv_fp16, kv_q8), byref(h)))
        self._h = h
        self.model = model
        self.max_tokens = max_tokens
        self.batch = batch

    def tokens(self, seq: int) -> int:
        return int(lib.hero_state_seq_tokens(self._h, seq))

    def reset(self) -> None:
        check(lib.hero_state_reset(self._h))

    def close(self) -> None:
        if self._h:
            lib.hero_state_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Qwen35Model:
    """The GPU model. Immutable after load; weights are never copied."""

    def __init__(self, handle: c_void_p):
        self._h = handle
        d = ModelDims()
        check(lib.hero_model_dims_get(handle, byref(d)))
        self.dims = d
        self.V, self.D, self.L, self.CTX = d.vocab, d.d_model, d.layers, d.ctx

    @classmethod
    def open(cls, path: str) -> "Qwen35Model":
        h = c_void_p()
        check(lib.hero_model_open(path.encode(), byref(h)))
        return cls(h)

    @classmethod
    def open_image(cls, image: np.ndarray) -> "Qwen35Model":
        h = c_void_p()
        check(lib.hero_model_open_image(_ptr(image), image.nbytes, byref(h)))
        m = cls(h)
        m._image = image  # keep the caller's bytes alive for the model's lifetime
        return m

    def close(self) -> None:
        if self._h:
            lib.hero_model_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_state(self, max_tokens: int | None = None, kv_fp16: bool = False, gdn_chunked: bool = False, kv_q8: bool = False) -> PrefixState:
        return PrefixState(self, max_tokens or min(self.CTX, 4096), kv_fp16, gdn_chunked, kv_q8)

    def new_batch_state(self, max_tokens: int, batch: int, kv_fp16: bool = False, kv_q8: bool = False) -> BatchState:
        return BatchState(self, max_tokens, batch, kv_fp16, kv_q8)

    def forward_seq(self, state: BatchState, seq: int, rows: np.ndarray | None = None, ids=None, want_logits: bool = True) -> Logits | int:
        """forward() for sequence `seq` of a batch state."""
        logits = np.empty(self.V, dtype=np.float32) if want_logits else None
        nxt = c_int32(-1)
        if rows is not None:
            rows = np.ascontiguousarray(rows, dtype=np.float32).reshape(-1, self.D)
            check(lib.hero_model_forward_seq(self._h, state._h, seq, _ptr(rows), None, rows.shape[0], _ptr(logits) if want_logits else None, byref(nxt)))
        else:
            ids = np.ascontiguousarray(ids, dtype=np.int32)
            check(lib.hero_model_forward_seq(self._h, state._h, seq, None, _ptr(ids), len(ids), _ptr(logits) if want_logits else None, byref(nxt)))
        return Logits(logits) if want_logits else int(nxt.value)

    def decode_batch(self, state: BatchState, first_ids, steps: int, want_logits: bool = False):
        """Greedy decode of every sequence at once (one hipGraph replay per
        pass). Returns (ids[steps][B], logits [B][V] of the last pass)."""
        first = np.ascontiguousarray(first_ids, dtype=np.int32)
        assert first.shape == (state.batch,)
        out = np.empty((steps, state.batch), dtype=np.int32)
        logits = np.empty((state.batch, self.V), dtype=np.float32) if want_logits else None
        check(lib.hero_model_decode_batch(self._h, state._h, _ptr(first), steps, _ptr(out), _ptr(logits) if want_logits else None))
        return out, logits

    def embed(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((len(ids), self.D), dtype=np.float32)
        check(lib.hero_model_embed(self._h, _ptr(ids), len(ids), _ptr(out)))
        return out

    def forward(self, state: PrefixState, rows: np.ndarray | None = None, ids=None, want_logits: bool = True) -> Logits | int:
        """Qwen35Model::forward (nm/src/qwen35.hpp:288-303): T new rows at the
        state's position. Returns Logits of the last row (or its greedy id if
        want_logits is False)."""
        logits = np.empty(self.V, dtype=np.float32) if want_logits else None
        nxt = c_int32(-1)
        if rows is not None:
            rows = np.ascontiguousarray(rows, dtype=np.float32).reshape(-1, self.D)
            t = rows.shape[0]
            check(lib.hero_model_forward(self._h, state._h, _ptr(rows), None, t, _ptr(logits) if want_logits else None, byref(nxt)))
        else:
            ids = np.ascontiguousarray(ids, dtype=np.int32)
            t = len(ids)
            check(lib.hero_model_forward(self._h, state._h, None, _ptr(ids), t, _ptr(logits) if want_logits else None, byref(nxt)))
        return Logits(logits) if want_logits else int(nxt.value)

    def decode_greedy(self, state: PrefixState, first_id: int, steps: int, want_logits: bool = False):
        """steps forward passes, each fed the previous greedy id; the whole step
        is one hipGraph replay. Returns (ids[steps], logits of the last pass)."""
        out = np.empty(steps, dtype=np.int32)
        logits = np.empty(self.V, dtype=np.float32) if want_logits else None
        check(lib.hero_model_decode_greedy(self._h, state._h, int(first_id), steps, _ptr(out), _ptr(logits) if want_logits else None))
        return out, (Logits(logits) if want_logits else None)

    def last_decode_seconds(self) -> float:
        return float(lib.hero_model_last_decode_seconds(self._h))

    def time_gemvs(self, state: PrefixState, reps: int = 5):
        """(seconds, launches per step, algorithmic bytes per step) of the
        step's Q8_0 matvecs launched reps times back to back"""
        sec, n, b = ctypes.c_double(), ctypes.c_int64(), ctypes.c_int64()
        check(lib.hero_model_time_gemvs(self._h, state._h, reps, byref(sec), byref(n), byref(b)))
        return sec.value, n.value, b.value


_sequence_ids = itertools.count(1)


class EmbeddedSequence:
    """Append-only decoder input with an identity (nm/src/multimodal.hpp:76-123)."""

    def __init__(self, d_model: int):
        self.rows = np.empty((0, d_model), dtype=np.float32)
        self.ids: list[int] = []
        self.sequence_id = next(_sequence_ids)

    def tokens(self) -> int:
        return self.rows.shape[0]

    def append(self, rows: np.ndarray, ids) -> None:
        rows = np.asarray(rows, dtype=np.float32).reshape(-1, self.rows.shape[1])
        if rows.shape[0] == 0:
            raise ValueError("EmbeddedSequence: empty append")
        if len(ids) != rows.shape[0]:
            raise ValueError("EmbeddedSequence: one id per row")
        self.rows = np.concatenate([self.rows, rows])
        self.ids.extend(int(i) for i in ids)


class PrefixCache:
    """Reuse the carried state while the same sequence grows
    (nm/src/transformer.hpp:97-169)."""

    def __init__(self, model: Qwen35Model, max_tokens: int | None = None):
        self.model = model
        self.state = model.new_state(max_tokens)
        self.sequence_id = 0
        self.last_logits: Logits | None = None
        self.reused_tokens = 0
        self.computed_tokens = 0

    def cached_tokens(self) -> int:
        return self.state.tokens()

    def clear(self) -> None:
        self.state.reset()
        self.sequence_id = 0
        self.last_logits = None
        self.reused_tokens = self.computed_tokens = 0

    def evaluate(self, seq: EmbeddedSequence) -> Logits:
        if seq.tokens() == 0:
            raise ValueError("evaluate: empty input")
        if seq.tokens() > self.state.max_tokens:
            raise ContextExhausted(3, "evaluate: context exhausted")
        if self.sequence_id != seq.sequence_id or self.cached_tokens() > seq.tokens():
            self.clear()
        reused = self.cached_tokens()
        self.reused_tokens, self.computed_tokens = reused, seq.tokens() - reused
        if reused == seq.tokens():
            if self.last_logits is None:
                raise RuntimeError("evaluate: prefix cache has no logits")
            return Logits(self.last_logits.values.copy())
        try:
            logits = self.model.forward(self.state, rows=seq.rows[reused:])
            if self.cached_tokens() != seq.tokens():
                raise RuntimeError("evaluate: the model did not advance its state by the rows it was given")
        except Exception:
            self.clear()
            raise
        self.sequence_id = seq.sequence_id
        self.last_logits = Logits(logits.values.copy())
        return logits


# ---- synthetic models ---------------------------------------------------------

@dataclass(frozen=True)
class HybridShape:
    vocab: int
    d_model: int
    layers: int
    ffn: int
    q_heads: int
    kv_heads: int
    head_dim: int
    key_heads: int
    value_heads: int
    key_head_dim: int = 128
    value_head_dim: int = 128
    conv_width: int = 4
    rope_base: float = 1e6


# 4 layers (3 gated delta-net + 1 GQA), d_model 1024, 8 q / 2 kv heads of 128,
# delta-net 8 heads of 128, SwiGLU 2816, vocab 32000
TINY_CONFIG = HybridShape(vocab=32000, d_model=1024, layers=4, ffn=2816, q_heads=8, kv_heads=2, head_dim=128, key_heads=8, value_heads=8)
# 32 layers (24 gated delta-net + 8 GQA), d_model 4096, 32 q / 8 kv heads of 128,
# delta-net 32 heads of 128, SwiGLU 12288, vocab 151936
HYBRID_8B_CONFIG = HybridShape(vocab=151936, d_model=4096, layers=32, ffn=12288, q_heads=32, kv_heads=8, head_dim=128, key_heads=32, value_heads=32)


# weight_mix values of the synthetic writer
WEIGHTS_Q8_0 = 0  # every 2-D weight Q8_0
WEIGHTS_K_MIX = 1  # the tensor types of a Q4_K_M checkpoint: Q4_K, Q5_K, Q6_K and Q8_0
WEIGHTS_Q8_FFN_MIX = 2  # Q8_0 in-projections, gate and up; Q6_K embedding and down; Q4_K output projections


def synth_config(shape: HybridShape, seed: int, ctx: int = 4096, tied: bool = True, weight_mix: int = WEIGHTS_Q8_0) -> SynthConfig:
    return SynthConfig(shape.vocab, shape.d_model, shape.layers, shape.ffn, shape.q_heads, shape.kv_heads, shape.head_dim,
                       shape.key_head_dim, shape.value_head_dim, shape.key_heads, shape.value_heads, shape.conv_width,
                       ctx, shape.rope_base, 1 if tied else 0, seed, weight_mix)


def write_synthetic_gguf(path: str, shape: HybridShape = TINY_CONFIG, seed: int = 1, ctx: int = 4096, tied: bool = True,
                         weight_mix: int = WEIGHTS_Q8_0) -> None:
    cfg = synth_config(shape, seed, ctx, tied, weight_mix)
    check(lib.hero_synth_qwen35_file(byref(cfg), path.encode()))


def synthetic_gguf_image(shape: HybridShape = TINY_CONFIG, seed: int = 1, ctx: int = 4096, tied: bool = True,
                         weight_mix: int = WEIGHTS_Q8_0) -> np.ndarray:
    cfg = synth_config(shape, seed, ctx, tied, weight_mix)
    n = lib.hero_synth_qwen35_size(byref(cfg))
    if n < 0:
        check(1)
    image = np.empty(n, dtype=np.uint8)
    check(lib.hero_synth_qwen35_image(byref(cfg), _ptr(image), n))
    return image
