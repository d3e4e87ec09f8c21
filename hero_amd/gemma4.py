"""Gemma 4 text models (E4B schema) on the GPU, over include/hero_gemma4.h.

Mirrors the reference's model contract for Gemma4E4BModel
(nm/src/gemma4.hpp:386-482, nm/src/transformer.hpp:70-78):

    model = Gemma4Model.open("gemma4.gguf")     # gemma4_loader::load_e4b_text
    rows = model.embed(ids)                     # Gemma4E4BModel::embed -> [T, D] fp32
    state = model.new_state(max_tokens)         # Gemma4E4BCache
    logits = model.forward(state, ids)          # Gemma4E4BModel::forward -> Logits (soft-capped)
    ids, last = model.decode_greedy(state, logits.argmax(), 32)

Inputs are token ids (the per-layer inputs read a table row per id).
"""
from __future__ import annotations

from ctypes import byref, c_int32, c_void_p
from dataclasses import dataclass

import numpy as np

from ._lib import Gemma4Dims, Gemma4SynthConfig, check, lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class Gemma4State:
    """One sequence's K/V caches (Gemma4E4BCache, nm/src/gemma4.hpp:343-378)."""

    def __init__(self, model: "Gemma4Model", max_tokens: int):
        self.model = model
        self._h = c_void_p()
        check(lib.hero_gemma4_state_create(model._h, max_tokens, byref(self._h)))
        self.max_tokens = max_tokens

    def tokens(self) -> int:
        return int(lib.hero_gemma4_state_tokens(self._h))

    def reset(self) -> None:
        check(lib.hero_gemma4_state_reset(self._h))

    def close(self) -> None:
        if self._h:
            lib.hero_gemma4_state_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Gemma4Model:
    """The GPU Gemma 4 text model. Immutable after load."""

    def __init__(self, handle: c_void_p):
        self._h = handle
        d = Gemma4Dims()
        check(lib.hero_gemma4_dims_get(handle, byref(d)))
        self.dims = d
        self.V, self.D, self.L, self.CTX = d.vocab, d.d_model, d.layers, d.ctx

    @classmethod
    def open(cls, path: str) -> "Gemma4Model":
        h = c_void_p()
        check(lib.hero_gemma4_open(path.encode(), byref(h)))
        return cls(h)

    @classmethod
    def open_image(cls, image: np.ndarray) -> "Gemma4Model":
        h = c_void_p()
        check(lib.hero_gemma4_open_image(_ptr(image), image.nbytes, byref(h)))
        return cls(h)  # every tensor was copied at load: the image may go

    def close(self) -> None:
        if self._h:
            lib.hero_gemma4_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_state(self, max_tokens: int | None = None) -> Gemma4State:
        return Gemma4State(self, max_tokens or min(self.CTX, 4096))

    def embed(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((len(ids), self.D), dtype=np.float32)
        check(lib.hero_gemma4_embed(self._h, _ptr(ids), len(ids), _ptr(out)))
        return out

    def forward(self, state: Gemma4State, ids, want_logits: bool = True):
        """Gemma4E4BModel::forward (nm/src/gemma4.hpp:424-445) over token ids:
        the soft-capped logits of the last row (or its greedy id)."""
        from . import Logits

        ids = np.ascontiguousarray(ids, dtype=np.int32)
        logits = np.empty(self.V, dtype=np.float32) if want_logits else None
        nxt = c_int32(-1)
        check(lib.hero_gemma4_forward(self._h, state._h, _ptr(ids), len(ids), _ptr(logits) if want_logits else None, byref(nxt)))
        return Logits(logits) if want_logits else int(nxt.value)

    def decode_greedy(self, state: Gemma4State, first_id: int, steps: int, want_logits: bool = False):
        """steps passes, each fed the previous greedy id (one hipGraph replay
        each). Returns (ids[steps], Logits of the last pass or None)."""
        from . import Logits

        out = np.empty(steps, dtype=np.int32)
        logits = np.empty(self.V, dtype=np.float32) if want_logits else None
        check(lib.hero_gemma4_decode_greedy(self._h, state._h, int(first_id), steps, _ptr(out), _ptr(logits) if want_logits else None))
        return out, (Logits(logits) if want_logits else None)

    def last_decode_seconds(self) -> float:
        return float(lib.hero_gemma4_last_decode_seconds(self._h))


# ---- synthetic models ---------------------------------------------------------

@dataclass(frozen=True)
class Gemma4Shape:
    vocab: int = 262144
    d_model: int = 2560
    layers: int = 42
    ffn: int = 10240
    q_heads: int = 8
    kv_heads: int = 2
    local_head_dim: int = 256
    full_head_dim: int = 512
    per_layer_input: int = 256
    window: int = 512
    shared_kv_layers: int = 18
    ctx: int = 131072


# the reference's Gemma4E4BTextConfig (nm/src/gemma4.hpp:19-35)
GEMMA4_E4B = Gemma4Shape()
# the same schema at small width: 12 layers (two full-attention layers, the
# last 4 reusing K/V), d_model 512, a 64-position window, vocabulary 4096
GEMMA4_TINY = Gemma4Shape(vocab=4096, d_model=512, layers=12, ffn=1024, q_heads=4, kv_heads=2, per_layer_input=64, window=64,
                          shared_kv_layers=4, ctx=4096)


def gemma4_synth_config(shape: Gemma4Shape, seed: int) -> Gemma4SynthConfig:
    return Gemma4SynthConfig(shape.vocab, shape.d_model, shape.layers, shape.ffn, shape.q_heads, shape.kv_heads, shape.local_head_dim,
                             shape.full_head_dim, shape.per_layer_input, shape.window, shape.shared_kv_layers, shape.ctx, seed)


def write_synthetic_gemma4(path: str, shape: Gemma4Shape = GEMMA4_E4B, seed: int = 1) -> None:
    cfg = gemma4_synth_config(shape, seed)
    check(lib.hero_synth_gemma4_file(byref(cfg), path.encode()))


def synthetic_gemma4_image(shape: Gemma4Shape = GEMMA4_E4B, seed: int = 1) -> np.ndarray:
    cfg = gemma4_synth_config(shape, seed)
    n = lib.hero_synth_gemma4_size(byref(cfg))
    if n < 0:
        check(1)
    image = np.empty(n, dtype=np.uint8)
    check(lib.hero_synth_gemma4_image(byref(cfg), _ptr(image), n))
    return image
