"""The oracle's Gemma 4 restatement on the CPU (its agreement with the
reference's own outputs is checked against the E4B goldens on the GPU box,
where the 7.9 GB model is built): the layer schedule against the reference's
static_asserts, the batched prefill against token-by-token passes, the
soft-cap bound, and the GELU / soft-cap against the same fp32 expressions
over glibc's tanhf."""
import ctypes
import os

import numpy as np
import pytest

import oracle


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from hero_amd.gemma4 import GEMMA4_TINY, write_synthetic_gemma4

    path = str(tmp_path_factory.mktemp("g4") / "tiny.gguf")
    write_synthetic_gemma4(path, GEMMA4_TINY, seed=5)
    m = oracle.Gemma4(path=path)
    yield m
    m.close()


def test_e4b_schedule_matches_the_reference_static_asserts(tmp_path):
    """nm/src/gemma4.hpp:59-67: layers 22 (local) and 23 (full) feed the last 18;
    a layer is full attention when l % 6 == 5. Checked on a 42-layer model
    with the E4B schedule at small width."""
    from hero_amd.gemma4 import Gemma4Shape, write_synthetic_gemma4

    shape = Gemma4Shape(vocab=64, d_model=64, layers=42, ffn=64, q_heads=1, kv_heads=1, local_head_dim=32, full_head_dim=64,
                        per_layer_input=32, window=8, shared_kv_layers=18, ctx=64)
    path = str(tmp_path / "sched.gguf")
    write_synthetic_gemma4(path, shape, seed=1)
    m = oracle.Gemma4(path=path)
    assert [m.kv_source(l) for l in (0, 5, 21, 22, 23)] == [0, 5, 21, 22, 23]
    assert all(m.kv_source(l) == (23 if l % 6 == 5 else 22) for l in range(24, 42))
    m.close()


def test_batched_prefill_equals_single_token_passes(tiny):
    """The reference's prefill runs every layer over all rows at once; each row
    must equal the same row run alone (past the window too)."""
    prompt = np.random.default_rng(1).integers(0, tiny.V, 80).astype(np.int32)
    tiny.reset()
    batched = tiny.forward(prompt)
    tiny.reset()
    for t in prompt:
        single = tiny.forward([t])
    assert np.array_equal(batched.view(np.uint32), single.view(np.uint32))
    assert tiny.tokens() == 80
    assert np.abs(batched).max() <= 30.0  # cap * tanh(.)


def test_gelu_and_softcap_match_glibc_arithmetic():
    libm = ctypes.CDLL("libm.so.6")
    libm.tanhf.restype = ctypes.c_float
    libm.tanhf.argtypes = [ctypes.c_float]
    x = np.concatenate([np.random.default_rng(2).standard_normal(2000).astype(np.float32) * s for s in (0.1, 3.0, 30.0)])
    gelu, cap = oracle.gemma_math(x, 30.0)
    f = np.float32
    for i, v in enumerate(x[:600]):
        v = f(v)
        inner = f(f(0.7978845608) * f(v + f(f(f(f(0.044715) * v) * v) * v)))
        assert gelu[i] == f(f(f(0.5) * v) * f(f(1.0) + f(libm.tanhf(inner))))
        assert cap[i] == f(f(30.0) * f(libm.tanhf(f(v / f(30.0)))))
