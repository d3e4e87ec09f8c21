"""Shared fixtures. Tests marked `gpu` need an MI355X; everything else runs on
the CPU (oracle vs the reference's golden vectors, host logic, the C ABI)."""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def manifest():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def kernels_golden():
    return dict(np.load(os.path.join(GOLDEN, "kernels.npz")))


@pytest.fixture(scope="session")
def tiny_golden():
    return dict(np.load(os.path.join(GOLDEN, "tiny_model.npz")))


@pytest.fixture(scope="session")
def tiny_gguf(tmp_path_factory, manifest):
    """The tiny Q8_0 hybrid GGUF, regenerated from its seed; its bytes must be
    the ones the reference produced the golden vectors from."""
    import hero_amd

    t = manifest["tiny_model"]
    path = str(tmp_path_factory.mktemp("tiny") / "tiny.gguf")
    hero_amd.write_synthetic_gguf(path, hero_amd.TINY_CONFIG, seed=t["seed"], ctx=t["ctx"])
    with open(path, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == t["gguf_sha256"], "synthetic tiny model bytes changed"
    return path


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def window_golden(manifest):
    """the reference's windowed-attention outputs; the inputs are regenerated
    from the seed as tests/golden/make_golden.py made them, and their sha256
    must match the one recorded then"""
    w = manifest["window"]
    rng = np.random.default_rng(w["seed"])
    s = np.float32(1 / np.sqrt(128.0))
    k = np.ascontiguousarray(rng.standard_normal((w["ctx"], 256)) * s, np.float32)
    v = np.ascontiguousarray(rng.standard_normal((w["ctx"], 256)) * s, np.float32)
    q = np.ascontiguousarray(rng.standard_normal((w["ctx"], 512)), np.float32)
    assert hashlib.sha256(k.tobytes() + v.tobytes() + q.tobytes()).hexdigest() == w["inputs_sha256"], "window inputs changed"
    return dict(np.load(os.path.join(GOLDEN, "window.npz")), k=k, v=v, q=q)


@pytest.fixture(scope="session")
def variant_golden():
    return dict(np.load(os.path.join(GOLDEN, "tiny_hk4u_model.npz")))


# the tiny shape with 4 delta-net key heads tiled over 8 value heads and an
# untied output.weight (the golden's model)
def variant_shape():
    import hero_amd

    return hero_amd.HybridShape(vocab=32000, d_model=1024, layers=4, ffn=2816, q_heads=8, kv_heads=2, head_dim=128,
                                key_heads=4, value_heads=8)


@pytest.fixture(scope="session")
def variant_gguf(tmp_path_factory, manifest):
    import hero_amd

    t = manifest["tiny_hk4u_model"]
    path = str(tmp_path_factory.mktemp("variant") / "tiny_hk4u.gguf")
    hero_amd.write_synthetic_gguf(path, variant_shape(), seed=t["seed"], ctx=t["ctx"], tied=False)
    with open(path, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == t["gguf_sha256"], "synthetic variant model bytes changed"
    return path


@pytest.fixture(scope="session")
def dh256_golden():
    return dict(np.load(os.path.join(GOLDEN, "tiny_dh256_model.npz")))


# the attention geometry of the reference's Qwen 3.5 4B / 9B configs (256-wide
# heads, a quarter rotating, RoPE base 1e7, 4 key heads over 8 value heads,
# untied head) at tiny width (the golden's model)
@pytest.fixture(scope="session")
def dh256_gguf(tmp_path_factory, manifest):
    import hero_amd

    t = manifest["tiny_dh256_model"]
    path = str(tmp_path_factory.mktemp("dh256") / "tiny_dh256.gguf")
    hero_amd.write_synthetic_gguf(path, hero_amd.HybridShape(**t["shape"]), seed=t["seed"], ctx=t["ctx"], tied=False)
    with open(path, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == t["gguf_sha256"], "synthetic 256-wide-head model bytes changed"
    return path


# the tiny shape with the tensor types of a Q4_K_M checkpoint (Q4_K, Q5_K, Q6_K
# and Q8_0 tensors; the golden's model)
@pytest.fixture(scope="session")
def kmix_gguf(tmp_path_factory, manifest):
    import hero_amd

    t = manifest["tiny_kmix_model"]
    path = str(tmp_path_factory.mktemp("kmix") / "tiny_kmix.gguf")
    hero_amd.write_synthetic_gguf(path, hero_amd.TINY_CONFIG, seed=t["seed"], ctx=t["ctx"], tied=t["tied"],
                                  weight_mix=t["weight_mix"])
    with open(path, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == t["gguf_sha256"], "synthetic K-quant model bytes changed"
    return path


@pytest.fixture(scope="session")
def kmix_golden():
    return dict(np.load(os.path.join(GOLDEN, "tiny_kmix_model.npz")))


# the tiny shape with SwiGLU width 3584 (above every input projection's width)
# and Q8_0 in-projections, gate and up beside a Q6_K embedding and down
# projection and Q4_K output projections (the golden's model): every Q8_0
# linear here writes a strided output through the typed path's scratch
@pytest.fixture(scope="session")
def q8ffn_gguf(tmp_path_factory, manifest):
    import hero_amd

    t = manifest["tiny_q8ffn_model"]
    path = str(tmp_path_factory.mktemp("q8ffn") / "tiny_q8ffn.gguf")
    hero_amd.write_synthetic_gguf(path, hero_amd.HybridShape(**t["shape"]), seed=t["seed"], ctx=t["ctx"], tied=t["tied"],
                                  weight_mix=t["weight_mix"])
    with open(path, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == t["gguf_sha256"], "synthetic Q8_0-FFN mix model bytes changed"
    return path


@pytest.fixture(scope="session")
def q8ffn_golden():
    return dict(np.load(os.path.join(GOLDEN, "tiny_q8ffn_model.npz")))
