"""The C ABI on the CPU: the library loads, exports every entry point the
headers declare, and reports argument and file errors without touching a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

import hero_amd
from hero_amd import _lib
from conftest import ROOT


def declared_symbols():
    names = set()
    for h in ("hero_kernels.h", "hero_model.h", "hero_gemma4.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        names |= set(re.findall(r"\b(hero_[A-Za-z0-9_]+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    declared = declared_symbols()
    assert len(declared) >= 30
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_gemma4_loader_rejects_a_qwen_file_and_bad_synth_configs(tmp_path):
    """hero_gemma4_open checks general.architecture before touching the
    device, and the synthetic writer rejects impossible shapes."""
    from hero_amd.gemma4 import GEMMA4_TINY, gemma4_synth_config

    lib = _lib.lib
    path = str(tmp_path / "tiny_qwen.gguf")
    hero_amd.write_synthetic_gguf(path, hero_amd.TINY_CONFIG, seed=1)
    h = ctypes.c_void_p()
    assert lib.hero_gemma4_open(path.encode(), ctypes.byref(h)) == _lib.HERO_EIO
    assert b"gemma4" in lib.hero_last_error()
    cfg = gemma4_synth_config(GEMMA4_TINY, 1)
    assert lib.hero_synth_gemma4_size(ctypes.byref(cfg)) > 0
    cfg.shared_kv_layers = cfg.layers
    assert lib.hero_synth_gemma4_size(ctypes.byref(cfg)) == -1
    cfg = gemma4_synth_config(GEMMA4_TINY, 1)
    cfg.d_model = 500
    assert lib.hero_synth_gemma4_size(ctypes.byref(cfg)) == -1


def test_kquant_argument_errors_are_reported_before_any_launch():
    lib = _lib.lib
    assert lib.hero_q8_K_act_bytes(3, 4096) == 3 * 16 * 292 + 3 * 16 * 256  # blocks, then the regrouped copy
    assert lib.hero_kquant_gemm(13, 16, 16, 16, 1, 64, 4096, None) == _lib.HERO_EINVAL  # Q5_K has its own form
    assert b"Q4_K" in lib.hero_last_error()
    assert lib.hero_kquant_gemm(12, 16, 16, 16, 1, 64, 4000, None) == _lib.HERO_EINVAL
    assert b"multiple of 256" in lib.hero_last_error()
    assert lib.hero_kquant_gemm(14, None, 16, 16, 1, 64, 4096, None) == _lib.HERO_EINVAL
    assert lib.hero_kquant_gemm(12, 8, 16, 16, 1, 64, 4096, None) == _lib.HERO_EINVAL  # alignment
    assert lib.hero_q8_K_quantize(16, 16, 1, 300, None) == _lib.HERO_EINVAL
    assert lib.hero_q5_K_gemm(16, 16, 16, 1, 64, 16384 + 256, None) == _lib.HERO_EINVAL  # Q5_K: k <= 16384
    assert b"too large" in lib.hero_last_error()
    assert lib.hero_kquant_pack(11, 16, 32, 64, 4096, None) == _lib.HERO_EINVAL
    assert lib.hero_kquant_pack(12, 16, 16, 64, 4096, None) == _lib.HERO_EINVAL  # in place
    assert lib.hero_kquant_dequant_rows(14, 16, 64, 4096, 16, 0, 16, None) == _lib.HERO_EINVAL
    # the packed form: the GGUF bytes in tiles of 256 / (k / 256) rows, each tile
    # padded to whole waves of 64 blocks (k 512: tiles of 128 rows, 4 waves)
    for t, per_block in ((12, 144), (13, 176), (14, 210)):
        assert lib.hero_kquant_packed_bytes(t, 3, 512) == 256 * per_block
        assert lib.hero_kquant_packed_bytes(t, 4096, 4096) == 4096 * 16 * per_block  # whole tiles: no padding
    assert lib.hero_kquant_packed_bytes(8, 3, 512) == -1


def test_size_helpers():
    assert _lib.lib.hero_q8_0_packed_bytes(4096, 4096) == 4096 * 4096 * 34 // 32
    assert _lib.lib.hero_q8_0_act_bytes(2, 1024) == 2 * 1024 + 2 * 32 * 4


def test_argument_errors_are_reported_before_any_launch():
    lib = _lib.lib
    assert lib.hero_q8_0_gemv(None, None, None, None, 64, 4096, None) == _lib.HERO_EINVAL
    assert b"null" in lib.hero_last_error()
    assert lib.hero_q8_0_gemv(16, 16, 16, None, 64, 100, None) == _lib.HERO_EINVAL  # K % 32
    assert b"multiple of 32" in lib.hero_last_error()
    assert lib.hero_q8_0_quantize(16, 16, 0, 4096, None) == _lib.HERO_EINVAL
    assert lib.hero_rmsnorm_quant(16, 16, 1e-6, None, None, 1, 32768, None) == _lib.HERO_EINVAL
    assert lib.hero_gdn_decode(None, None) == _lib.HERO_EINVAL
    args = _lib.GdnDecodeArgs()
    args.dk = args.dv = 64
    assert lib.hero_gdn_decode(ctypes.byref(args), None) == _lib.HERO_EINVAL
    assert b"128" in lib.hero_last_error()


def write(path, data: bytes):
    with open(path, "wb") as f:
        f.write(data)


@pytest.mark.parametrize("mutate,needle", [
    (lambda b: b"XXXX" + b[4:], b"bad magic"),
    (lambda b: b[:4] + (2).to_bytes(4, "little") + b[8:], b"unsupported version"),
    (lambda b: b[: len(b) // 3], b"out of range"),
    (lambda b: b[:40], b"truncated"),
])
def test_malformed_gguf_is_rejected(tmp_path, tiny_gguf, mutate, needle):
    data = open(tiny_gguf, "rb").read()
    bad = str(tmp_path / "bad.gguf")
    write(bad, mutate(data))
    with pytest.raises(hero_amd.HeroError) as e:
        hero_amd.Qwen35Model.open(bad)
    assert e.value.code == _lib.HERO_EIO
    assert needle.decode() in str(e.value)


def test_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(hero_amd.HeroError) as e:
        hero_amd.Qwen35Model.open(str(tmp_path / "none.gguf"))
    assert e.value.code == _lib.HERO_EIO


def test_synthetic_model_is_deterministic(tiny_gguf):
    img = hero_amd.synthetic_gguf_image(hero_amd.TINY_CONFIG, seed=1234, ctx=4096)
    assert img.tobytes() == open(tiny_gguf, "rb").read()
    other = hero_amd.synthetic_gguf_image(hero_amd.TINY_CONFIG, seed=1235, ctx=4096)
    assert other.tobytes() != img.tobytes() and other.nbytes == img.nbytes


def test_synth_rejects_bad_shapes():
    cfg = hero_amd.synth_config(hero_amd.TINY_CONFIG, 1)
    cfg.layers = 3
    assert _lib.lib.hero_synth_qwen35_size(ctypes.byref(cfg)) == -1
    assert b"multiple of 4" in _lib.lib.hero_last_error()


def test_one_hip_runtime_per_process():
    """torch-ROCm bundles its own libamdhip64; the package must bind to the
    same copy rather than load a second runtime (pointers would not be shared)."""
    import hero_amd  # noqa: F401

    maps = open(f"/proc/{os.getpid()}/maps").read()
    hip = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    hsa = {l.split()[-1] for l in maps.splitlines() if "libhsa-runtime64" in l}
    assert len(hip) == 1, hip
    assert len(hsa) == 1, hsa


def test_libm_header_equals_glibc_on_the_host(tmp_path):
    """hero/libm.hpp's expf / log1pf / expm1f / tanhf (the device's exp, log1p,
    expm1 and tanh) against glibc on a dense stride of all float bit patterns
    and the branch edges; pass 1 as the stride to sweep all 2^32."""
    import subprocess

    exe = str(tmp_path / "libm_check")
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "-std=c++20", "-O2", "-ffp-contract=off", "-fno-builtin",
                    "--offload-arch=gfx950", "-I", os.path.join(ROOT, "hero_amd", "csrc"),
                    os.path.join(ROOT, "tests", "libm_check.cpp"), "-o", exe], check=True, capture_output=True)
    out = subprocess.run([exe, "257"], capture_output=True, text=True)
    n, be, bl, bm, bt = (int(v) for v in out.stdout.split())
    assert n > 16_000_000 and be == bl == bm == bt == 0, out.stdout


def test_seqsum_equals_the_sequential_loop_on_the_host(tmp_path):
    """hero/seqsum.hpp's parallel sum of non-negative floats, run phase by
    phase on the host, equals the left-to-right fp32 loop bit for bit on random
    sums of squares, exponentials, mixed magnitudes, zeros and overflow."""
    import subprocess

    exe = str(tmp_path / "seqsum_check")
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "-std=c++20", "-O2", "-ffp-contract=off",
                    "--offload-arch=gfx950", "-I", os.path.join(ROOT, "hero_amd", "csrc"),
                    os.path.join(ROOT, "tests", "seqsum_check.cpp"), "-o", exe], check=True, capture_output=True)
    out = subprocess.run([exe, "3000"], capture_output=True, text=True, timeout=300)
    trials, bad, _fallbacks = (int(v) for v in out.stdout.split()[-3:])
    assert trials == 3000 and bad == 0, out.stdout
