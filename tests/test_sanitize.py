"""The two GGUF readers (the product's host reader hero_amd/csrc/host/gguf.cpp
and the oracle's reader and model loader) under AddressSanitizer and
UndefinedBehaviorSanitizer: oracle/_san/gguf_check parses malformed files made
from the tiny model (bad magic and version, truncations at many points, corrupt
counts, lengths, types, dimensions and offsets) and must report an error for
each without a sanitizer finding. CPU only; skipped where g++ cannot build the
sanitizers."""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT

BIN = os.path.join(ROOT, "oracle", "_san", "gguf_check")


@pytest.fixture(scope="module")
def checker():
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True, text=True)
    if r.returncode != 0 or not os.path.exists(BIN):
        pytest.skip("no sanitizer build here: " + r.stderr[-300:])
    return BIN


def header_fields(data: bytes):
    """offsets of the header counts and of the first metadata key / value"""
    n_tensors, n_kv = struct.unpack_from("<QQ", data, 8)
    return {"n_tensors": 8, "n_kv": 16, "key0_len": 24}, n_tensors, n_kv


def mutations(data: bytes):
    off, n_tensors, n_kv = header_fields(data)
    put = lambda b, o, fmt, v: b[:o] + struct.pack(fmt, v) + b[o + struct.calcsize(fmt):]  # noqa: E731
    yield "bad magic", b"XXXX" + data[4:]
    yield "version 2", data[:4] + (2).to_bytes(4, "little") + data[8:]
    for cut in (0, 7, 23, 40, 100, 1000, 5000, len(data) // 3, len(data) - 1):
        yield f"truncated at {cut}", data[:cut]
    yield "huge tensor count", put(data, off["n_tensors"], "<Q", 1 << 62)
    yield "huge key count", put(data, off["n_kv"], "<Q", 1 << 62)
    yield "key count + 1", put(data, off["n_kv"], "<Q", n_kv + 1)
    yield "huge first key length", put(data, off["key0_len"], "<Q", 1 << 60)
    rng = np.random.default_rng(99)
    head = 16384  # the metadata and the tensor table of the tiny model lie here
    for i in range(12):
        b = bytearray(data)
        for p in rng.integers(24, head, 8):
            b[int(p)] = int(rng.integers(0, 256))
        yield f"8 random bytes of the header changed ({i})", bytes(b)


def test_gguf_readers_reject_malformed_files_under_sanitizers(checker, tiny_gguf, tmp_path):
    data = open(tiny_gguf, "rb").read()
    ok = subprocess.run([checker, tiny_gguf], capture_output=True, text=True)
    assert ok.returncode == 0 and "hero: ok" in ok.stdout and "oracle model: ok" in ok.stdout, ok.stdout + ok.stderr
    bad = str(tmp_path / "bad.gguf")
    for name, blob in mutations(data):
        with open(bad, "wb") as f:
            f.write(blob)
        r = subprocess.run([checker, bad], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, f"{name}: sanitizer finding or crash\n{r.stdout}\n{r.stderr[-3000:]}"
        assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, f"{name}: {r.stderr[-3000:]}"
        if name in ("bad magic", "version 2") or name.startswith("truncated") or name.startswith("huge"):
            assert "hero: error" in r.stdout and "oracle model: error" in r.stdout, f"{name}: accepted\n{r.stdout}"
