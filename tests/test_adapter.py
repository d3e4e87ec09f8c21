"""The C++ adapter (include/qwen35_gpu.hpp) against the reference's own
headers: it must model the reference's TransformerModel concept, instantiate
with PrefixCache, link against libhero_amd.so, and map the C ABI's status
codes to the reference's exception types. Needs the reference tree (build
container only); the binary is written to oracle/_ref/, which is never
committed or shipped."""
import os
import subprocess

import pytest

from conftest import ROOT

REF = "/root/reference/nm/src"


@pytest.mark.skipif(not os.path.isdir(REF), reason="needs the reference tree")
def test_adapter_compiles_against_the_reference_and_maps_errors():
    out_dir = os.path.join(ROOT, "oracle", "_ref")
    os.makedirs(out_dir, exist_ok=True)
    exe = os.path.join(out_dir, "adapter_check")
    lib_dir = os.path.join(ROOT, "hero_amd")
    build = subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-Wno-unused-parameter", f"-I{REF}",
                    f"-I{os.path.join(ROOT, 'include')}", os.path.join(ROOT, "tests", "adapter_check.cpp"),
                    os.path.join(REF, "core.cpp"), os.path.join(REF, "gguf.cpp"), f"-L{lib_dir}", "-lhero_amd",
                    f"-Wl,-rpath,{lib_dir}", "-lpthread", "-o", exe], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-4000:]
    run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(run.stdout)
    assert run.returncode == 0 and run.stdout.strip().endswith("OK"), run.stdout + run.stderr
