"""CPU sanitizer build of libqvl's GPU-free host code: qwen3-vl-jax_amd/csrc/qvl_meta.cpp (metadata,
window index, attention work lists, argument checks) compiled with g++ -fsanitize=address,undefined
together with tests/host_sanitizer/driver.cpp, which runs it on random and malformed grids with
exactly-sized buffers. Any out-of-bounds access, leak or undefined operation fails the run."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_host_code_under_asan_ubsan(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "qvl_host_asan"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-I", str(ROOT / "include"), "-I", str(ROOT / "qwen3-vl-jax_amd" / "csrc"),
           str(ROOT / "tests" / "host_sanitizer" / "driver.cpp"), str(ROOT / "qwen3-vl-jax_amd" / "csrc" / "qvl_meta.cpp"),
           "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "asan" in r.stderr.lower() and "cannot find" in r.stderr.lower():
        pytest.skip("the sanitizer runtime is not installed")
    assert r.returncode == 0, r.stderr[-4000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "PATH": "/usr/bin:/bin"})
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-4000:])
    assert "0 failures" in run.stdout
