"""The library's host-only structures (HMA free list, KV page policy) under
the address and undefined-behaviour sanitizers: tests/native/host_sanitize.cpp
is built with g++ from the library's own headers and run (CPU only)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "host_sanitize.cpp")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_structures_under_sanitizers(tmp_path):
    exe = str(tmp_path / "host_sanitize")
    flags = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", *flags, "-Wall", "-Wextra", SRC, "-o", exe],
                   check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks held" in r.stdout
