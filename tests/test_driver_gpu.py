"""The native C++ caller of the C ABI on the GPU (gpu): decode, prefill and
Q4_K GEMV through plain pointers from the library's arena, each checked by
the driver against its own double-precision host loops (max-abs <= 2e-3,
rel <= 1e-3)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "nyion.rs_amd", "nyion_driver")


def test_native_driver_runs_and_agrees():
    assert os.path.exists(DRIVER), "run __graft_entry__.build() first"
    r = subprocess.run([DRIVER], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    for what in ("decode", "prefill", "gemv_q4k"):
        assert f"nyion_driver: {what}" in r.stdout
