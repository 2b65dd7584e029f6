"""The native C++ caller of the C ABI (nyion.rs_amd/nyion_driver): built by
the package Makefile; without a device it reports one instead of running
(CPU).  The GPU run is in test_driver_gpu.py."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "nyion.rs_amd", "nyion_driver")


def test_driver_reports_missing_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a device is present: covered by test_driver_gpu.py")
    assert os.path.exists(DRIVER), "run __graft_entry__.build() first"
    r = subprocess.run([DRIVER], capture_output=True, text=True, timeout=60)
    assert r.returncode == 3 and "no usable device" in r.stderr
