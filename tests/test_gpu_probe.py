"""The C++ host layer end to end: the port of the reference's attention probe (Diag.swift:86-110) built on
host/FlashVSRLCSA.hpp must report kernel == dense (rel <= 1e-6) and bf16 kernel vs fp32 within 1e-2."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
PROBE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mlx-flashvsr-swift_amd", "lib",
                     "fvsr_probe_attn")


def test_probe_quick(dev):
    assert os.path.exists(PROBE), "build the host probe first (__graft_entry__.build())"
    res = subprocess.run([PROBE, "--quick"], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "FAIL" not in res.stdout
    assert res.stdout.count("rel") == 5
