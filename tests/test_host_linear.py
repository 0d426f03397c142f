"""The C++ host side (agens-engine_amd/host/agens_linear.*: wq_upload_kt, linear, linear_shared) on the GPU, through
its own test program tests/host/test_linear (built by agens-engine_amd/build.py)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "host", "test_linear")


def test_host_program_built():
    assert os.path.exists(BIN), "tests/host/test_linear missing: run `python agens-engine_amd/build.py`"


@pytest.mark.gpu
def test_host_linear_gpu():
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0 and "host linear: OK" in r.stdout, r.stdout + r.stderr
