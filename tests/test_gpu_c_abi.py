"""The library used from a plain host program through the C ABI alone
(tests/c_abi/osm_c_smoke.cpp: include/osm.h and the HIP runtime, no Python
or torch in the process): the fused forward against a double-precision
restatement, workspace reuse, and an argument error as a status code."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "osm_c_smoke")


def test_c_program_through_the_abi():
    assert os.path.exists(BIN), "build first: python -m orthossm_amd.build"
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=60)
    print(res.stdout, res.stderr)
    assert res.returncode == 0, res.stderr
    assert res.stdout.startswith("ok:")
