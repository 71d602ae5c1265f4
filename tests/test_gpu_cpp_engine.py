"""Runs the C++ host-API test driver (tests/cpp/engine_test.cpp), which
restates the reference's MoE helper and backend tests against
include/nexus_engine.hpp on the GPU."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_cpp_engine_driver():
    exe = os.path.join(HERE, "cpp", "engine_test")
    if not os.path.exists(exe):
        pytest.fail("tests/cpp/engine_test is not built (run __graft_entry__.build())")
    print("running", exe, flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "OK (0 failures)" in r.stdout
