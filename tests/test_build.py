"""The library build fails when hipcc fails.

A copy of nexus_amd/csrc with one source broken is built into a scratch
directory that already holds an object of that source from an earlier
build: make must fail, name the compile error, and leave no object behind
(a stale object must never be linked into libnexus_hip.so).
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_failed_compile_fails_the_build(tmp_path):
    src = tmp_path / "nexus_amd" / "csrc"
    shutil.copytree(os.path.join(ROOT, "nexus_amd", "csrc"), src,
                    ignore=shutil.ignore_patterns("*.so", "*.o"))
    (tmp_path / "include").mkdir()
    shutil.copy(os.path.join(ROOT, "include", "nexus_hip.h"), tmp_path / "include")
    build = tmp_path / "_build"
    build.mkdir()
    stale = build / "nx_norm.o"
    stale.write_bytes(b"an object from an earlier build")
    with open(src / "nx_norm.hip", "a") as f:
        f.write("\nthis is not C++;\n")
    t = os.stat(src / "nx_norm.hip").st_mtime - 3600  # the object predates the edit
    os.utime(stale, (t, t))
    r = subprocess.run(["make", "-C", str(src), f"BUILD={build}", f"OUT={tmp_path / 'lib.so'}",
                        str(stale)], capture_output=True, text=True)
    assert r.returncode != 0
    assert "error" in (r.stdout + r.stderr)
    assert not stale.exists()
    assert not (tmp_path / "lib.so").exists()
