"""Row preconditions of the register-run kernels (CPU only).

k_block_prologue and k_rms_runs clamp their load indices into the row
(min(i, H / 4 - 1)), which is in range only for rows of at least one float4.
nexus_amd/csrc/nx_rows.hpp states the precondition once (register_row_fits);
this test compiles that header with the host compiler and checks it at its
edges, and checks that every function of the library that launches one of
those kernels tests the precondition before its launch.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "nexus_amd", "csrc")
GXX = shutil.which("g++")

CHECK = r"""
#include <cstdio>
#include "nx_rows.hpp"
using nx::register_row_fits;
static_assert(nx::kPrologueMaxH == 7168 && nx::kRmsRunsMaxH == 7168, "widest rows");
int main() {
  struct { long h, max; bool fits; } cases[] = {
      {0, 7168, false},    {-4, 7168, false},  {1, 7168, false},   {3, 7168, false},
      {4, 7168, true},     {5, 7168, false},   {4096, 7168, true}, {7168, 7168, true},
      {7172, 7168, false}, {7170, 7168, false}, {4, 4, true},      {8, 4, false},
      {4, 0, false},
  };
  int bad = 0;
  for (auto &c : cases)
    if (register_row_fits(c.h, c.max) != c.fits) {
      std::printf("H=%ld max=%ld: expected %d\n", c.h, c.max, (int)c.fits);
      ++bad;
    }
  return bad;
}
"""


@pytest.mark.skipif(GXX is None, reason="no host C++ compiler")
def test_register_row_fits_edges(tmp_path):
    src = tmp_path / "check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "check"
    r = subprocess.run([GXX, "-std=c++17", "-Wall", "-Werror", f"-I{CSRC}", str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout


def functions(text):
    """(name, body) of each top-level function definition of a source file."""
    out = []
    for m in re.finditer(r"^[A-Za-z][^\n;{}]*?\b(\w+)\s*\([^;{}]*\)\s*\{", text, re.M):
        depth, i = 1, m.end()
        while depth and i < len(text):
            depth += {"{": 1, "}": -1}.get(text[i], 0)
            i += 1
        out.append((m.group(1), text[m.end():i]))
    return out


CLAMPING = ("k_block_prologue", "k_rms_runs")
CHECKS = ("register_row_fits(", "block_prologue_fits(", "rms_runs_fit(")


def test_every_launcher_checks_the_row():
    launchers = []
    for fn in ("nx_logits.hip", "nx_norm.hip"):
        with open(os.path.join(CSRC, fn)) as f:
            text = f.read()
        for name, body in functions(text):
            for kern in CLAMPING:
                launch = body.find(f"go(c, {kern}<")
                if launch < 0:
                    continue
                launchers.append((fn, name))
                first_check = min((body.find(c) for c in CHECKS if c in body), default=-1)
                assert 0 <= first_check < launch, f"{fn}: {name} launches {kern} unchecked"
    # the exact router logits, the block prologue and the exact RMSNorm
    assert {n for _, n in launchers} >= {"launch_router_logits", "launch_block_prologue",
                                         "launch_rms_exact_runs"}, launchers
    # and the helpers the launchers call state it through register_row_fits
    with open(os.path.join(CSRC, "nx_logits.hip")) as f:
        logits = dict(functions(f.read()))
    with open(os.path.join(CSRC, "nx_norm.hip")) as f:
        norm = dict(functions(f.read()))
    assert "register_row_fits(" in logits["block_prologue_fits"]
    assert "register_row_fits(" in norm["rms_runs_fit"]
