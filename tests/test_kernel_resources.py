"""Every HIP kernel of the library keeps its working values in registers.

The library build writes hipcc's per-kernel resource remarks next to each
object (`_build/<source>.diag.txt`, see nexus_amd/csrc/Makefile).  A kernel
with private arrays the compiler could not keep in registers, or with
vector registers spilled, reports scratch memory: every access to it is a
round trip to memory, which turns a bandwidth-bound kernel into a
latency-bound one (a combine kernel whose float4 selects were lowered to
selects of addresses ran 13x slower with correct results, so no parity
test sees it).  Scalar-register spills go to vector-register lanes and are
allowed.
"""
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DIAGS = sorted(glob.glob(os.path.join(ROOT, "_build", "nx_*.diag.txt")))


def kernel_resources(path):
    """{kernel symbol: {remark name: int value}} from one remarks file."""
    out, cur = {}, None
    for line in open(path, errors="replace"):
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[bytes/lane\])?: (\d+)", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    return out


@pytest.mark.skipif(not DIAGS, reason="no build remarks (run nexus_amd.build() first)")
def test_no_kernel_uses_scratch_or_spills_vector_registers():
    kernels = {}
    for p in DIAGS:
        kernels.update(kernel_resources(p))
    assert len(kernels) > 50  # every source's kernels were reported
    bad = {k: v for k, v in kernels.items()
           if v.get("ScratchSize", 0) or v.get("VGPRs Spill", 0)}
    assert not bad, bad


def test_parser_reads_the_remark_format(tmp_path):
    # the remark lines hipcc prints for one kernel (names and values as printed)
    p = tmp_path / "x.diag.txt"
    p.write_text(
        "a.hip:1:1: remark: Function Name: _Z1kv [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     VGPRs: 12 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 144 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     VGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     SGPRs Spill: 2 [-Rpass-analysis=kernel-resource-usage]\n")
    r = kernel_resources(str(p))
    assert r == {"_Z1kv": {"VGPRs": 12, "ScratchSize": 144, "VGPRs Spill": 3, "SGPRs Spill": 2}}
