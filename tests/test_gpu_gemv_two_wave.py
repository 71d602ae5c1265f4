"""GEMV rows of 65-128 segments (e.g. DeepSeek-V3's 7168 columns of Q4_K, or
Q8_0 rows of 4096 with two tokens per group): a two-wave row group, two row
groups per workgroup.  Bar: relative L2 1e-4 against the oracle's dispatch
(src/engine/mod.rs:969-1024) and matvec, with row counts that leave the last
workgroup's second row group short or empty, a shared expert, more than two
slots (the per-slot down kernel) and two (the down kernel with the
combine).
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import Q4_0, Q4_K, Q8_0, Layer, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("fmt,E,H,F,k,T,shared", [
    (Q4_K, 8, 7168, 1024, 2, 1, 0),     # gate/up rows of 112 segments
    (Q4_K, 8, 7168, 1024, 2, 3, 0),
    (Q4_K, 16, 7168, 512, 4, 2, 512),   # shared expert beside the routed ones
    (Q4_K, 4, 256, 6144, 2, 1, 0),      # down rows of 96 segments, combine in the kernel
    (Q4_K, 4, 256, 6144, 2, 5, 0),      # ... and per slot
    (Q4_0, 8, 4352, 512, 2, 2, 0),
    (Q8_0, 8, 4096, 1024, 2, 4, 0),     # 128 segments, two tokens per group
])
def test_two_wave_layer(ctx, fmt, E, H, F, k, T, shared):
    print(f"two-wave GEMV fmt={fmt} E={E} H={H} F={F} k={k} T={T} shared={shared}", flush=True)
    L = Layer(fmt, E, H, F, k, T, seed=E + H + F + T, shared_F=shared)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, 0, nx.PATH_GEMV)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL


@pytest.mark.parametrize("rows,T", [(333, 1), (333, 3), (7, 2), (1, 1)])
def test_two_wave_matvec(ctx, rows, T):
    cols = 6144
    print(f"two-wave matvec rows={rows} cols={cols} T={T}", flush=True)
    rng = np.random.default_rng(rows + T)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    q = oracle.quantize(Q4_K, w)
    wf = oracle.dequantize(Q4_K, q, rows * cols)
    m = nx.Matrix(ctx, Q4_K, rows, cols)
    m.load(q)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    got = m.matvec(x)
    m.close()
    for t in range(T):
        assert rel_l2(got[t], oracle.matvec(wf, rows, cols, x[t])) <= TOL
