"""Q2_K on device (src/quant/mod.rs:851-937, src/gguf/mod.rs:1058-1088).

Bars: dequantization and the quantizer bit-exact against the oracle
(crafted blocks with special f16 scales and every scale/min nibble, random
data at several magnitudes, zero, positive-only and constant sub-blocks, a
ragged tail); the MoE layer with Q2_K experts on the GEMV path within
relative L2 1e-4 of the oracle over the same payloads (1 to 64 tokens, a
shared expert, the sigmoid score mode); the split-activation MFMA path to the
same bar (1 to 64 tokens, several tiles per expert, a shared expert as wide as
the routed ones, rows of very different magnitudes, Mixtral's full shape); the
grouped GEMM paths reject Q2_K with NX_ERR_UNSUPPORTED; AUTO gives the bits of
the path it picks.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import Q2_K, Layer, assert_same_bits, rel_l2
from test_oracle_quant import crafted_blocks

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def test_q2k_dequant_crafted(ctx):
    data = crafted_blocks(Q2_K, 512, seed=77)
    n = 512 * 256
    assert_same_bits(ctx.dequant(Q2_K, data, n), oracle.dequantize(Q2_K, data, n))
    # output length mid-block, and a truncated payload
    assert_same_bits(ctx.dequant(Q2_K, data, n - 100), oracle.dequantize(Q2_K, data, n - 100))
    with pytest.raises(nx.NexusError) as ei:
        ctx.dequant(Q2_K, data[:84 * 3], 4 * 256)
    assert str(ei.value) == "Q2_K tensor payload is truncated"


@pytest.mark.parametrize("scale", [1e-3, 0.02, 1.0, 300.0])
def test_q2k_quantize_bit_exact(ctx, scale):
    rng = np.random.default_rng(int(scale * 1000) + 1)
    n = 97 * 256 + 131  # ragged last block
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    x[:256] = 0.0
    x[256:512] = np.abs(x[256:512])
    x[512:528] = np.float32(scale)
    x[1000] = np.float32(3e38)
    x[2000] = np.float32(-1e-40)
    got = ctx.quantize(Q2_K, x)
    want = oracle.quantize(Q2_K, x)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("E,H,F,k,T,shared,score", [
    (8, 512, 1024, 2, 1, 0, 0), (8, 1024, 512, 2, 5, 0, 0), (16, 256, 768, 4, 16, 256, 1),
    (32, 512, 256, 8, 64, 0, 0),
    (4, 4096, 512, 2, 1, 0, 0),     # gate/up rows of 64 segments: one wave per row, shared operands
    (4, 4096, 512, 2, 2, 0, 0),     # the same, two tokens per group
    (4, 512, 14336, 2, 1, 0, 0),    # down rows of 224 segments: K slices
    (8, 7168, 256, 4, 1, 256, 1)])  # gate/up rows of 112 segments: two-wave row groups
def test_q2k_layer_gemv_parity(ctx, E, H, F, k, T, shared, score):
    print(f"q2k layer E={E} H={H} F={F} k={k} T={T} shared={shared}", flush=True)
    L = Layer(Q2_K, E, H, F, k, T, seed=E + H + F + T, shared_F=shared, score_mode=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_GEMV)
    ex.close()
    ref = L.oracle_out()
    assert rel_l2(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("E,H,F,k,T,shared,score", [
    (8, 512, 1024, 2, 1, 0, 0), (8, 1024, 512, 2, 5, 0, 0), (8, 256, 768, 2, 33, 0, 0),
    (32, 512, 256, 8, 24, 0, 1), (16, 1024, 512, 4, 64, 0, 0),
    (16, 512, 512, 4, 8, 512, 1), (8, 256, 768, 2, 40, 768, 0),
    (4, 4096, 512, 2, 3, 0, 0), (4, 512, 14336, 2, 6, 0, 0)])
def test_q2k_layer_split_parity(ctx, E, H, F, k, T, shared, score):
    """Q2_K on the split-activation MFMA path: segment g of a 256-weight
    chunk per lane group, each 16-weight sub-block's 4-bit scale inside the
    code operands and its 4-bit min in operands of its own."""
    print(f"q2k split E={E} H={H} F={F} k={k} T={T} shared={shared}", flush=True)
    L = Layer(Q2_K, E, H, F, k, T, seed=E * 3 + H + F + T, shared_F=shared, score_mode=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= GEMV_TOL


def test_q2k_split_magnitudes_and_mixtral_shape(ctx):
    L = Layer(Q2_K, 8, 512, 512, 2, 12, seed=45)
    scale = np.array([1e-30, 1e-6, 1.0, 3e3, 1e6, 0.0, 1.0, 1e-3, 7.0, 0.0, 1e4, 1e-2],
                     np.float32)[:, None]
    L.x = (L.x * scale).astype(np.float32)
    L.x[2, 256:] = 0.0  # one zero chunk inside a live row
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    ex.close()
    ref = L.oracle_out()
    for t in range(L.T):
        den = np.linalg.norm(ref[t])
        if den == 0:
            assert np.all(got[t] == 0)
        else:
            assert rel_l2(got[t], ref[t]) <= GEMV_TOL, t
    M = Layer(Q2_K, 8, 4096, 14336, 2, 8, seed=11)
    ex = M.upload(nx, ctx)
    got = ex.forward(M.x, M.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, M.oracle_out()) <= GEMV_TOL


def test_q2k_prefill_size_split_matches_gemv(ctx):
    """Q2_K has no grouped GEMM, so prefill-sized batches run on the split
    path (here 512 tokens at Mixtral's shape: 1024 pairs in 64+ tiles, K-slice
    partial sums of ~235 MB): every row within 2e-4 of the GEMV's (each path
    is within 1e-4 of the oracle at this shape with 8 tokens, above)."""
    T = 512
    print(f"q2k split vs gemv, Mixtral shape, T={T}", flush=True)
    L = Layer(Q2_K, 8, 4096, 14336, 2, T, seed=12, experts_needed=[])
    ex = L.upload(nx, ctx)
    split = ex.forward(L.x, L.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    gemv = ex.forward(L.x, L.logits, 2, 0, nx.PATH_GEMV)
    auto = ex.forward(L.x, L.logits, 2, 0, nx.PATH_AUTO)
    ex.close()
    assert np.isfinite(split).all()
    worst = max(rel_l2(split[t], gemv[t]) for t in range(T))
    assert worst <= 2 * GEMV_TOL, worst
    assert_same_bits(auto, split)


def test_q2k_rejects_mfma(ctx):
    L = Layer(Q2_K, 4, 256, 256, 2, 4, seed=3)
    ex = L.upload(nx, ctx)
    for path in (nx.PATH_MFMA_F16, nx.PATH_MFMA_BF16):
        with pytest.raises(nx.NexusError) as ei:
            ex.forward(L.x, L.logits, 2, 0, path)
        assert ei.value.code == nx.NX_ERR_UNSUPPORTED
    ex.close()
