"""Few-token MoE layer on MFMA with split-fp16 activations (NX_PATH_MFMA_SPLIT).

The Q4_K codes go into fp16 MFMA operands untouched (no dequantization) and
each 32-weight sub-block's scale and offset are applied to the products;
activations are split per pair and 256-element chunk into two fp16 halves
after a power-of-two scaling.  Bar: the GEMV path's, relative L2 1e-4
against the oracle's dispatch (src/engine/mod.rs:969-1024) over the same
payloads: 1 to 64 tokens, experts with more than 16 tokens (several tiles),
top-8 routing, the sigmoid score mode, token rows of very different
magnitudes and zero rows, Mixtral's full shape, and a shared expert as wide
as the routed ones (one pair per token, several tiles of 16); Q4_0 and Q8_0
experts whose widths are whole 256-weight chunks on the same kinds of case;
other formats, other Q4_0 and Q8_0 widths and shared experts of another width
are rejected with NX_ERR_UNSUPPORTED.
"""
import numpy as np
import pytest

import nexus_amd as nx
from moe_cases import F32, Q2_K, Q4_0, Q4_K, Q8_0, Layer, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("E,H,F,k,T,score", [
    (8, 512, 1024, 2, 1, 0), (8, 512, 1024, 2, 5, 0), (8, 256, 768, 2, 33, 0),
    (32, 512, 256, 8, 24, 1), (16, 1024, 512, 4, 64, 0), (4, 256, 256, 1, 40, 0)])
def test_split_parity(ctx, E, H, F, k, T, score):
    print(f"mfma split E={E} H={H} F={F} k={k} T={T} score={score}", flush=True)
    L = Layer(Q4_K, E, H, F, k, T, seed=E * 5 + H + F + T, score_mode=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL


@pytest.mark.parametrize("E,H,F,k,T,score", [
    (16, 512, 512, 4, 1, 1), (16, 512, 512, 4, 8, 1), (8, 256, 768, 2, 40, 0),
    (64, 1024, 256, 8, 17, 1)])
def test_split_parity_shared_expert(ctx, E, H, F, k, T, score):
    """A shared expert (every token, after the routed experts) on the split
    path: its tiles come after the routed ones in the permutation's list."""
    print(f"mfma split shared E={E} H={H} F={F} k={k} T={T} score={score}", flush=True)
    L = Layer(Q4_K, E, H, F, k, T, seed=E * 7 + H + F + T, shared_F=F, score_mode=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL


@pytest.mark.parametrize("T,k", [(31, 8), (32, 8), (33, 8), (32, 16), (64, 8)])
def test_fused_router_limits(ctx, T, k):
    """Batches around the one-workgroup router's limits (32 tokens, 512
    pairs; beyond them the router and permutation kernels run), on the split
    path and the GEMV."""
    L = Layer(Q4_K, 64, 256, 512, k, T, seed=T + k)
    ex = L.upload(nx, ctx)
    split = ex.forward(L.x, L.logits, k, 0, nx.PATH_MFMA_SPLIT)
    gemv = ex.forward(L.x, L.logits, k, 0, nx.PATH_GEMV)
    ex.close()
    ref = L.oracle_out()
    assert rel_l2(split, ref) <= TOL
    assert rel_l2(gemv, ref) <= TOL


def test_split_magnitudes_and_zero_rows(ctx):
    L = Layer(Q4_K, 8, 512, 512, 2, 12, seed=41)
    scale = np.array([1e-30, 1e-6, 1.0, 3e3, 1e6, 0.0, 1.0, 1e-3, 7.0, 0.0, 1e4, 1e-2],
                     np.float32)[:, None]
    L.x = (L.x * scale).astype(np.float32)
    L.x[2, :256] = 0.0  # one zero chunk inside a live row
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    ex.close()
    ref = L.oracle_out()
    # per row, so that small rows are held to their own scale
    for t in range(L.T):
        den = np.linalg.norm(ref[t])
        if den == 0:
            assert np.all(got[t] == 0)
        else:
            assert rel_l2(got[t], ref[t]) <= TOL, t


def test_split_mixtral_shape(ctx):
    L = Layer(Q4_K, 8, 4096, 14336, 2, 8, seed=9)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL


@pytest.mark.parametrize("fmt", [Q4_0, Q8_0])
@pytest.mark.parametrize("E,H,F,k,T,Fs,score", [
    (8, 512, 1024, 2, 1, 0, 0), (8, 256, 768, 2, 33, 0, 0), (32, 512, 256, 8, 24, 0, 1),
    (16, 1024, 512, 4, 64, 0, 0), (16, 512, 512, 4, 8, 512, 1), (8, 256, 768, 2, 40, 768, 0)])
def test_split_parity_block_formats(ctx, fmt, E, H, F, k, T, Fs, score):
    """Q4_0 experts (w = d (q - 8) per 32-weight block, src/quant/mod.rs:
    723-745) and Q8_0 experts (w = d q, q a signed byte, :689-703) on the
    split path: one MFMA per block with the codes made unsigned, the block
    sums of the staged activations taking off the offset (8, 128)."""
    print(f"mfma split fmt={fmt} E={E} H={H} F={F} k={k} T={T} Fs={Fs} score={score}", flush=True)
    L = Layer(fmt, E, H, F, k, T, seed=E * 3 + H + F + T + fmt, shared_F=Fs, score_mode=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL


@pytest.mark.parametrize("fmt", [Q4_0, Q8_0])
def test_split_block_formats_magnitudes_and_mixtral_shape(ctx, fmt):
    L = Layer(fmt, 8, 512, 512, 2, 12, seed=43 + fmt)
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
            assert rel_l2(got[t], ref[t]) <= TOL, t
    M = Layer(fmt, 8, 4096, 14336, 2, 8, seed=10 + fmt)
    ex = M.upload(nx, ctx)
    got = ex.forward(M.x, M.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, M.oracle_out()) <= TOL


def _sweep_cases(n=16, seed=2026):
    """Seeded random split-path layers: every format, widths in whole
    256-weight chunks (1 to 6 chunks, so K slices of 1 to 4 chunks and
    partial last slices), 2 to 40 experts, top-1 to top-8, 1 to 70 tokens,
    with and without a shared expert, both score modes."""
    rng = np.random.default_rng(seed)
    fmts = [Q4_K, Q4_0, Q8_0, Q2_K]
    out = []
    for i in range(n):
        fmt = fmts[i % 4]
        E = int(rng.integers(2, 41))
        k = int(rng.integers(1, min(8, E) + 1))
        H = 256 * int(rng.integers(1, 7))
        F = 256 * int(rng.integers(1, 7))
        T = int(rng.integers(1, 71))
        Fs = F if rng.random() < 0.3 else 0
        out.append((fmt, E, H, F, k, T, Fs, int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: "-".join(map(str, c)))
def test_split_random_shapes(ctx, case):
    fmt, E, H, F, k, T, Fs, score = case
    print(f"mfma split sweep fmt={fmt} E={E} H={H} F={F} k={k} T={T} Fs={Fs} score={score}",
          flush=True)
    L = Layer(fmt, E, H, F, k, T, seed=E + H + F + T + fmt, shared_F=Fs, score_mode=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_MFMA_SPLIT)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL


def test_split_rejects(ctx):
    L = Layer(F32, 4, 256, 256, 2, 4, seed=3)
    ex = L.upload(nx, ctx)
    with pytest.raises(nx.NexusError) as ei:
        ex.forward(L.x, L.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    assert ei.value.code == nx.NX_ERR_UNSUPPORTED
    ex.close()
    # Q4_0 and Q8_0 widths that are not whole 256-weight chunks
    for fmt, H, F in ((Q4_0, 288, 256), (Q4_0, 256, 224), (Q8_0, 288, 256), (Q8_0, 256, 224)):
        Q = Layer(fmt, 4, H, F, 2, 4, seed=5)
        ex = Q.upload(nx, ctx)
        with pytest.raises(nx.NexusError) as ei:
            ex.forward(Q.x, Q.logits, 2, 0, nx.PATH_MFMA_SPLIT)
        assert ei.value.code == nx.NX_ERR_UNSUPPORTED
        ex.close()
    S = Layer(Q4_K, 4, 256, 256, 2, 4, seed=4, shared_F=512)  # a wider shared expert
    ex = S.upload(nx, ctx)
    with pytest.raises(nx.NexusError) as ei:
        ex.forward(S.x, S.logits, 2, 0, nx.PATH_MFMA_SPLIT)
    assert ei.value.code == nx.NX_ERR_UNSUPPORTED
    ex.close()


@pytest.mark.parametrize("E,H,F,k,T,want", [
    (8, 512, 1024, 2, 1, nx.PATH_GEMV), (8, 512, 1024, 2, 8, nx.PATH_GEMV),
    (8, 512, 1024, 2, 16, nx.PATH_MFMA_SPLIT), (64, 256, 256, 8, 8, nx.PATH_MFMA_SPLIT),
    (8, 256, 256, 2, 64, nx.PATH_MFMA_BF16), (8, 256, 256, 2, 256, nx.PATH_MFMA_BF16)])
def test_auto_path_choice(ctx, E, H, F, k, T, want):
    """AUTO gives the bits of the path it chooses for Q4_K: the GEMV up to ~2
    tokens per expert, the split-activation MFMA path up to ~12, the grouped
    GEMM beyond."""
    L = Layer(Q4_K, E, H, F, k, T, seed=E + T)
    ex = L.upload(nx, ctx)
    auto = ex.forward(L.x, L.logits, k, 0, nx.PATH_AUTO)
    chosen = ex.forward(L.x, L.logits, k, 0, want)
    ex.close()
    np.testing.assert_array_equal(auto.view(np.uint32), chosen.view(np.uint32))


@pytest.mark.parametrize("fmt,E,H,F,k,T,shared,want", [
    (Q8_0, 8, 512, 1024, 2, 8, 0, nx.PATH_GEMV),        # 2 tokens per expert
    (Q8_0, 8, 512, 1024, 2, 16, 0, nx.PATH_MFMA_SPLIT),  # 4
    (Q8_0, 8, 512, 1024, 2, 64, 0, nx.PATH_MFMA_BF16),   # 16
    (Q8_0, 8, 288, 1024, 2, 16, 0, nx.PATH_MFMA_BF16),   # H not whole 256-weight chunks
    (Q4_0, 8, 512, 1024, 2, 4, 0, nx.PATH_GEMV),         # 1 token per expert
    (Q4_0, 8, 512, 1024, 2, 16, 0, nx.PATH_MFMA_SPLIT),  # 4
    (Q4_0, 8, 512, 1024, 2, 64, 0, nx.PATH_MFMA_BF16),   # 16
    (Q4_0, 8, 512, 992, 2, 16, 0, nx.PATH_MFMA_BF16),    # F not whole 256-weight chunks
    (Q4_0, 16, 512, 512, 4, 8, 512, nx.PATH_MFMA_BF16),  # a shared expert, 8 tokens
    (Q2_K, 8, 512, 1024, 2, 4, 0, nx.PATH_GEMV),         # 1.5 tokens per expert
    (Q2_K, 8, 512, 1024, 2, 8, 0, nx.PATH_MFMA_SPLIT),   # 2.2
    (Q2_K, 8, 256, 256, 2, 256, 0, nx.PATH_MFMA_SPLIT),  # 64: no grouped GEMM for Q2_K
    (Q2_K, 16, 512, 512, 4, 2, 512, nx.PATH_GEMV),         # a shared expert, 2 tokens
    (Q2_K, 16, 512, 512, 4, 4, 512, nx.PATH_MFMA_SPLIT),   # ... 4 tokens
    (Q2_K, 16, 256, 768, 4, 16, 256, nx.PATH_GEMV),        # a narrower shared expert
    (Q4_K, 16, 512, 512, 4, 2, 512, nx.PATH_GEMV),        # a shared expert, 2 tokens
    (Q4_K, 16, 512, 512, 4, 4, 512, nx.PATH_MFMA_SPLIT),  # ... 4 tokens
    (Q4_K, 16, 512, 512, 4, 8, 512, nx.PATH_MFMA_SPLIT),  # ... 8 tokens
    (Q4_K, 16, 512, 512, 4, 24, 512, nx.PATH_MFMA_SPLIT),  # ... 6 tokens per routed expert
    (Q4_K, 16, 512, 512, 4, 32, 512, nx.PATH_MFMA_BF16),   # ... 8 tokens per routed expert
    (Q4_K, 4, 256, 256, 2, 48, 256, nx.PATH_MFMA_BF16),   # ... 24 tokens per routed expert
    (Q4_K, 16, 512, 512, 4, 8, 1024, nx.PATH_MFMA_BF16)])  # a wider shared expert, 8 tokens
def test_auto_path_choice_other(ctx, fmt, E, H, F, k, T, shared, want):
    """AUTO for formats other than Q4_K and for layers with a shared expert:
    the grouped GEMM from ~3 tokens per routed expert, or from 6 tokens with
    a shared expert, the GEMV below; Q4_0 and Q8_0 without a shared expert,
    in whole 256-weight chunks, follow Q4_K's rule (split path from ~3 tokens per
    expert up to 12); Q2_K takes the split path from ~1.8 tokens per expert
    (or 4 tokens with a shared expert as wide as the routed ones), the GEMV
    below; Q4_K with a shared expert as wide as the routed ones
    takes the split-activation path from 4 tokens up to 8 tokens per routed
    expert (the bits of the chosen path)."""
    L = Layer(fmt, E, H, F, k, T, seed=E + T + fmt, shared_F=shared)
    ex = L.upload(nx, ctx)
    auto = ex.forward(L.x, L.logits, k, 0, nx.PATH_AUTO)
    chosen = ex.forward(L.x, L.logits, k, 0, want)
    ex.close()
    np.testing.assert_array_equal(auto.view(np.uint32), chosen.view(np.uint32))
