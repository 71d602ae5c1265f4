"""Router logits on device (nx_router_logits / nx_router_logits_dev) against the
oracle's InferenceEngine::matvec (src/engine/mod.rs:775-801).

Bars: exact mode bit-identical to the oracle's sequential, unfused f32 matvec
for every token row (NaN positions identical, payloads not compared); fast
mode within 2 (H+1) 2^-24 sum_c |w x| of the exact logits, the bound that holds
for any two summation orders of the same rounded-or-fused products.  The
shapes cover every kernel the dispatcher picks: eight-lane chains (few
chains, rows not a multiple of 4 floats, unaligned device pointers), LDS tiles
with 1x1, 2x2 and 4x4 chains per lane (partial tiles in tokens, experts and
columns), the fast workgroup dot product, the fast register-held weights for
at most 8 experts, and the fast f32 MFMA tiles.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import DeviceArray, assert_same_bits

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def say(*a):
    print(*a, flush=True)


def oracle_logits(w, x, E, H):
    T = x.shape[0]
    out = np.empty((T, E), np.float32)
    for t in range(T):
        out[t] = oracle.matvec(w, E, H, x[t])
    return out


def data(seed, T, E, H, scale=0.05):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((E, H)) * scale).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    return w, x


def fast_bound(w, x):
    H = w.shape[1]
    absdot = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    return 2.0 * (H + 1) * U / (1 - (H + 1) * U) * absdot + 1e-38


# (T, E, H): register-run chains (rows of whole float4 up to 4096 on 32-lane
# chains in groups of 8 experts, up to 7168 on 64-lane chains in groups of 4;
# at most 256 groups: partial groups, partial last runs, the limit either
# side), chain-kernel shapes, rows not a multiple of 4 floats or 32 columns,
# then tiled grids with each register block (1x1: up to 256K chains, 2x2: up
# to 1M, 4x4 beyond) and partial tiles
EXACT_SHAPES = [
    (1, 8, 4096), (1, 128, 2048), (1, 256, 7168), (4, 8, 4096), (3, 60, 2880),
    (32, 8, 4096), (1, 20, 1056), (2, 128, 4), (16, 128, 1024), (17, 128, 1024),
    (2, 10, 4100), (3, 7, 5000), (4, 256, 7168), (5, 256, 7168),
    (2, 7, 1001), (5, 3, 100), (1, 1, 1), (64, 256, 512),
    (300, 64, 512), (2100, 8, 256), (700, 40, 128), (1500, 12, 64),
    (1024, 256, 1024), (4096, 128, 256), (8192, 256, 64),
]


@pytest.mark.parametrize("T,E,H", EXACT_SHAPES)
def test_exact_bit_identical_to_reference_matvec(ctx, T, E, H):
    say(f"router logits exact T={T} E={E} H={H}")
    w, x = data(1000 + T + E + H, T, E, H)
    got = ctx.router_logits(w, x, E, H, exact=True)
    ref = oracle_logits(w, x, E, H)
    assert_same_bits(got, ref)


def test_exact_order_matters(ctx):
    # a case where the sequential order and a pairwise order round differently,
    # so matching bits is evidence of the order and not of luck
    T, E, H = 2, 16, 4096
    w, x = data(7, T, E, H, scale=1.0)
    got = ctx.router_logits(w, x, E, H, exact=True)
    ref = oracle_logits(w, x, E, H)
    assert_same_bits(got, ref)
    prod = (w[None, :, :] * x[:, None, :]).astype(np.float32)
    pairwise = prod.sum(axis=2, dtype=np.float32)  # numpy pairwise summation
    assert np.any(pairwise != ref)


def test_exact_special_values(ctx):
    T, E, H = 4, 9, 96
    w, x = data(8, T, E, H)
    w[0, :] = 1e-20                 # products below the normal range (subnormal sums)
    x[0, :] = 1e-20
    x[1, 5] = np.inf                # inf * w -> +-inf, NaN where w == 0
    w[3, 5] = 0.0
    x[2, 7] = np.nan
    x[3, :] = -0.0                  # all-zero products: +0.0 result
    w[4, :] = 3e38                  # overflow to inf mid-chain
    w[5, ::2] = 3e38
    w[5, 1::2] = -3e38
    got = ctx.router_logits(w, x, E, H, exact=True)
    ref = oracle_logits(w, x, E, H)
    assert_same_bits(got, ref)
    assert np.signbit(got[3]).sum() == 0
    assert got[0, 0] != 0.0 and abs(got[0, 0]) < 1.2e-38  # subnormal kept, not flushed


# (T, E, H): the workgroup dot product (up to 32 tokens, partial token blocks;
# rows not a multiple of 4 floats on the chain kernel), then the f32 MFMA
# tiles (more tokens): 16 x 16 with K
# split four ways (up to 16 experts), one 32 x 32 tile per workgroup with K
# split (fewer than two workgroups per CU of output tiles), four 32 x 32
# tiles per workgroup; partial token and expert tiles and a partial last
# 16-column step (H % 16 != 0) on each
FAST_SHAPES = [(1, 8, 4096), (1, 256, 7168), (3, 128, 2048), (8, 60, 2880), (2, 7, 1001),
               (64, 256, 512), (2100, 8, 256), (4096, 128, 256), (9, 8, 4096), (50, 5, 100),
               (1000, 40, 1000), (8200, 250, 72), (1030, 256, 7168), (32, 8, 4096),
               (27, 128, 2048), (33, 9, 4096),
               # at most 8 experts from 33 tokens: W held in registers, rows streamed
               (2048, 8, 4096), (40, 3, 1536), (100, 8, 4000), (4097, 1, 2048), (300, 8, 1024)]


@pytest.mark.parametrize("T,E,H", FAST_SHAPES)
def test_fast_within_order_bound(ctx, T, E, H):
    say(f"router logits fast T={T} E={E} H={H}")
    w, x = data(2000 + T + E + H, T, E, H)
    fast = ctx.router_logits(w, x, E, H, exact=False)
    exact = oracle_logits(w, x, E, H)
    err = np.abs(fast.astype(np.float64) - exact.astype(np.float64))
    assert np.all(err <= fast_bound(w, x)), float(np.max(err / fast_bound(w, x)))


def test_exact_logits_route_like_reference(ctx):
    T, E, H, k = 16, 64, 1024, 6
    w, x = data(9, T, E, H)
    got = ctx.router_logits(w, x, E, H, exact=True)
    ex, wt, cnt, lists = ctx.route_topk(got, T, E, k)
    rex, rwt, rcnt, rlists = oracle.route(oracle_logits(w, x, E, H), T, E, k)
    assert lists == rlists == T
    np.testing.assert_array_equal(cnt, rcnt)
    np.testing.assert_array_equal(ex, rex)


def test_shape_errors_match_reference(ctx):
    E, H = 4, 8
    w, x = data(10, 2, E, H)
    with pytest.raises(nx.NexusError, match=r"^Matvec input shape mismatch: got 15, expected 16$"):
        ctx.router_logits_raw(w, w.size, x, 15, 2, E, H)
    with pytest.raises(nx.NexusError, match=r"^Matvec input shape mismatch: got 7, expected 8$"):
        ctx.router_logits_raw(w, w.size, x, 7, 1, E, H)
    with pytest.raises(nx.NexusError, match=r"^Matvec weight too small: got 31, expected at least 32$"):
        ctx.router_logits_raw(w, 31, x, 16, 2, E, H)
    # input checked before weight, as in the reference
    with pytest.raises(nx.NexusError, match=r"^Matvec input shape mismatch"):
        ctx.router_logits_raw(w, 3, x, 3, 2, E, H)
    with pytest.raises(nx.NexusError) as ei:
        ctx.router_logits_raw(w, w.size, x, 16, -2, E, H)
    assert ei.value.code == nx.NX_ERR_INVALID_ARG
    # a longer weight is accepted (only the first E*H floats are read)
    long_w = np.concatenate([w.ravel(), np.full(5, np.nan, np.float32)])
    got = ctx.router_logits_raw(long_w, long_w.size, x, 16, 2, E, H)
    assert_same_bits(got, oracle_logits(w.ravel(), x, E, H))


def test_empty_sizes(ctx):
    got = ctx.router_logits(np.zeros(0, np.float32), np.zeros((3, 0), np.float32), 5, 0)
    assert got.shape == (0, 5) or got.size == 0
    # H = 0 with tokens: matvec returns zeros
    out = ctx.router_logits_raw(np.zeros(1, np.float32), 0, np.zeros(1, np.float32), 0, 3, 5, 0)
    assert out.shape == (3, 5) and np.all(out == 0) and not np.any(np.signbit(out))
    out = ctx.router_logits_raw(np.zeros(35, np.float32), 35, np.zeros(1, np.float32), 0, 0, 5, 7)
    assert out.size == 0
    # the weight is checked against E*H even when there are no tokens
    with pytest.raises(nx.NexusError, match=r"^Matvec weight too small: got 0, expected at least 35$"):
        ctx.router_logits_raw(np.zeros(1, np.float32), 0, np.zeros(1, np.float32), 0, 0, 5, 7)


@pytest.mark.parametrize("exact", [True, False])
def test_dev_entry_unaligned_and_reused(ctx, exact):
    T, E, H = 5, 24, 1024
    w, x = data(12, T, E, H)
    # device copies offset by one float so the rows are not 16-byte aligned
    dw, dx = DeviceArray(E * H + 1), DeviceArray(T * H + 1)
    dw.upload(w, 1)
    dx.upload(x, 1)
    out = DeviceArray(T * E + 1, fill=np.nan)
    ref = oracle_logits(w, x, E, H)
    for _ in range(2):
        ctx.router_logits_dev(dw.ptr + 4, E * H, dx.ptr + 4, T * H, T, E, H, out.ptr + 4,
                              exact=exact)
        ctx.sync()
        o = out.download()
        got = o[1:].reshape(T, E)
        if exact:
            assert_same_bits(got, ref)
        else:
            err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
            assert np.all(err <= fast_bound(w, x))
        assert np.isnan(o[0])  # nothing written before the output
