"""One-token routing inside the gate/up GEMV (decode, E <= 256).

For one token the gate/up kernel routes the token itself (top-k with ties
to the lower index, softmax or sigmoid weights) and writes the route and
permutation arrays that the down pass and the combine read; there is no
router launch.  The routes it wrote (read back with nx_moe_last_routes) are
the oracle's route_moe_experts (src/engine/mod.rs:918-966): experts and
counts bit-exact, weights within 2 ulp (the device's exp is not glibc's
expf).  The layer's bar is the GEMV path's: relative L2 1e-4 against the
oracle's dispatch (src/engine/mod.rs:918-1024) over the same payloads, for
logits full of ties, signed zeros, NaN and infinities, k above E, the
256-expert limit and one past it (which takes the router kernels), a shared
expert, and one-token calls right after batches (no stale routes).
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import Q4_K, Q8_0, Layer, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4
POOL = np.array([0.0, -0.0, 1.0, 1.0, np.nan, np.inf, -np.inf, 0.5, -1.0], np.float32)


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def one_token(fmt, E, k, seed, special, score=0, shared_F=0, H=256, F=256):
    L = Layer(fmt, E, H, F, k, 1, seed=seed, shared_F=shared_F, score_mode=score,
              experts_needed=range(E))
    rng = np.random.default_rng(seed + 1)
    lg = rng.standard_normal(E).astype(np.float32)
    m = rng.random(E) < special
    lg[m] = POOL[rng.integers(0, POOL.size, m.sum())]
    L.logits = lg.reshape(1, E)
    return L


def assert_routes(ctx, logits, E, k, score):
    """The last forward's routes against the oracle router on the same logits."""
    T = logits.shape[0]
    ex, w, cnt = ctx.last_routes(T, k)
    rex, rw, rcnt, _ = oracle.route(logits, T, E, k, score)
    np.testing.assert_array_equal(cnt, rcnt)
    np.testing.assert_array_equal(ex, rex)
    ulp = np.abs(w.view(np.int32).astype(np.int64) - rw.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2, f"route weights differ by {ulp.max()} ulp"


@pytest.mark.parametrize("E,k,special,score", [
    (8, 2, 0.0, 0), (8, 2, 0.6, 0), (3, 7, 0.3, 0), (64, 8, 0.5, 1), (65, 4, 0.4, 0),
    (256, 8, 0.3, 0), (256, 64, 0.2, 1), (257, 8, 0.3, 0), (16, 16, 1.0, 0)])
def test_one_token_routing(ctx, E, k, special, score):
    print(f"one-token route E={E} k={k} special={special} score={score}", flush=True)
    L = one_token(Q8_0, E, k, seed=E * 31 + k, special=special, score=score)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, score, nx.PATH_GEMV)
    assert_routes(ctx, L.logits, E, k, score)
    ex.close()
    ref = L.oracle_out()
    assert rel_l2(got, ref) <= TOL


def test_one_token_no_finite_logits(ctx):
    L = one_token(Q4_K, 8, 2, seed=5, special=0.0, shared_F=256)
    L.logits[:] = np.array([np.nan, np.inf, -np.inf, np.nan, np.inf, np.nan, -np.inf, np.nan],
                           np.float32)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, 2, 0, nx.PATH_GEMV)
    assert_routes(ctx, L.logits, 8, 2, 0)
    assert ctx.last_routes(1, 2)[2][0] == 0
    ex.close()
    # no routes: only the shared expert contributes
    assert rel_l2(got, L.oracle_out()) <= TOL


def test_one_token_after_batches(ctx):
    """Alternating batch and one-token calls on one expert set: every call's
    routes are its own."""
    E, k, H, F = 32, 4, 256, 512
    big = Layer(Q4_K, E, H, F, k, 9, seed=77, experts_needed=range(E))
    ex = big.upload(nx, ctx)
    rng = np.random.default_rng(8)
    for i in range(4):
        got = ex.forward(big.x, big.logits, k, 0, nx.PATH_GEMV)
        assert_routes(ctx, big.logits, E, k, 0)
        assert rel_l2(got, big.oracle_out()) <= TOL
        lg = rng.standard_normal((1, E)).astype(np.float32)
        lg[0, rng.integers(0, E, 3)] = 2.5  # a three-way tie at the top
        one = Layer.__new__(Layer)
        one.__dict__.update(big.__dict__)
        one.x = big.x[i:i + 1].copy()
        one.logits = lg
        one.T = 1
        got1 = ex.forward(one.x, one.logits, k, 0, nx.PATH_GEMV)
        assert_routes(ctx, lg, E, k, 0)
        assert rel_l2(got1, one.oracle_out()) <= TOL
    ex.close()


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("E,k,score", [(8, 2, 0), (128, 8, 0), (256, 8, 1), (256, 64, 0),
                                       (5, 5, 1), (40, 3, 0)])
def test_one_token_routes_bit_exact(ctx, E, k, score, seed):
    """Many logit vectors through the in-kernel router: ties from a coarse
    value grid, signed zeros and non-finite values, at every decode shape
    (Mixtral E=8 k=2, Qwen3 E=128 k=8, DeepSeek E=256 k=8 sigmoid)."""
    rng = np.random.default_rng(1000 * E + 10 * k + seed)
    L = Layer(Q4_K, E, 256, 256, k, 1, seed=E + k, score_mode=score, experts_needed=[])
    ex = L.upload(nx, ctx)
    for rep in range(8):
        if rep % 2:
            lg = (rng.integers(-4, 5, E) * 0.25).astype(np.float32)  # many exact ties
        else:
            lg = rng.standard_normal(E).astype(np.float32)
        m = rng.random(E) < (0.1 * (rep % 4))
        lg[m] = POOL[rng.integers(0, POOL.size, m.sum())]
        lg = lg.reshape(1, E)
        ex.forward(L.x, lg, k, score, nx.PATH_GEMV)
        assert_routes(ctx, lg, E, k, score)
    ex.close()
