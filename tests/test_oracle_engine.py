"""Pins the oracle's router, permutation and layer arithmetic.

Anchors: the reference's engine tests (src/engine/mod.rs:1622-1656, with the
closed form of the dispatch test), the matmul known answer
(src/backend/cpu.rs:234-241), brute force against Python's stable sort with an
independent total-order key, identity-weight and linearity properties, and a
float64 numpy statement of the layer.
"""
import math
import struct

import numpy as np
import pytest


# ----------------------------------------------------------------------------- router
def test_reference_router_case(oracle):
    """src/engine/mod.rs:1622-1630."""
    ex, w, cnt, n = oracle.route([0.1, 3.0, 1.0, 2.0, 0.5, 0.2], 2, 3, 2)
    assert n == 2
    assert ex[0].tolist() == [1, 2]
    assert abs(float(w[0].sum()) - 1.0) < 1e-6
    assert ex[1].tolist() == [0, 1]


def _total_key(f):
    """IEEE totalOrder as an integer, written from the definition."""
    b = struct.unpack("<i", struct.pack("<f", f))[0]
    return b if b >= 0 else -(b & 0x7FFFFFFF) - 1


def brute_route(logits, T, E, k):
    out = []
    for t in range(T):
        if (t + 1) * E > len(logits):
            break
        row = [(e, float(np.float32(logits[t * E + e]))) for e in range(E)]
        row = [(e, v) for e, v in row if math.isfinite(v)]
        # Python's sort is stable: descending key, ties keep ascending index order
        row = sorted(row, key=lambda ev: -_total_key(ev[1]))
        out.append(row[: min(k, E)])
    return out


@pytest.mark.parametrize("seed", range(40))
def test_router_brute_force(oracle, seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 12))
    T = int(rng.integers(1, 6))
    k = int(rng.integers(0, E + 3))
    pool = np.array([0.0, -0.0, 1.0, -1.0, 0.5, np.nan, np.inf, -np.inf, 2.0, 1e-30, -1e-30],
                    np.float32)
    lg = np.where(rng.random(T * E) < 0.5, pool[rng.integers(0, pool.size, T * E)],
                  rng.standard_normal(T * E).astype(np.float32)).astype(np.float32)
    short = int(rng.integers(0, 2))
    L = lg.size - short * int(rng.integers(0, E + 1))
    ex, w, cnt, n = oracle.route(lg[:L], T, E, k)
    ref = brute_route(lg[:L].tolist(), T, E, k) if k > 0 else []
    assert n == len(ref)
    for t, row in enumerate(ref):
        assert cnt[t] == len(row)
        assert ex[t, : len(row)].tolist() == [e for e, _ in row]
        assert all(v == -1 for v in ex[t, len(row):])
        if row:
            m = max(v for _, v in row)
            p = np.array([math.exp(v - m) for _, v in row])
            p /= p.sum()
            np.testing.assert_allclose(w[t, : len(row)], p, rtol=3e-7, atol=1e-30)
            # closed form: the top weight is 1 / sum(exp(l_i - l_max))
            assert abs(w[t, 0] - 1.0 / np.exp(np.array([v - m for _, v in row])).sum()) < 3e-7


def test_router_ties_and_signed_zero(oracle):
    lg = np.array([1.0, 3.0, 3.0, -0.0, 0.0, 3.0], np.float32)
    ex, w, cnt, _ = oracle.route(lg, 1, 6, 6)
    assert ex[0].tolist() == [1, 2, 5, 0, 4, 3]  # ties -> lower index; +0 above -0
    ex, w, cnt, _ = oracle.route(np.array([-0.0, 0.0], np.float32), 1, 2, 2)
    assert ex[0].tolist() == [1, 0]


def test_router_degenerate(oracle):
    assert oracle.route([1.0, 2.0], 1, 2, 0)[3] == 0
    assert oracle.route([1.0, 2.0], 0, 2, 1)[3] == 0
    ex, w, cnt, n = oracle.route([np.nan, np.inf], 1, 2, 2)
    assert n == 1 and cnt[0] == 0 and ex[0].tolist() == [-1, -1]
    ex, w, cnt, n = oracle.route([1.0, 2.0, 3.0], 1, 3, 9)  # k > E clamps
    assert cnt[0] == 3 and ex[0, :3].tolist() == [2, 1, 0]


def test_sigmoid_mode_invariants(oracle):
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal(64 * 32) * 0.02).astype(np.float32)
    ex0, _, c0, _ = oracle.route(lg, 64, 32, 8, score_mode=0)
    ex1, w1, c1, _ = oracle.route(lg, 64, 32, 8, score_mode=1)
    assert np.array_equal(ex0, ex1) and np.array_equal(c0, c1)  # same selection
    np.testing.assert_allclose(w1.sum(axis=1), 1.0, atol=1e-6)
    sig = 1.0 / (1.0 + np.exp(-lg.reshape(64, 32).astype(np.float64)))
    sel = np.take_along_axis(sig, ex1.astype(np.int64), axis=1)
    np.testing.assert_allclose(w1, sel / sel.sum(axis=1, keepdims=True), rtol=1e-6)
    assert np.all(np.diff(w1, axis=1) <= 0)  # monotone scores keep descending order


# ----------------------------------------------------------------------------- permutation
@pytest.mark.parametrize("seed", range(10))
def test_permutation_brute_force(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    T, E, k = int(rng.integers(1, 300)), int(rng.integers(1, 40)), int(rng.integers(1, 9))
    lg = rng.standard_normal(T * E).astype(np.float32)
    lg[rng.random(T * E) < 0.1] = np.nan
    ex, w, cnt, _ = oracle.route(lg, T, E, k)
    ec, off, pt, ps, inv = oracle.permute(ex, cnt, E)
    pairs = sorted(((int(ex[t, r]), t, r) for t in range(T) for r in range(cnt[t])))
    assert [(t, r) for _, t, r in pairs] == list(zip(pt.tolist(), ps.tolist()))
    assert ec.tolist() == [sum(1 for e, _, _ in pairs if e == x) for x in range(E)]
    assert off[0] == 0 and np.array_equal(np.diff(off), ec) and off[-1] == cnt.sum()
    for p, (t, r) in enumerate(zip(pt, ps)):
        assert inv[t, r] == p
    assert np.all(inv[np.arange(k)[None, :] >= cnt[:, None]] == -1)


# ----------------------------------------------------------------------------- engine
def _identity(rows, cols):
    w = np.zeros(rows * cols, np.float32)
    for i in range(min(rows, cols)):
        w[i * cols + i] = 1.0
    return w


def test_reference_dispatch_case_closed_form(oracle):
    """src/engine/mod.rs:1632-1656, value fixed by hand: expert 1 (w=1), g=u/0.5*...:
    g = [1.5,1.5], u = [0.75,0.75], a = silu(1.5)*0.75, y = 0.1*(a+a)."""
    out = oracle.dispatch_moe_ffn([1.0, 2.0], [0.0, 4.0],
                                  [_identity(2, 2), np.full(4, 0.5)],
                                  [_identity(2, 2), np.full(4, 0.25)],
                                  [_identity(2, 2), np.full(4, 0.1)], 1, 2, 2)
    a = 1.5 / (1.0 + math.exp(-1.5)) * 0.75
    assert out.shape == (2,)
    np.testing.assert_allclose(out, [0.2 * a, 0.2 * a], rtol=1e-6)
    assert abs(out[0] - 0.18395) < 1e-5


def test_dispatch_error_strings(oracle):
    I2 = _identity(2, 2)
    with pytest.raises(oracle.OracleError, match=r"^MoE hidden shape mismatch: got 3, expected 2$"):
        oracle.dispatch_moe_ffn([1, 2, 3], [0, 1], [I2, I2], [I2, I2], [I2, I2], 1, 2, 2)
    with pytest.raises(oracle.OracleError, match=r"^MoE router produced no routes$"):
        oracle.dispatch_moe_ffn([1, 2], [0, 1], [I2, I2], [I2, I2], [I2, I2], 0, 2, 2)
    with pytest.raises(oracle.OracleError, match=r"^MoE router produced no routes$"):
        oracle.dispatch_moe_ffn([1, 2], [0], [I2, I2], [I2, I2], [I2, I2], 1, 2, 2)
    with pytest.raises(oracle.OracleError,
                       match=r"^Matvec weight too small: got 3, expected at least 4$"):
        oracle.dispatch_moe_ffn([1, 2], [0, 1], [I2, I2[:3]], [I2, I2], [I2, I2], 1, 2, 2)
    with pytest.raises(oracle.OracleError,
                       match=r"^MoE expert weight lists must be non-empty and aligned$"):
        oracle.dispatch_moe_ffn([1, 2], [0, 1], [], [], [], 1, 2, 2)
    # an un-routed expert may be empty; longer weights are accepted
    out = oracle.dispatch_moe_ffn([1, 2], [0, 1], [None, np.r_[I2, 9]], [None, I2], [None, I2],
                                  1, 2, 2)
    assert np.all(np.isfinite(out))
    # all logits non-finite: one empty route list -> zero output, no error
    out = oracle.dispatch_moe_ffn([1, 2], [np.nan, np.inf], [I2, I2], [I2, I2], [I2, I2], 2, 2, 2)
    assert out.tolist() == [0.0, 0.0]
    with pytest.raises(oracle.OracleError, match=r"^Matvec input shape mismatch: got 3, expected 2$"):
        oracle.matvec(I2, 2, 2, [1, 2, 3])


def test_identity_experts_give_silu_x_times_x(oracle):
    rng = np.random.default_rng(11)
    H = 64
    x = rng.standard_normal(H).astype(np.float32)
    I = _identity(H, H)
    out = oracle.dispatch_moe_ffn(x, [5.0, 0.0], [I, I], [I, I], [I, I], 1, H, H)
    xd = x.astype(np.float64)
    np.testing.assert_allclose(out, xd / (1 + np.exp(-xd)) * xd, rtol=2e-7, atol=1e-30)


def test_matvec_is_sequential_unfused(oracle):
    rng = np.random.default_rng(12)
    w = rng.standard_normal(3 * 257).astype(np.float32)
    x = rng.standard_normal(257).astype(np.float32)
    y = oracle.matvec(w, 3, 257, x)
    for r in range(3):
        s = np.float32(0.0)
        for c in range(257):
            s = np.float32(s + np.float32(w[r * 257 + c] * x[c]))
        assert y[r] == s


def make_layer(seed, T, H, F, E, scale=0.02):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    gate = [(rng.standard_normal(F * H) * scale).astype(np.float32) for _ in range(E)]
    up = [(rng.standard_normal(F * H) * scale).astype(np.float32) for _ in range(E)]
    down = [(rng.standard_normal(H * F) * scale).astype(np.float32) for _ in range(E)]
    rw = (rng.standard_normal((E, H)) * scale).astype(np.float32)
    logits = (x.astype(np.float64) @ rw.T.astype(np.float64)).astype(np.float32)
    return x, logits, gate, up, down


def np_layer64(x, logits, gate, up, down, k, score_mode=0, shared=None):
    T, H = x.shape
    E = logits.shape[1]
    out = np.zeros((T, H))
    for t in range(T):
        row = [(e, float(logits[t, e])) for e in range(E) if np.isfinite(logits[t, e])]
        row = sorted(row, key=lambda ev: -_total_key(ev[1]))[:min(k, E)]
        if score_mode == 0:
            m = row[0][1]
            p = np.array([math.exp(v - m) for _, v in row])
        else:
            p = np.array([1 / (1 + math.exp(-v)) for _, v in row])
        p /= p.sum()
        xt = x[t].astype(np.float64)
        experts = [(gate[e], up[e], down[e], pw) for (e, _), pw in zip(row, p)]
        if shared is not None:
            experts.append((*shared, 1.0))
        for g, u, d, pw in experts:
            Fe = g.size // H
            gv = g.reshape(Fe, H).astype(np.float64) @ xt
            uv = u.reshape(Fe, H).astype(np.float64) @ xt
            a = gv / (1 + np.exp(-gv)) * uv
            out[t] += pw * (d.reshape(H, Fe).astype(np.float64) @ a)
    return out


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def test_layer_matches_float64_statement(oracle):
    x, lg, g, u, d = make_layer(21, 16, 128, 256, 8)
    got = oracle.moe_layer(x, lg, g, u, d, 2)
    assert rel_l2(got, np_layer64(x, lg, g, u, d, 2)) < 1e-5
    # row t of the batched layer == dispatch_moe_ffn on row t, bit for bit
    for t in (0, 7, 15):
        one = oracle.dispatch_moe_ffn(x[t], lg[t], g, u, d, 2, 128, 256)
        assert np.array_equal(one, got[t])


def test_layer_sigmoid_and_shared_expert(oracle):
    x, lg, g, u, d = make_layer(22, 8, 64, 96, 16)
    rng = np.random.default_rng(23)
    shared = [(rng.standard_normal(64 * 80) * 0.02).astype(np.float32) for _ in range(3)]
    got = oracle.moe_layer(x, lg, g, u, d, 4, score_mode=1, shared=shared)
    assert rel_l2(got, np_layer64(x, lg, g, u, d, 4, 1, shared)) < 1e-5


def test_layer_linear_in_down_weights(oracle):
    x, lg, g, u, d = make_layer(24, 6, 64, 128, 4)
    a = oracle.moe_layer(x, lg, g, u, d, 2)
    b = oracle.moe_layer(x, lg, g, u, [m * np.float32(2.0) for m in d], 2)
    assert np.array_equal(b, a * np.float32(2.0))  # power-of-two scaling is exact


def test_thread_count_does_not_change_layer(oracle):
    x, lg, g, u, d = make_layer(25, 12, 64, 64, 4)
    assert np.array_equal(oracle.moe_layer(x, lg, g, u, d, 2, nthreads=1),
                          oracle.moe_layer(x, lg, g, u, d, 2, nthreads=5))


# ----------------------------------------------------------------------------- baselines
def test_swiglu_ffn_reference_case(oracle):
    """src/kernel/mod.rs:336-348 input, value fixed in float64: (w1.x)*silu(w3.x) then w2."""
    H, F = 2, 4
    w1 = np.arange(F * H) * 0.1
    w3 = np.arange(F * H) * 0.05
    w2 = np.arange(H * F) * 0.02
    got = oracle.swiglu_ffn([1.0, 2.0], w1, w3, w2, H, F)
    x = np.array([1.0, 2.0])
    g = w1.reshape(F, H) @ x
    u = w3.reshape(F, H) @ x
    ref = w2.reshape(H, F) @ (g * (u / (1 + np.exp(-u))))
    assert got.shape == (2,)
    np.testing.assert_allclose(got, ref, rtol=1e-6)


def test_swiglu_with_swapped_operands_equals_dispatch(oracle):
    """kernel::swiglu_ffn(w1=up, w3=gate) equals one routed expert bit for bit."""
    x, lg, g, u, d = make_layer(26, 1, 64, 128, 1)
    out = oracle.dispatch_moe_ffn(x[0], [1.0], g, u, d, 1, 64, 128)
    sw = oracle.swiglu_ffn(x[0], u[0], g[0], d[0], 64, 128)
    assert np.array_equal(out, sw)


def test_cpu_matmul_known_answer(oracle):
    """src/backend/cpu.rs:234-241."""
    assert oracle.cpu_matmul([1, 2, 3, 4], [5, 6, 7, 8], 2, 2, 2).tolist() == [19, 22, 43, 50]


# ----------------------------------------------------------------------------- rms_norm
def test_rms_norm_reference_case(oracle):
    # src/kernel/mod.rs:289-301
    out = oracle.rms_norm([1.0, 2.0, 3.0, 4.0], [1.0, 1.0, 1.0, 1.0], 1e-5)[0]
    scale = np.float32(1.0) / np.sqrt(np.float32(30.0) / np.float32(4.0))
    assert out.shape == (4,)
    assert np.all(np.abs(out - np.array([1, 2, 3, 4], np.float32) * scale) < 1e-5)


def test_rms_norm_closed_form(oracle):
    # x = 2: every square, partial sum and the mean are exact, rstd = 1/2
    H = 1000
    w = (np.arange(H, dtype=np.float32) - 300) / np.float32(7)
    out = oracle.rms_norm(np.full(H, 2.0, np.float32), w, 0.0)[0]
    np.testing.assert_array_equal(out, w)


def test_rms_norm_sequential_order(oracle):
    rng = np.random.default_rng(21)
    H = 4096
    x = (rng.standard_normal(H) * np.exp(rng.uniform(-6, 6, H))).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    eps = np.float32(1e-5)
    out = oracle.rms_norm(x, w, float(eps))[0]
    s = np.float32(0.0)
    for v in x:
        s = np.float32(s + np.float32(v * v))
    rstd = np.float32(1.0) / np.sqrt(np.float32(s / np.float32(H)) + eps)
    np.testing.assert_array_equal(out, (x * rstd) * w)
    # a pairwise float32 sum of the same squares rounds differently here
    assert np.float32((x * x).sum(dtype=np.float32)) != s
    ref64 = x.astype(np.float64) * w / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    assert np.max(np.abs(out - ref64) / (np.abs(ref64) + 1e-30)) < 1e-3
