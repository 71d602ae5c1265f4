"""GPU parity of the HIP path against the oracle, through the C ABI.

Bars: dequantized values, quantized bytes, router indices/counts and the
permutation bit-exact; router weights within 2 ulp (device exp vs glibc
expf); layer outputs within relative L2 1e-4 on the fp32-accumulate GEMV path.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import F32, Q4_0, Q4_K, Q8_0, Layer, assert_same_bits, rel_l2

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def say(*a):
    print(*a, flush=True)


# ----------------------------------------------------------------------------- quant
def crafted(fmt, nblocks, seed):
    from test_oracle_quant import crafted_blocks
    return crafted_blocks(fmt, nblocks, seed)


@pytest.mark.parametrize("fmt", [Q8_0, Q4_0, Q4_K])
def test_dequant_bit_exact_crafted(ctx, fmt):
    say(f"dequant crafted fmt={fmt}")
    blk = oracle.BLOCK[fmt][0]
    data = crafted(fmt, 512, seed=fmt + 1)
    n = 512 * blk - 3
    got = ctx.dequant(fmt, data, n)
    ref = oracle.dequantize(fmt, data, n)
    assert_same_bits(got, ref)


@pytest.mark.parametrize("fmt", [Q8_0, Q4_0, Q4_K])
def test_dequant_bit_exact_quantized_weights(ctx, fmt):
    rng = np.random.default_rng(fmt)
    w = (rng.standard_normal(4096 * 1024) * 0.02).astype(np.float32)
    q = oracle.quantize(fmt, w)
    say(f"dequant N(0,0.02) fmt={fmt} n={w.size}")
    got = ctx.dequant(fmt, q, w.size)
    assert_same_bits(got, oracle.dequantize(fmt, q, w.size))


def test_dequant_truncated_payload_error(ctx):
    with pytest.raises(nx.NexusError, match="^Q4_K tensor payload is truncated$") as e:
        ctx.dequant(Q4_K, np.zeros(143, np.uint8), 256)
    assert e.value.code == nx.NX_ERR_TRUNCATED
    # the Q8_0 known answer (src/gguf/mod.rs:1681-1695) on the device
    scale = np.array([0.5], np.float32).astype(np.float16).view(np.uint8)
    block = np.concatenate([scale, (np.arange(32) - 16).astype(np.int8).view(np.uint8)])
    v = ctx.dequant(Q8_0, block, 32)
    assert v[0] == -8.0 and v[16] == 0.0 and v[31] == 7.5


@pytest.mark.parametrize("fmt", [Q8_0, Q4_0, Q4_K])
def test_quantize_bit_exact(ctx, fmt):
    rng = np.random.default_rng(10 + fmt)
    parts = [
        (rng.standard_normal(256 * 2048) * 0.02).astype(np.float32),
        rng.standard_normal(256 * 512).astype(np.float32),
        (rng.standard_normal(256 * 64) * 1e-6).astype(np.float32),  # subnormal f16 scales
        np.arange(300, dtype=np.float32) / np.float32(31.0) - np.float32(4.0),
        np.zeros(256, np.float32),
        np.full(256, 3.0, np.float32),
        (rng.standard_normal(256 * 16) * 1e5).astype(np.float32),  # f16 overflow of scales
    ]
    for x in parts:
        x = np.concatenate([x, rng.standard_normal(77).astype(np.float32)])  # ragged tail
        say(f"quantize fmt={fmt} n={x.size}")
        assert np.array_equal(ctx.quantize(fmt, x), oracle.quantize(fmt, x))


# ----------------------------------------------------------------------------- router
def router_case(rng, T, E, special=0.0):
    lg = rng.standard_normal(T * E).astype(np.float32)
    if special:
        pool = np.array([0.0, -0.0, 1.0, np.nan, np.inf, -np.inf, 0.5, -1.0], np.float32)
        m = rng.random(T * E) < special
        lg[m] = pool[rng.integers(0, pool.size, m.sum())]
    return lg


@pytest.mark.parametrize("T,E,k,special", [(1, 8, 2, 0), (64, 8, 2, 0.3), (512, 128, 8, 0),
                                           (33, 128, 8, 0.5), (4096, 256, 8, 0),
                                           (7, 256, 8, 0.9), (5, 1000, 16, 0.2),
                                           (9, 3, 7, 0.4), (16, 64, 64, 0.1)])
@pytest.mark.parametrize("score", [0, 1])
def test_router_matches_reference_order(ctx, T, E, k, special, score):
    rng = np.random.default_rng(T * 1000 + E + k)
    lg = router_case(rng, T, E, special)
    say(f"router T={T} E={E} k={k} special={special} score={score}")
    ex, w, cnt, n = ctx.route_topk(lg, T, E, k, score)
    rex, rw, rcnt, rn = oracle.route(lg, T, E, k, score)
    assert n == rn
    assert np.array_equal(cnt, rcnt)
    assert np.array_equal(ex, rex)
    # weights: exp() on the device is not glibc's expf; a 1-ulp difference in
    # one exp also moves the sum, so each normalised weight is within 2 ulp
    ulp = np.abs(w.view(np.int32).astype(np.int64) - rw.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2, f"max ulp {ulp.max()}"
    assert np.count_nonzero(ulp) <= max(2, 0.02 * ulp.size)


def test_router_reference_case_and_short_logits(ctx):
    ex, w, cnt, n = ctx.route_topk([0.1, 3.0, 1.0, 2.0, 0.5, 0.2], 2, 3, 2)
    assert n == 2 and ex[0].tolist() == [1, 2] and abs(float(w[0].sum()) - 1) < 1e-6
    ex, w, cnt, n = ctx.route_topk([0.1, 3.0, 1.0, 2.0, 0.5], 2, 3, 2)  # second row cut short
    assert n == 1 and cnt.tolist() == [2, 0] and ex[1].tolist() == [-1, -1]
    assert ctx.route_topk([1.0, 2.0], 1, 2, 0)[3] == 0


# one workgroup (up to 4096 pairs; few experts over at most two of its
# chunks), then one workgroup per chunk of 64 to 1024 tokens (at most 64
# chunks: partial last chunks, chunks of 64, 128 and 512 tokens, 8 to 1000
# experts)
@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (32, 8, 2), (64, 16, 4), (65, 16, 4), (2048, 8, 2),
                                   (512, 128, 8), (4096, 256, 8), (3000, 1000, 5), (100, 3, 3),
                                   (4000, 8, 2), (8192, 64, 6), (20000, 128, 8)])
def test_permutation_bit_exact(ctx, T, E, k):
    rng = np.random.default_rng(T + E)
    lg = router_case(rng, T, E, 0.05)
    ex, w, cnt, _ = oracle.route(lg, T, E, k)
    say(f"permute T={T} E={E} k={k}")
    got = ctx.permute(ex, cnt, E)
    ref = oracle.permute(ex, cnt, E)
    for g, r in zip(got, ref):
        assert np.array_equal(g, r)


def test_permutation_rejects_bad_routes(ctx):
    with pytest.raises(nx.NexusError):
        ctx.permute(np.array([[0, 0]], np.int32), np.array([2], np.int32), 4)
    with pytest.raises(nx.NexusError):
        ctx.permute(np.array([[0, 9]], np.int32), np.array([2], np.int32), 4)


# ----------------------------------------------------------------------------- layer
def run_layer(ctx, L, path=nx.PATH_GEMV):
    ex = L.upload(nx, ctx)
    try:
        return ex.forward(L.x, L.logits, L.k, L.score_mode, path)
    finally:
        ex.close()


@pytest.mark.parametrize("fmt,E,H,F,k,T", [
    (F32, 8, 512, 1024, 2, 16),    # tiny F32 layer
    (Q4_K, 8, 512, 1024, 2, 16),
    (Q8_0, 8, 512, 1024, 2, 16),
    (Q4_0, 8, 512, 1024, 2, 16),
    (Q4_K, 8, 1024, 768, 2, 1),
    (Q4_K, 16, 256, 256, 4, 37),
    (Q8_0, 128, 256, 768, 8, 9),
    (F32, 4, 36, 20, 3, 5),        # row lengths that are not multiples of 4
])
def test_layer_gemv_parity(ctx, fmt, E, H, F, k, T):
    L = Layer(fmt, E, H, F, k, T, seed=E * 7 + H + F + T)
    say(f"layer gemv fmt={fmt} E={E} H={H} F={F} k={k} T={T}")
    err = rel_l2(run_layer(ctx, L), L.oracle_out())
    assert err <= GEMV_TOL, err


def test_layer_sigmoid_and_shared_expert(ctx):
    L = Layer(Q4_K, 32, 512, 512, 8, 6, seed=3, shared_F=512, score_mode=1)
    say("layer sigmoid + shared expert")
    assert rel_l2(run_layer(ctx, L), L.oracle_out()) <= GEMV_TOL


def test_reference_dispatch_case(ctx):
    """src/engine/mod.rs:1632-1656 on the device: [0.18395..] x 2."""
    ex = nx.Experts(ctx, F32, 2, 2, 2)
    eye = np.eye(2, dtype=np.float32).ravel()
    for e, (g, u, d) in enumerate([(eye, eye, eye), (np.full(4, 0.5), np.full(4, 0.25),
                                                      np.full(4, 0.1))]):
        for role, m in enumerate((g, u, d)):
            ex.load(e, role, np.asarray(m, np.float32))
    out = ex.forward(np.array([[1.0, 2.0]]), np.array([[0.0, 4.0]]), 1)
    ref = oracle.dispatch_moe_ffn([1.0, 2.0], [0.0, 4.0], [eye, np.full(4, 0.5)],
                                  [eye, np.full(4, 0.25)], [eye, np.full(4, 0.1)], 1, 2, 2)
    np.testing.assert_allclose(out[0], ref, rtol=1e-6)
    # all-non-finite logits: the token has no routes and its output is zero
    out = ex.forward(np.array([[1.0, 2.0]]), np.array([[np.nan, np.inf]]), 2)
    assert out.tolist() == [[0.0, 0.0]]
    with pytest.raises(nx.NexusError, match="^MoE router produced no routes$"):
        ex.forward(np.array([[1.0, 2.0]]), np.array([[0.0, 4.0]]), 0)
    ex.close()


def test_run_to_run_bit_identical(ctx):
    L = Layer(Q4_K, 8, 512, 1024, 2, 24, seed=99)
    ex = L.upload(nx, ctx)
    a = ex.forward(L.x, L.logits, 2, path=nx.PATH_GEMV)
    b = ex.forward(L.x, L.logits, 2, path=nx.PATH_GEMV)
    ex.close()
    assert np.array_equal(a, b)


@pytest.mark.slow
def test_mixtral_decode_full_size(ctx):
    """Mixtral-shaped Q4_K layer at its real size, batch 1 (only the two routed
    experts need f32 copies for the oracle)."""
    L = Layer(Q4_K, 8, 4096, 14336, 2, 1, seed=2024)
    say("mixtral Q4_K T=1 full size")
    err = rel_l2(run_layer(ctx, L), L.oracle_out())
    say(f"  rel L2 = {err:.2e}")
    assert err <= GEMV_TOL


# ----------------------------------------------------------------------------- MFMA path
MFMA_TOL = 1e-2


@pytest.mark.parametrize("path", [nx.PATH_MFMA_F16, nx.PATH_MFMA_BF16])
@pytest.mark.parametrize("fmt,E,H,F,k,T,zipf", [
    (Q8_0, 8, 512, 1024, 2, 300, 1.2),   # Zipf-imbalanced expert popularity
    (Q4_K, 8, 512, 768, 2, 200, None),
    (Q4_0, 8, 256, 512, 2, 130, None),
    (F32, 8, 512, 1024, 2, 64, None),
    (Q4_K, 32, 256, 512, 4, 77, None),
    (Q8_0, 4, 256, 320, 1, 129, None),   # F not a multiple of the 128-row tile
    # a hundred or more pairs per expert: several M-tiles per expert, full
    # and partial, with Zipf-skewed counts and rows not a multiple of 128
    (Q8_0, 4, 512, 640, 2, 700, 1.2),
    (Q4_K, 4, 512, 768, 2, 600, None),
    (Q4_0, 2, 256, 320, 1, 400, None),
    # about 100-160 pairs per expert: 160-pair M-tiles (Q8_0: down only),
    # some experts past 160 with Zipf-skewed counts
    (Q8_0, 4, 512, 512, 2, 250, None),
    (Q4_K, 8, 256, 512, 2, 560, 1.1),
    (Q4_0, 4, 256, 256, 2, 260, None),
    # at most 48 pairs per expert: 64-pair M-tiles, with the Zipf-popular
    # experts spread over several of them (full and partial)
    (Q8_0, 16, 512, 640, 2, 300, 1.2),
    (Q4_0, 16, 256, 320, 2, 200, 1.1),
    (Q4_K, 16, 512, 768, 4, 150, None),
    # Q4_K widths 256 past a multiple of 512: the down pass's last window
    # holds one block and runs as 4 steps in element order (the only window;
    # after two full ones; on 160-pair tiles; after eight, with the K split
    # in two so that only the second split has it)
    (Q4_K, 8, 256, 256, 2, 200, None),
    (Q4_K, 4, 256, 1280, 2, 300, None),
    (Q4_K, 4, 256, 768, 2, 560, None),
    (Q4_K, 8, 512, 7424, 2, 64, None),
    # output rows the bf16 per-pair rows cannot take in pairs (odd H: f32
    # rows) or in fours (H % 4 == 2: bf16 rows through the scalar combine)
    (F32, 4, 37, 24, 2, 70, None),
    (F32, 4, 38, 24, 2, 70, None),
])
def test_layer_mfma_parity(ctx, path, fmt, E, H, F, k, T, zipf):
    L = Layer(fmt, E, H, F, k, T, seed=3 * E + H + F + T, zipf=zipf)
    say(f"layer mfma path={path} fmt={fmt} E={E} H={H} F={F} k={k} T={T} zipf={zipf}")
    err = rel_l2(run_layer(ctx, L, path), L.oracle_out())
    say(f"  rel L2 = {err:.2e}")
    assert err <= MFMA_TOL, err


def _layer_sweep(n=12, seed=4242):
    """Seeded random layers: F32, Q8_0, Q4_0 and Q4_K experts at widths in
    whole blocks (F32 also odd widths), 2 to 48 experts, top-1 to top-8, 1 to
    200 tokens, with and without a shared expert (of its own width), both
    score modes."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        fmt = (F32, Q8_0, Q4_0, Q4_K)[i % 4]
        blk = {F32: 1, Q8_0: 32, Q4_0: 32, Q4_K: 256}[fmt]
        unit = 256 if fmt == Q4_K else 32
        H = int(rng.integers(1, 768 // unit + 1)) * unit
        F = int(rng.integers(1, 768 // unit + 1)) * unit
        if fmt == F32 and i % 8 == 0:
            H, F = H + 3, F + 5  # rows not a multiple of 4 floats
        E = int(rng.integers(2, 49))
        k = int(rng.integers(1, min(8, E) + 1))
        T = int(rng.integers(1, 201))
        Fs = int(rng.integers(1, 768 // unit + 1)) * unit if rng.random() < 0.3 else 0
        assert H % blk == 0 and F % blk == 0
        out.append((fmt, E, H, F, k, T, Fs, int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _layer_sweep(), ids=lambda c: "-".join(map(str, c)))
def test_layer_random_shapes(ctx, case):
    """GEMV (1e-4), bf16 grouped GEMM (1e-2) and AUTO (1e-2: any of its
    paths) against the oracle's dispatch on the same random layer."""
    fmt, E, H, F, k, T, Fs, score = case
    say(f"layer sweep fmt={fmt} E={E} H={H} F={F} k={k} T={T} Fs={Fs} score={score}")
    L = Layer(fmt, E, H, F, k, T, seed=E + H + F + T + fmt, shared_F=Fs, score_mode=score)
    ref = L.oracle_out()
    ex = L.upload(nx, ctx)
    try:
        for path, tol in ((nx.PATH_GEMV, GEMV_TOL), (nx.PATH_MFMA_BF16, MFMA_TOL),
                          (nx.PATH_AUTO, MFMA_TOL)):
            got = ex.forward(L.x, L.logits, k, score, path)
            err = rel_l2(got, ref)
            say(f"  path {path}: rel L2 = {err:.2e}")
            assert err <= tol, (path, err)
    finally:
        ex.close()


@pytest.mark.parametrize("path", [nx.PATH_MFMA_F16, nx.PATH_MFMA_BF16])
@pytest.mark.parametrize("F,Fs", [(512, 768), (768, 512), (768, 256)])
def test_layer_mfma_half_window_shared(ctx, path, F, Fs):
    """Q4_K routed and shared experts of different widths, one or both 256
    past a multiple of 512 (the down pass's half window per expert kind)."""
    L = Layer(Q4_K, 8, 256, F, 2, 150, seed=F + Fs, shared_F=Fs, score_mode=1)
    say(f"layer mfma half window path={path} F={F} Fs={Fs}")
    err = rel_l2(run_layer(ctx, L, path), L.oracle_out())
    say(f"  rel L2 = {err:.2e}")
    assert err <= MFMA_TOL, err


def test_layer_mfma_shared_expert_sigmoid(ctx):
    # 24 pairs per routed expert: 64-pair M-tiles, the shared expert's 96
    # tokens over two of them
    L = Layer(Q4_K, 16, 512, 512, 4, 96, seed=5, shared_F=512, score_mode=1)
    say("layer mfma shared + sigmoid")
    assert rel_l2(run_layer(ctx, L, nx.PATH_MFMA_F16), L.oracle_out()) <= MFMA_TOL
    # the shared expert's 300 tokens over two 160-pair M-tiles (150 pairs
    # per routed expert), the last partial
    L = Layer(Q4_K, 4, 512, 512, 2, 300, seed=6, shared_F=512, score_mode=1)
    say("layer mfma shared + sigmoid, many pairs per expert")
    assert rel_l2(run_layer(ctx, L, nx.PATH_MFMA_BF16), L.oracle_out()) <= MFMA_TOL


@pytest.mark.parametrize("fmt", [Q8_0, Q4_K])
def test_auto_mfma_keeps_float_range(ctx, fmt):
    """Activations near 1e3 give SwiGLU outputs near 1e5, past fp16's 65504:
    the grouped GEMM that AUTO picks (bf16 operands) stays within the MFMA
    bar of the oracle."""
    L = Layer(fmt, 8, 512, 512, 2, 256, seed=31)
    L.x = (L.x * np.float32(1000.0)).astype(np.float32)
    ref = L.oracle_out()
    act_max = 0.0
    for e in L.routed[:2]:
        g = L.dense[(e, 0)].reshape(512, 512) @ L.x[0].astype(np.float64)
        u = L.dense[(e, 1)].reshape(512, 512) @ L.x[0].astype(np.float64)
        with np.errstate(over="ignore"):  # exp(-g) for g << 0: silu -> -0
            act_max = max(act_max, float(np.max(np.abs(g / (1 + np.exp(-g)) * u))))
    say(f"auto mfma range fmt={fmt}: max |act| of token 0 = {act_max:.3g}")
    assert act_max > 65504.0  # the inputs do leave fp16's range
    ex = L.upload(nx, ctx)
    ctx.profile(True)
    ctx.profile_reset()
    out = ex.forward(L.x, L.logits, L.k, path=nx.PATH_AUTO)
    stats = ctx.profile_stats()
    ctx.profile(False)
    ex.close()
    assert "gemm_gateup" in stats
    assert np.isfinite(out).all()
    assert rel_l2(out, ref) <= MFMA_TOL


def test_auto_path_picks_mfma_for_prefill(ctx):
    L = Layer(Q8_0, 8, 512, 512, 2, 256, seed=8)
    ex = L.upload(nx, ctx)
    ctx.profile(True)
    ctx.profile_reset()
    out = ex.forward(L.x, L.logits, L.k, path=nx.PATH_AUTO)
    stats = ctx.profile_stats()
    ctx.profile(False)
    ex.close()
    assert "gemm_gateup" in stats and "gemm_down" in stats
    assert rel_l2(out, L.oracle_out()) <= MFMA_TOL
