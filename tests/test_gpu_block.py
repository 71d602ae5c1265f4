"""RMSNorm (nx_rms_norm) and the MoE block (nx_moe_block) against the oracle.

Bars: exact-mode RMSNorm bit-identical to the oracle's kernel::rms_norm
(src/kernel/mod.rs:199-209) on every row, including zero rows, overflowing
squares, subnormal squares and non-finite inputs; fast mode within
(H + 8) 2^-24 of the exact output, relatively.  The block
hidden + MoE(rms_norm(hidden)) with on-device router logits: its normed
input and logits are the reference's bit for bit in exact mode, so routing is
identical, and its FFN part (output minus the residual) is within the GEMV
path's relative L2 1e-4 of the oracle's dispatch_moe_ffn over the same
quantized experts.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import F32, Q4_K, Q8_0, DeviceArray, Layer, assert_same_bits, rel_l2

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


# rows of whole float4 up to 4096 and up to 7168 (one wave per token, four
# tokens per workgroup: partial workgroups, partial last runs), then rows the
# two-launch chain path takes (not whole float4, or longer than 7168)
@pytest.mark.parametrize("T,H", [(1, 4096), (3, 7168), (33, 2048), (5, 5120), (2, 4100),
                                 (6, 4), (1, 1056), (2, 1001), (4, 5), (9, 64), (2, 7200)])
def test_rms_norm_exact_bit_identical(ctx, T, H):
    rng = np.random.default_rng(T * 1000 + H)
    x = (rng.standard_normal((T, H)) * np.exp(rng.uniform(-3, 3, (T, 1)))).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    got = ctx.rms_norm(x, w, 1e-5, exact=True)
    assert_same_bits(got, oracle.rms_norm(x, w, 1e-5))


def test_rms_norm_dev_unaligned_and_reused(ctx):
    # rows offset by one float: not 16-byte aligned, so the chain path runs;
    # then the aligned copies, on the same buffers
    T, H = 3, 2048
    rng = np.random.default_rng(31)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    ref = oracle.rms_norm(x, w, 1e-5)
    dx, dw, do = DeviceArray(T * H + 4), DeviceArray(H + 4), DeviceArray(T * H + 4, fill=np.nan)
    for off in (1, 0, 1):
        dx.upload(x, off)
        dw.upload(w, off)
        ctx.rms_norm_dev(dx.ptr + 4 * off, T * H, dw.ptr + 4 * off, H, 1e-5, T, H,
                         do.ptr + 4 * off, exact=True)
        ctx.sync()
        o = do.download()
        assert_same_bits(o[off:off + T * H].reshape(T, H), ref)


def test_rms_norm_special_rows(ctx):
    H = 256
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, H)).astype(np.float32)
    x[0] = 0.0                   # sum 0: rstd = 1/sqrt(eps)
    x[1, 7] = 3e20               # square overflows: inf sum, zero output
    x[2] = 1e-25                 # subnormal squares
    x[3, 9] = np.nan
    x[4, 11] = np.inf
    x[5] = -0.0
    w = rng.standard_normal(H).astype(np.float32)
    for eps in (1e-5, 1e-6, 0.0):
        got = ctx.rms_norm(x, w, eps, exact=True)
        assert_same_bits(got, oracle.rms_norm(x, w, eps))


@pytest.mark.parametrize("T,H", [(1, 4096), (17, 7168), (5, 1001)])
def test_rms_norm_fast_within_bound(ctx, T, H):
    rng = np.random.default_rng(T + H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    fast = ctx.rms_norm(x, w, 1e-5, exact=False).astype(np.float64)
    exact = oracle.rms_norm(x, w, 1e-5).astype(np.float64)
    assert np.all(np.abs(fast - exact) <= (H + 8) * U * np.abs(exact) + 1e-37)


def test_rms_norm_errors(ctx):
    x = np.ones((2, 8), np.float32)
    with pytest.raises(nx.NexusError, match=r"^RMSNorm weight too small: got 7, expected at least 8$"):
        ctx.rms_norm(x, np.ones(7, np.float32), 1e-5)
    # a longer weight is accepted, only the first H entries are read
    got = ctx.rms_norm(x, np.r_[np.ones(8, np.float32), np.float32(np.nan)], 1e-5)
    assert_same_bits(got, oracle.rms_norm(x, np.ones(8, np.float32), 1e-5))


def block_case(fmt, E, H, F, k, T, seed, shared_F=0):
    L = Layer(fmt, E, H, F, k, T, seed=seed, shared_F=shared_F, experts_needed=range(E))
    rng = np.random.default_rng(seed + 1)
    hidden = (rng.standard_normal((T, H)) * 0.7).astype(np.float32)
    norm_w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    router = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    return L, hidden, norm_w, router


def oracle_block(L, hidden, norm_w, eps, router):
    T, H = hidden.shape
    normed = oracle.rms_norm(hidden, norm_w, eps)
    logits = np.stack([oracle.matvec(router.ravel(), L.E, H, normed[t]) for t in range(T)])
    g = [L.dense[(e, 0)] for e in range(L.E)]
    u = [L.dense[(e, 1)] for e in range(L.E)]
    d = [L.dense[(e, 2)] for e in range(L.E)]
    ffn = oracle.moe_layer(normed, logits, g, u, d, L.k, L.score_mode, shared=L.shared_dense)
    return normed, logits, ffn


@pytest.mark.parametrize("fmt,E,H,F,k,T,shared", [
    (Q4_K, 8, 1024, 1536, 2, 1, 0), (Q4_K, 8, 1024, 1536, 2, 7, 0),
    (Q8_0, 16, 512, 768, 4, 40, 512)])
def test_moe_block_exact(ctx, fmt, E, H, F, k, T, shared):
    print(f"moe block fmt={fmt} E={E} H={H} F={F} k={k} T={T} shared={shared}", flush=True)
    L, hidden, norm_w, router = block_case(fmt, E, H, F, k, T, seed=E + H + T, shared_F=shared)
    eps = 1e-5
    normed, logits, ffn = oracle_block(L, hidden, norm_w, eps, router)
    assert_same_bits(ctx.rms_norm(hidden, norm_w, eps), normed)
    assert_same_bits(ctx.router_logits(router, normed, E, H, exact=True), logits)
    ex = L.upload(nx, ctx)
    got = ex.block(hidden, norm_w, eps, router, k, path=nx.PATH_GEMV, exact=True)
    assert rel_l2(got.astype(np.float64) - hidden, ffn) <= 1e-4
    # the residual add rounds hidden + ffn once per element
    want = (hidden + ex.forward(normed, logits, k, path=nx.PATH_GEMV)).astype(np.float32)
    assert_same_bits(got, want)
    ex.close()


@pytest.mark.parametrize("fmt,E,H,F,k,T", [
    (Q4_K, 8, 4096, 256, 2, 1),    # Mixtral's width, one expert group: 32 runs of 128 columns
    (Q8_0, 20, 2048, 128, 4, 5),   # three expert groups, the last partial
    (Q8_0, 128, 1024, 64, 8, 2),   # sixteen groups per token
    (Q8_0, 12, 1056, 64, 2, 3),    # a partial last run
    (Q8_0, 8, 4128, 64, 2, 3),     # just past 4096: chains on 64 lanes, runs of 112 columns
    (Q4_K, 12, 7168, 256, 2, 2),   # DeepSeek's width: 64 full runs, three expert groups
    (Q8_0, 8, 7200, 64, 2, 2),     # wider than the one launch holds: three launches
    (Q8_0, 8, 10240, 64, 2, 2),
    (Q8_0, 8, 512, 64, 2, 64)])    # the most tokens the single launch takes
def test_moe_block_exact_prologue(ctx, fmt, E, H, F, k, T):
    """The exact block's prologue (one launch: the sum-of-squares chain, the
    normalised row, the router chains) gives the oracle's normalised rows and
    logits: the block output equals hidden + the layer on them, bit for bit."""
    print(f"block prologue fmt={fmt} E={E} H={H} F={F} k={k} T={T}", flush=True)
    L, hidden, norm_w, router = block_case(fmt, E, H, F, k, T, seed=3 * E + H + T)
    eps = 1e-6
    normed, logits, ffn = oracle_block(L, hidden, norm_w, eps, router)
    ex = L.upload(nx, ctx)
    ctx.profile(True)
    ctx.profile_reset()
    got = ex.block(hidden, norm_w, eps, router, k, path=nx.PATH_GEMV, exact=True)
    ran = set(ctx.profile_stats())
    ctx.profile(False)
    fused = H % 4 == 0 and H <= 7168
    assert ("block_prologue" in ran) == fused, ran
    assert ("rms_sumsq_chain8" in ran) == (not fused), ran
    want = (hidden + ex.forward(normed, logits, k, path=nx.PATH_GEMV)).astype(np.float32)
    assert_same_bits(got, want)
    assert rel_l2(got.astype(np.float64) - hidden, ffn) <= 1e-4
    ex.close()


@pytest.mark.parametrize("H", [1536, 4096, 5120, 7168])  # chains of 32 and 64 lanes
def test_moe_block_exact_prologue_special_rows(ctx, H):
    """Rows that stress the prologue's sum of squares: dyadic values (squares
    that land exactly halfway between representable sums), magnitudes across
    the exponent range (the running sum changes binade many times), tiny
    values (subnormal squares), zeros, and a square near the top of the
    float range (the sum overflows to inf, rstd becomes 0).  Normalised rows
    and logits must stay the oracle's, so the block output is bit-identical
    to hidden + the layer on the oracle's normalised rows."""
    E, F, k = 8, 128, 2
    T = 6
    print(f"block prologue special rows H={H}", flush=True)
    L, hidden, norm_w, router = block_case(Q8_0, E, H, F, k, T, seed=97)
    rng = np.random.default_rng(98)
    hidden[1] = rng.integers(-12, 13, H).astype(np.float32) / 8
    hidden[2] = (rng.standard_normal(H) * 10.0 ** rng.integers(-12, 12, H)).astype(np.float32)
    hidden[3] = (rng.standard_normal(H) * 1e-23).astype(np.float32)
    hidden[4] = 0.0
    hidden[5, :] = rng.standard_normal(H).astype(np.float32)
    hidden[5, 100] = np.float32(3e19)
    eps = 1e-6
    normed, logits, _ = oracle_block(L, hidden, norm_w, eps, router)
    assert np.all(np.isfinite(normed)) and np.all(np.isfinite(logits))
    ex = L.upload(nx, ctx)
    got = ex.block(hidden, norm_w, eps, router, k, path=nx.PATH_GEMV, exact=True)
    want = (hidden + ex.forward(normed, logits, k, path=nx.PATH_GEMV)).astype(np.float32)
    assert_same_bits(got, want)
    ex.close()


# the residual added by the combine over each kind of per-pair rows: f32
# (fp16 GEMM), bf16 in eight-column runs without and with K splits (the
# down pass split in two at F = 4096), bf16 in four-column runs (H % 8 == 4)
@pytest.mark.parametrize("path,H,F", [(nx.PATH_MFMA_F16, 512, 512), (nx.PATH_MFMA_BF16, 512, 512),
                                      (nx.PATH_MFMA_BF16, 512, 4096), (nx.PATH_MFMA_BF16, 516, 512)])
def test_moe_block_mfma_residual(ctx, path, H, F):
    E, k, T = 8, 2, 192
    fmt = Q8_0 if H % 32 == 0 else F32
    print(f"moe block mfma residual path={path} fmt={fmt} H={H} F={F}", flush=True)
    L, hidden, norm_w, router = block_case(fmt, E, H, F, k, T, seed=31, shared_F=512)
    eps = 1e-5
    normed, logits, ffn = oracle_block(L, hidden, norm_w, eps, router)
    ex = L.upload(nx, ctx)
    got = ex.block(hidden, norm_w, eps, router, k, path=path, exact=True)
    want = (hidden + ex.forward(normed, logits, k, path=path)).astype(np.float32)
    assert_same_bits(got, want)
    assert rel_l2(got.astype(np.float64) - hidden, ffn) <= 1e-2
    ex.close()


def test_moe_block_dev_repeated_and_fast(ctx):
    from moe_cases import DeviceArray
    E, H, F, k, T = 8, 1024, 1024, 2, 3
    L, hidden, norm_w, router = block_case(Q4_K, E, H, F, k, T, seed=77)
    ex = L.upload(nx, ctx)
    want = ex.block(hidden, norm_w, 1e-5, router, k, path=nx.PATH_GEMV, exact=True)
    dh, dn, dr = DeviceArray(T * H), DeviceArray(H), DeviceArray(E * H)
    dn.upload(norm_w)
    dr.upload(router)
    for _ in range(2):
        dh.upload(hidden)
        ex.block_dev(dh.ptr, dn.ptr, H, 1e-5, dr.ptr, E * H, T, k, path=nx.PATH_GEMV, exact=True)
        ctx.sync()
        assert_same_bits(dh.download().reshape(T, H), want)
    fast = ex.block(hidden, norm_w, 1e-5, router, k, path=nx.PATH_GEMV, exact=False)
    _, logits, ffn = oracle_block(L, hidden, norm_w, 1e-5, router)
    srt = np.sort(logits, axis=1)
    clear = (srt[:, -k] - srt[:, -k - 1]) > 1e-3  # tokens whose routing has a margin
    assert clear.any()
    assert rel_l2((fast.astype(np.float64) - hidden)[clear], ffn[clear]) <= 1e-4
    ex.close()


def test_moe_block_errors(ctx):
    E, H, F, k, T = 4, 256, 256, 2, 2
    L, hidden, norm_w, router = block_case(Q8_0, E, H, F, k, T, seed=5)
    ex = L.upload(nx, ctx)
    with pytest.raises(nx.NexusError, match=r"^Matvec weight too small: got 1023, expected at least 1024$"):
        ex.block(hidden, norm_w, 1e-5, router.ravel()[:1023], k)
    with pytest.raises(nx.NexusError, match=r"^RMSNorm weight too small"):
        ex.block(hidden, norm_w[:100], 1e-5, router, k)
    with pytest.raises(nx.NexusError, match=r"^MoE router produced no routes$"):
        ex.block(hidden, norm_w, 1e-5, router, 0)
    ex.close()


def test_experts_outlive_context():
    """An expert set destroyed after its context (a set kept alive past the
    context's close, e.g. by a failing test's traceback) frees cleanly."""
    c2 = nx.Context(0)
    ex = nx.Experts(c2, Q8_0, 4, 256, 256)
    c2.close()
    ex.close()
