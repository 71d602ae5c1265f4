"""nx_moe_forward_noalloc (the entry point that allocates nothing) against
nx_moe_forward_dev, through the C ABI.

Both run the same kernels; the no-allocation call takes every intermediate
from the library's static scratch array instead of context workspace.  The
outputs must be bit-identical on two calls in a row, the second with fewer
tokens (so stale scratch contents from the first call are present), on every
path the dispatcher has: the one-token GEMV with the router inside the gate/up
kernel, the decode-batch GEMV, the split-activation MFMA path (Q4_K, Q4_0,
Q8_0, Q2_K) and the grouped GEMM, with and without a shared expert.  Calls whose intermediates do not fit
the array fail with NX_ERR_UNSUPPORTED and leave the output untouched.
"""
import numpy as np
import pytest

import nexus_amd as nx
from moe_cases import Q2_K, Q4_0, Q4_K, Q8_0, DeviceArray, Layer, assert_same_bits

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def run_pair(ex, layer, T, path, score, fn):
    x = DeviceArray(T * layer.H)
    x.upload(layer.x[:T])
    lg = DeviceArray(T * layer.E)
    lg.upload(layer.logits[:T])
    out = DeviceArray(T * layer.H, fill=np.nan)
    fn(x.ptr, lg.ptr, T, layer.k, out.ptr, score_mode=score, path=path)
    return out.download().reshape(T, layer.H)


CASES = [
    # fmt, E, H, F, k, shared F, score, path, (T first, T second)
    (Q4_K, 8, 1024, 2048, 2, 0, 0, nx.PATH_GEMV, (1, 1)),
    (Q4_K, 8, 1024, 2048, 2, 0, 0, nx.PATH_GEMV, (6, 2)),
    (Q4_K, 8, 1024, 2048, 2, 0, 0, nx.PATH_MFMA_SPLIT, (24, 5)),
    (Q8_0, 8, 512, 1024, 2, 0, 0, nx.PATH_MFMA_F16, (300, 77)),
    (Q4_K, 16, 512, 512, 4, 512, 1, nx.PATH_MFMA_BF16, (200, 33)),
    (Q4_K, 16, 512, 512, 4, 512, 1, nx.PATH_GEMV, (1, 1)),
    (Q8_0, 8, 512, 1024, 2, 0, 0, nx.PATH_AUTO, (40, 1)),
    (Q4_0, 8, 512, 1024, 2, 0, 0, nx.PATH_MFMA_SPLIT, (24, 5)),
    (Q8_0, 8, 512, 1024, 2, 0, 0, nx.PATH_MFMA_SPLIT, (24, 5)),
    (Q2_K, 8, 512, 1024, 2, 0, 0, nx.PATH_MFMA_SPLIT, (24, 5)),
    (Q2_K, 16, 512, 512, 4, 512, 1, nx.PATH_MFMA_SPLIT, (12, 4)),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[7]}-T{c[8]}" for c in CASES])
def test_noalloc_matches_forward_dev(ctx, case):
    fmt, E, H, F, k, Fs, score, path, (T1, T2) = case
    say(f"noalloc fmt={fmt} E={E} H={H} F={F} k={k} shared={Fs} path={path} T={T1},{T2}")
    layer = Layer(fmt, E, H, F, k, max(T1, T2), seed=E * 7 + H + T1, shared_F=Fs,
                  score_mode=score, experts_needed=[])
    ex = layer.upload(nx, ctx)
    for T in (T1, T2):
        got = run_pair(ex, layer, T, path, score, ex.forward_noalloc)
        routes_na = ctx.last_routes(T, k)
        ref = run_pair(ex, layer, T, path, score, ex.forward_dev)
        routes_dev = ctx.last_routes(T, k)
        assert np.isfinite(got).all()
        assert_same_bits(got, ref)
        for a, b in zip(routes_na, routes_dev):
            np.testing.assert_array_equal(a, b)
    ex.close()


def device_experts(ctx, fmt, E, H, F, seed):
    """Experts of the given shape built on the device: uniform weights (the
    distribution does not matter here), quantized by the library."""
    ex = nx.Experts(ctx, fmt, E, H, F)
    src = DeviceArray(H * F)
    q = DeviceArray(nx.quant_bytes(fmt, H * F) // 4 + 1)
    rng = np.random.default_rng(seed)
    for e in range(E):
        for role, (r, c) in ((nx.ROLE_GATE, (F, H)), (nx.ROLE_UP, (F, H)), (nx.ROLE_DOWN, (H, F))):
            src.upload((rng.random(r * c, dtype=np.float32) - np.float32(0.5)) * np.float32(0.07))
            nb = nx.quant_bytes(fmt, r * c)
            ctx.quantize_dev(fmt, src.ptr, r * c, q.ptr, nb)
            ex.load_dev(e, role, q.ptr, nb)
            ctx.sync()  # src and q are reused
    return ex


def test_noalloc_allocates_nothing_at_the_mixtral_shape(ctx):
    """On a fresh context (empty workspace), Mixtral-shaped Q4_K layers at 32
    and then 8 tokens on the GEMV and the split-activation path (about 48 MB of
    the 64 MiB array at 32 tokens): free device memory is the same before and
    after the calls, and the outputs equal nx_moe_forward_dev's, which runs
    afterwards."""
    E, H, F, k = 8, 4096, 14336, 2
    say(f"noalloc Mixtral shape E={E} H={H} F={F} k={k}, free memory")
    # load the library's kernels on the device first (a process's first
    # launch loads the code object), on another context
    warm = Layer(Q4_K, 8, 256, 512, 2, 2, seed=11, experts_needed=[])
    wex = warm.upload(nx, ctx)
    run_pair(wex, warm, 2, nx.PATH_GEMV, 0, wex.forward_noalloc)
    wex.close()
    fresh = nx.Context(0)
    try:
        ex = device_experts(fresh, Q4_K, E, H, F, seed=21)
        rng = np.random.default_rng(22)
        T = 32
        x = DeviceArray(T * H)
        x.upload(rng.standard_normal((T, H), dtype=np.float32))
        rw = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        lg = DeviceArray(T * E)
        xs = x.download().reshape(T, H)
        lg.upload((xs.astype(np.float64) @ rw.T.astype(np.float64)).astype(np.float32))
        cases = [(p, t) for p in (nx.PATH_GEMV, nx.PATH_MFMA_SPLIT) for t in (32, 8)]
        outs = {c: DeviceArray(T * H, fill=np.nan) for c in cases}
        fresh.sync()
        free0 = fresh.mem_info()[0]
        for (path, t), out in outs.items():
            ex.forward_noalloc(x.ptr, lg.ptr, t, k, out.ptr, path=path)
        fresh.sync()
        free1 = fresh.mem_info()[0]
        assert free1 == free0, f"free device memory changed by {free0 - free1} bytes"
        for (path, t), out in outs.items():
            ref = DeviceArray(T * H, fill=np.nan)
            ex.forward_dev(x.ptr, lg.ptr, t, k, ref.ptr, path=path)
            got = out.download().reshape(T, H)[:t]
            assert np.isfinite(got).all()
            assert_same_bits(got, ref.download().reshape(T, H)[:t])
        ex.close()
    finally:
        fresh.close()


def test_noalloc_rejects_calls_beyond_the_scratch(ctx):
    E, H, F, k, T = 8, 256, 512, 2, 40000
    say(f"noalloc oversize T={T}")
    layer = Layer(Q8_0, E, H, F, k, 4, seed=5, experts_needed=[])
    ex = layer.upload(nx, ctx)
    rng = np.random.default_rng(3)
    x = DeviceArray(T * H)
    x.upload(rng.standard_normal(T * H).astype(np.float32))
    lg = DeviceArray(T * E)
    lg.upload(rng.standard_normal(T * E).astype(np.float32))
    out = DeviceArray(T * H, fill=7.0)
    with pytest.raises(nx.NexusError, match="scratch array") as e:
        ex.forward_noalloc(x.ptr, lg.ptr, T, k, out.ptr, path=nx.PATH_MFMA_F16)
    assert e.value.code == nx.NX_ERR_UNSUPPORTED
    assert (out.download() == 7.0).all()
    # profiling creates events, which this entry point does not
    ctx.profile(True)
    try:
        with pytest.raises(nx.NexusError, match="profiling") as e:
            ex.forward_noalloc(x.ptr, lg.ptr, 1, k, out.ptr)
        assert e.value.code == nx.NX_ERR_INVALID_ARG
    finally:
        ctx.profile(False)
    # a call that fits still works after the rejected one
    small = run_pair(ex, layer, 4, nx.PATH_GEMV, 0, ex.forward_noalloc)
    ref = run_pair(ex, layer, 4, nx.PATH_GEMV, 0, ex.forward_dev)
    assert_same_bits(small, ref)
    ex.close()
