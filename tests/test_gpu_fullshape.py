"""The HIP path at the full size of every model workload, through the C ABI.

Each workload of tests/golden/make_golden.py's FULLSHAPE list (Mixtral Q4_K at
32 tokens, Qwen3 Q4_K at 64 and 512 tokens, Mixtral Q8_0 at 2048 tokens with
the Zipf(1.2) router, DeepSeek Q4_K at 4096 tokens with sigmoid scores and the
shared expert, Q4_0 at the Mixtral shape at 1 and 256 tokens), its expert
weights drawn from N(0, 0.02) as the configurations name them, is built on
the device at its real shape, with every expert of
the configuration resident, and run at its full token count on the path the
dispatcher picks (NX_PATH_AUTO) and on each explicit path.  Against the
oracle's fixtures (tests/golden/fullshape.npz):

  * the exact router logits of all tokens: SHA-256 equal (bit-exact);
  * every token's routed experts and counts: SHA-256 equal (bit-exact), the
    per-expert pair counts equal, the route weights of the sampled tokens
    within 2 ulp (the device's exp is not glibc's expf);
  * the output rows of the sampled tokens (which together route to every
    expert the workload uses, the least popular included): relative L2 over
    the rows <= 1e-4 on the fp32-accumulate paths (GEMV, split-activation
    MFMA) and <= 1e-2 on the fp16/bf16 grouped GEMM, and every single row
    within 10x that bar.

Row t of the batch equals InferenceEngine::dispatch_moe_ffn on row t
(src/engine/mod.rs:969-1024).
"""
import collections
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import nexus_amd as nx
from golden.make_golden import FULLSHAPE, SHARED, sha, shapes, weight, workload_inputs, zipf_bias
from moe_cases import DeviceArray, rel_l2

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fullshape.npz")
TOL = {"gemv": 1e-4, "split": 1e-4, "mfma": 1e-2}
PATH_NAMES = {nx.PATH_GEMV: "gemv", nx.PATH_MFMA_SPLIT: "split", nx.PATH_MFMA_F16: "mfma",
              nx.PATH_MFMA_BF16: "mfma"}
# explicit paths run besides AUTO, per workload
PATHS = {
    "mixtral_q4k_t32": [nx.PATH_GEMV, nx.PATH_MFMA_SPLIT, nx.PATH_MFMA_F16],
    "qwen3_q4k_t64": [nx.PATH_GEMV, nx.PATH_MFMA_SPLIT],
    "qwen3_q4k_t512": [nx.PATH_MFMA_SPLIT, nx.PATH_MFMA_F16, nx.PATH_MFMA_BF16],
    "mixtral_q8_0_prefill_t2048": [nx.PATH_GEMV, nx.PATH_MFMA_F16, nx.PATH_MFMA_BF16],
    "deepseek_q4k_sigmoid_shared_t4096": [nx.PATH_GEMV, nx.PATH_MFMA_SPLIT, nx.PATH_MFMA_F16,
                                          nx.PATH_MFMA_BF16],
    "mixtral_q4_0_t1": [nx.PATH_GEMV],
    "mixtral_q4_0_t256": [nx.PATH_MFMA_SPLIT, nx.PATH_MFMA_BF16],
}


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def build_experts(ctx, sid, fmt, E, H, F, Fs):
    """Every expert of the workload, drawn on the host (8 threads, a bounded
    window ahead), quantized on the device and loaded from device memory."""
    ex = nx.Experts(ctx, fmt, E, H, F, shared_ff_dim=Fs)
    members = [(e, e, F) for e in range(E)] + ([(nx.EXPERT_SHARED, SHARED, Fs)] if Fs else [])
    jobs = [(dst, seed_e, r, shp) for dst, seed_e, f in members
            for r, shp in enumerate(shapes(H, f))]
    nmax = max(r * c for _, _, _, (r, c) in jobs)
    src = DeviceArray(nmax)
    q = DeviceArray(nx.quant_bytes(fmt, nmax) // 4 + 1)
    with ThreadPoolExecutor(8) as pool:
        it = iter(jobs)
        window = collections.deque()

        def refill():
            while len(window) < 16:
                j = next(it, None)
                if j is None:
                    return
                window.append((j, pool.submit(weight, sid, j[1], j[2], *j[3])))

        refill()
        while window:
            (dst, _, role, (r, c)), fut = window.popleft()
            refill()
            w = fut.result()
            src.upload(w)
            nb = nx.quant_bytes(fmt, r * c)
            ctx.quantize_dev(fmt, src.ptr, r * c, q.ptr, nb)
            ex.load_dev(dst, role, q.ptr, nb)
            ctx.sync()  # src and q are reused by the next matrix
    return ex


def path_taken(stats):
    names = set(stats)
    if any(n.startswith("gemm_") for n in names):
        return "mfma"
    if any(n.startswith("mfv_") for n in names):
        return "split"
    assert any(n.startswith("gemv_") for n in names), names
    return "gemv"


@pytest.mark.parametrize("wl", FULLSHAPE, ids=[w[0] for w in FULLSHAPE])
def test_full_size_workload(ctx, gold, wl):
    name, sid, T, fmt, E, H, F, k, Fs, score, zipf = wl
    say(f"fullshape {name}: T={T} E={E} H={H} F={F} k={k} shared={Fs} fmt={fmt}")
    x, router = workload_inputs(sid, T, H, E)
    logits = zipf_bias(ctx.router_logits(router, x, E, H, exact=True), E, zipf)
    assert sha(logits) == str(gold[f"{name}/logits_sha256"])
    ex = build_experts(ctx, sid, fmt, E, H, F, Fs)
    say(f"  experts resident: {ex.device_bytes() / 1e9:.2f} GB")
    sel = gold[f"{name}/tokens"]
    ref = gold[f"{name}/rows"].astype(np.float64)
    for path in [nx.PATH_AUTO] + PATHS[name]:
        ctx.profile(True)
        ctx.profile_reset()
        out = ex.forward(x, logits, k, score_mode=score, path=path)
        taken = path_taken(ctx.profile_stats())
        ctx.profile(False)
        if path != nx.PATH_AUTO:
            assert taken == PATH_NAMES[path]
        tol = TOL[taken]
        # routes of every token, bit-exact
        rex, rw, rcnt = ctx.last_routes(T, k)
        assert sha(rex, rcnt) == str(gold[f"{name}/routes_sha256"])
        np.testing.assert_array_equal(np.bincount(rex[rex >= 0], minlength=E),
                                      gold[f"{name}/expert_counts"])
        gw = gold[f"{name}/route_weights"]
        ulp = np.abs(rw[sel].view(np.int32).astype(np.int64) - gw.view(np.int32).astype(np.int64))
        assert ulp.max() <= 2
        got = out[sel].astype(np.float64)
        err = rel_l2(got, ref)
        worst = max(rel_l2(got[i], ref[i]) for i in range(len(sel)))
        say(f"  path {path} ({taken}): rel L2 {err:.3e} over {len(sel)} rows, worst row {worst:.3e}")
        assert np.isfinite(out).all()
        assert err <= tol
        assert worst <= 10 * tol
    ex.close()
