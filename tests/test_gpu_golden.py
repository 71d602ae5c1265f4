"""The HIP path against the committed golden fixtures (tests/golden/).

Device dequantization of the crafted blocks and the device quantizer on the
full-size seeded expert 0 of every model configuration are bit-exact (their
SHA-256 equals the oracle's).  Router logits (exact mode), routes and the
permutation are bit-exact.  Layer outputs are within relative L2 1e-4 of the
fixtures: the tiny configuration's full [16 x 512] output, and for every
model configuration one token through its routed experts quantized on the
device (64 sampled output values).
"""
import json
import os

import numpy as np
import pytest

import nexus_amd as nx
from golden.make_golden import CONFIGS, SHARED, sha, shapes, tokens, weight

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.mark.parametrize("fmt,blk", [(8, 32), (2, 32), (12, 256)])
def test_crafted_blocks(ctx, fmt, blk):
    g = load("crafted_blocks.npz")
    got = ctx.dequant(fmt, g[f"payload_{fmt}"], 64 * blk)
    np.testing.assert_array_equal(got.view(np.uint32), g[f"deq_{fmt}"].view(np.uint32))


@pytest.mark.parametrize("path", [nx.PATH_GEMV, nx.PATH_AUTO])
def test_tiny_config(ctx, path):
    g = load("tiny_f32.npz")
    E, H, F, k, T = 8, 512, 1024, 2, 16
    x, router, _ = tokens(0, T, H, E)
    logits = ctx.router_logits(router, x, E, H, exact=True)
    np.testing.assert_array_equal(logits.view(np.uint32), g["logits"].view(np.uint32))
    ex_ids, w, cnt, _ = ctx.route_topk(logits, T, E, k)
    np.testing.assert_array_equal(ex_ids, g["experts"])
    np.testing.assert_array_equal(cnt, g["counts"])
    ec, off, pt, ps, inv = ctx.permute(ex_ids, cnt, E)
    for a, b in ((ec, "expert_counts"), (off, "offsets"), (pt, "perm_token"), (ps, "perm_slot"),
                 (inv, "inv_pos")):
        np.testing.assert_array_equal(a, g[b])
    ex = nx.Experts(ctx, nx.F32, E, H, F)
    for e in range(E):
        for r, shp in enumerate(shapes(H, F)):
            ex.load(e, r, weight(0, e, r, *shp))
    out = ex.forward(x, logits, k, path=path)
    ref = g["out"].astype(np.float64)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) <= 1e-4
    ex.close()


@pytest.mark.parametrize("cfg", [c for c in CONFIGS], ids=[c[1] for c in CONFIGS])
def test_config_quantizer_routes_and_token0(ctx, cfg):
    cid, name, fmt, E, H, F, k, Fs, score, T, zipf = cfg
    print(f"golden config {name}", flush=True)
    g = json.load(open(os.path.join(GOLD, "configs.json")))[name]
    x, router, _ = tokens(cid, T, H, E, zipf)
    logits = ctx.router_logits(router, x, E, H, exact=True)
    if zipf is not None:
        p = 1.0 / np.arange(1, E + 1) ** zipf
        logits = (logits + np.log(p / p.sum()).astype(np.float32)[None, :]).astype(np.float32)
    ex_ids, w, cnt, _ = ctx.route_topk(logits, T, E, k, score_mode=score)
    assert sha(ex_ids, w, cnt) == g["routes_sha256"]
    routed = [int(e) for e in ex_ids[0, :cnt[0]]]
    assert routed == g["token0_routed"]
    ex = nx.Experts(ctx, fmt, E, H, F, shared_ff_dim=Fs)
    for e in sorted(set(routed) | {0}):
        for r, shp in enumerate(shapes(H, F)):
            q = ctx.quantize(fmt, weight(cid, e, r, *shp))
            if e == 0:
                assert sha(q) == g["expert0_quant_sha256"][r]
            ex.load(e, r, q)
    if Fs:
        for r, shp in enumerate(shapes(H, Fs)):
            q = ctx.quantize(fmt, weight(cid, SHARED, r, *shp))
            assert sha(q) == g["shared_quant_sha256"][r]
            ex.load(nx.EXPERT_SHARED, r, q)
    y = ex.forward(x[:1], logits[:1], k, score_mode=score, path=nx.PATH_GEMV)[0]
    idx = np.array(g["token0_sample_index"])
    ref = np.array(g["token0_sample"])
    assert np.linalg.norm(y[idx] - ref) <= 1e-4 * np.linalg.norm(ref)
    assert abs(np.linalg.norm(y.astype(np.float64)) - g["token0_l2"]) <= 1e-4 * g["token0_l2"]
    ex.close()
