"""The oracle against the committed golden fixtures (tests/golden/).

The fixtures hold inputs and expected outputs written by
tests/golden/make_golden.py: crafted GGUF blocks and their values, the tiny
F32 configuration end to end, and per model configuration the SHA-256 of
the seeded expert 0 quantized with the reference's quantizer and of the
routes.  A change in the oracle, in the seeded generator's stream or in the
recipe shows up here first.  The GPU side checks the same fixtures in
tests/test_gpu_golden.py.
"""
import json
import os

import numpy as np
import pytest

import oracle
from golden.make_golden import CONFIGS, SHARED, sha, shapes, tokens, weight

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.mark.parametrize("fmt,blk", [(8, 32), (2, 32), (12, 256)])
def test_crafted_blocks(fmt, blk):
    g = load("crafted_blocks.npz")
    got = oracle.dequantize(fmt, g[f"payload_{fmt}"], 64 * blk)
    np.testing.assert_array_equal(got.view(np.uint32), g[f"deq_{fmt}"].view(np.uint32))


def test_tiny_config_end_to_end():
    g = load("tiny_f32.npz")
    E, H, F, k, T = 8, 512, 1024, 2, 16
    x, router, logits = tokens(0, T, H, E)
    np.testing.assert_array_equal(x, g["x"])
    np.testing.assert_array_equal(logits.view(np.uint32), g["logits"].view(np.uint32))
    mats = {(e, r): weight(0, e, r, *shp).ravel()
            for e in range(E) for r, shp in enumerate(shapes(H, F))}
    assert sha(*[mats[(e, r)] for e in range(E) for r in range(3)]) == str(g["weights_sha256"])
    ex, w, cnt, _ = oracle.route(logits, T, E, k)
    np.testing.assert_array_equal(ex, g["experts"])
    np.testing.assert_array_equal(w.view(np.uint32), g["weights"].view(np.uint32))
    np.testing.assert_array_equal(cnt, g["counts"])
    ec, off, pt, ps, inv = oracle.permute(ex, cnt, E)
    for a, b in ((ec, "expert_counts"), (off, "offsets"), (pt, "perm_token"), (ps, "perm_slot"),
                 (inv, "inv_pos")):
        np.testing.assert_array_equal(a, g[b])
    out = oracle.moe_layer(x, logits, [mats[(e, 0)] for e in range(E)],
                           [mats[(e, 1)] for e in range(E)], [mats[(e, 2)] for e in range(E)], k)
    np.testing.assert_array_equal(out.astype(np.float32).view(np.uint32), g["out"].view(np.uint32))


@pytest.mark.parametrize("cfg", [c for c in CONFIGS], ids=[c[1] for c in CONFIGS])
def test_config_routes(cfg):
    cid, name, fmt, E, H, F, k, Fs, score, T, zipf = cfg
    g = json.load(open(os.path.join(GOLD, "configs.json")))[name]
    x, router, logits = tokens(cid, T, H, E, zipf)
    assert sha(x) == g["x_sha256"] and sha(router) == g["router_sha256"]
    ex, w, cnt, _ = oracle.route(logits, T, E, k, score)
    assert sha(ex, w, cnt) == g["routes_sha256"]


@pytest.mark.parametrize("name", ["qwen3_q4k", "deepseek_q4k_sigmoid_shared"])
def test_config_expert0_quantized(name):
    cfg = next(c for c in CONFIGS if c[1] == name)
    cid, _, fmt, E, H, F, k, Fs, score, T, zipf = cfg
    g = json.load(open(os.path.join(GOLD, "configs.json")))[name]
    for r, shp in enumerate(shapes(H, F)):
        assert sha(oracle.quantize(fmt, weight(cid, 0, r, *shp))) == g["expert0_quant_sha256"][r]
    if Fs:
        for r, shp in enumerate(shapes(H, Fs)):
            assert sha(oracle.quantize(fmt, weight(cid, SHARED, r, *shp))) == \
                g["shared_quant_sha256"][r]
