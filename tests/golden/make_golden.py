"""Writes the golden fixtures under tests/golden/ from the oracle.

    python tests/golden/make_golden.py [crafted|tiny|configs|fullshape ...]

Fixtures (inputs and expected outputs only):
  crafted_blocks.npz  64 crafted GGUF blocks per format (special f16 scales,
                      every 6-bit Q4_K scale/min) and their dequantized values.
  tiny_f32.npz        the tiny configuration (H=512, F=1024, E=8, k=2, F32
                      experts, T=16): inputs, routes, permutation and the full
                      [16 x 512] output, plus SHA-256 of the seeded weights.
  configs.json        per model configuration: SHA-256 of expert 0's quantized
                      matrices (and the shared expert's), SHA-256 of the
                      routes of the seeded tokens, and sampled output rows at
                      one token.
  fullshape.npz       the parity workloads at full size (Mixtral Q4_K 32
                      tokens, Qwen3 Q4_K 64 and 512 tokens, Mixtral Q8_0 2048
                      tokens with the Zipf(1.2) router, DeepSeek Q4_K 4096
                      tokens with sigmoid scores and the shared expert,
                      Mixtral-shaped Q4_0 at 1 and 256 tokens): the
                      SHA-256 of the exact router logits and of every token's
                      routed experts, the per-expert pair counts, and the
                      oracle's output rows for a set of tokens that together
                      route to every expert the workload routes to.

Weights and activations come from numpy's PCG64 generator with seeds derived
from (configuration id, expert, role); regenerating them is part of each test.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402

F32, Q4_0, Q8_0, Q4_K = 0, 2, 8, 12
SHARED = 10**4  # expert index of the shared expert in seeds

# id, name, fmt, E, H, F, k, shared F, score mode, tokens, zipf
CONFIGS = [
    (1, "mixtral_q4k", Q4_K, 8, 4096, 14336, 2, 0, 0, 32, None),
    (2, "qwen3_q4k", Q4_K, 128, 2048, 768, 8, 0, 0, 64, None),
    (3, "mixtral_q8_0_prefill", Q8_0, 8, 4096, 14336, 2, 0, 0, 64, 1.2),
    (4, "deepseek_q4k_sigmoid_shared", Q4_K, 256, 7168, 2048, 8, 2048, 1, 32, None),
]


def weight(cfg_id, expert, role, rows, cols):
    rng = np.random.default_rng([cfg_id, expert, role])
    return rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)


def tokens(cfg_id, T, H, E, zipf=None):
    rng = np.random.default_rng([cfg_id, 7])
    x = rng.standard_normal((T, H), dtype=np.float32)
    router = rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)
    logits = np.stack([oracle.matvec(router.ravel(), E, H, x[t]) for t in range(T)])
    if zipf is not None:
        p = 1.0 / np.arange(1, E + 1) ** zipf
        logits = (logits + np.log(p / p.sum()).astype(np.float32)[None, :]).astype(np.float32)
    return x, router, logits


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def shapes(H, F):
    return ((F, H), (F, H), (H, F))


def crafted():
    sys.path.insert(0, os.path.join(os.path.dirname(HERE)))
    from test_oracle_quant import crafted_blocks
    out = {}
    for fmt, blk in ((Q8_0, 32), (Q4_0, 32), (Q4_K, 256)):
        data = crafted_blocks(fmt, 64, seed=100 + fmt)
        out[f"payload_{fmt}"] = data
        out[f"deq_{fmt}"] = oracle.dequantize(fmt, data, 64 * blk)
    np.savez(os.path.join(HERE, "crafted_blocks.npz"), **out)


def tiny():
    cid, E, H, F, k, T = 0, 8, 512, 1024, 2, 16
    x, router, logits = tokens(cid, T, H, E)
    mats = {(e, r): weight(cid, e, r, *shp).ravel()
            for e in range(E) for r, shp in enumerate(shapes(H, F))}
    ex, w, cnt, lists = oracle.route(logits, T, E, k)
    ec, off, pt, ps, inv = oracle.permute(ex, cnt, E)
    out = oracle.moe_layer(x, logits, [mats[(e, 0)] for e in range(E)],
                           [mats[(e, 1)] for e in range(E)], [mats[(e, 2)] for e in range(E)], k)
    np.savez(os.path.join(HERE, "tiny_f32.npz"), x=x, router=router, logits=logits, experts=ex,
             weights=w, counts=cnt, expert_counts=ec, offsets=off, perm_token=pt, perm_slot=ps,
             inv_pos=inv, out=out.astype(np.float32),
             weights_sha256=np.array(sha(*[mats[(e, r)] for e in range(E) for r in range(3)])))


def configs():
    res = {}
    for cid, name, fmt, E, H, F, k, Fs, score, T, zipf in CONFIGS:
        print("config", name, flush=True)
        x, router, logits = tokens(cid, T, H, E, zipf)
        ex, w, cnt, _ = oracle.route(logits, T, E, k, score)
        q0 = [oracle.quantize(fmt, weight(cid, 0, r, *shp)) for r, shp in enumerate(shapes(H, F))]
        entry = {"id": cid, "fmt": fmt, "experts": E, "hidden": H, "ffn": F, "top_k": k,
                 "shared_ffn": Fs, "score_mode": score, "tokens": T, "zipf": zipf,
                 "expert0_quant_sha256": [sha(q) for q in q0],
                 "routes_sha256": sha(ex, w, cnt), "router_sha256": sha(router),
                 "x_sha256": sha(x)}
        if Fs:
            qs = [oracle.quantize(fmt, weight(cid, SHARED, r, *shp))
                  for r, shp in enumerate(shapes(H, Fs))]
            entry["shared_quant_sha256"] = [sha(q) for q in qs]
        # one token through the layer: dequantized routed experts (+ shared)
        routed = [int(e) for e in ex[0, :cnt[0]]]
        g, u, d = [None] * E, [None] * E, [None] * E
        for e in routed:
            qe = q0 if e == 0 else [oracle.quantize(fmt, weight(cid, e, r, *shp))
                                    for r, shp in enumerate(shapes(H, F))]
            g[e], u[e], d[e] = (oracle.dequantize(fmt, qe[r], shapes(H, F)[r][0] * shapes(H, F)[r][1])
                                for r in range(3))
        shared = None
        if Fs:
            shared = [oracle.dequantize(fmt, qs[r], Fs * H) for r in range(3)]
        y = oracle.moe_layer(x[:1], logits[:1], g, u, d, k, score, shared=shared)[0]
        idx = np.linspace(0, H - 1, 64).astype(np.int64)
        entry["token0_routed"] = routed
        entry["token0_sample_index"] = idx.tolist()
        entry["token0_sample"] = [float(v) for v in y[idx]]
        entry["token0_l2"] = float(np.linalg.norm(y.astype(np.float64)))
        res[name] = entry
    with open(os.path.join(HERE, "configs.json"), "w") as f:
        json.dump(res, f, indent=1)


# Full-size parity workloads: name, seed id, tokens, fmt, E, H, F, k, shared F,
# score mode, zipf.  Shapes, formats, routing, activations and the expert
# weights' distribution (N(0, 0.02), drawn by weight() above, then quantized)
# are the model configurations'.  The Q4_0 workloads (a format no
# configuration names) take the Mixtral shape.
FULLSHAPE = [
    ("mixtral_q4k_t32", 101, 32, Q4_K, 8, 4096, 14336, 2, 0, 0, None),
    ("qwen3_q4k_t64", 102, 64, Q4_K, 128, 2048, 768, 8, 0, 0, None),
    ("qwen3_q4k_t512", 102, 512, Q4_K, 128, 2048, 768, 8, 0, 0, None),
    ("mixtral_q8_0_prefill_t2048", 103, 2048, Q8_0, 8, 4096, 14336, 2, 0, 0, 1.2),
    ("deepseek_q4k_sigmoid_shared_t4096", 104, 4096, Q4_K, 256, 7168, 2048, 8, 2048, 1, None),
    ("mixtral_q4_0_t1", 105, 1, Q4_0, 8, 4096, 14336, 2, 0, 0, None),
    ("mixtral_q4_0_t256", 105, 256, Q4_0, 8, 4096, 14336, 2, 0, 0, None),
]


def workload_inputs(seed_id, T, H, E):
    """Activations ~N(0,1) [T x H] and router weight ~N(0,0.02) [E x H], from
    separate streams, so the first tokens do not depend on T."""
    x = np.random.default_rng([seed_id, 7]).standard_normal((T, H), dtype=np.float32)
    router = (np.random.default_rng([seed_id, 8]).standard_normal((E, H), dtype=np.float32)
              * np.float32(0.02))
    return x, router


def zipf_bias(logits, E, zipf):
    """logit_e += ln p_e with p_e proportional to (e+1)^-zipf, in f32."""
    if zipf is None:
        return logits
    p = 1.0 / np.arange(1, E + 1) ** zipf
    return (logits + np.log(p / p.sum()).astype(np.float32)[None, :]).astype(np.float32)


def covering_tokens(ex, cnt, E, minimum=8):
    """Tokens that together route to every routed expert: greedy set cover
    (most uncovered experts first, lower token first), then evenly spaced
    tokens up to `minimum`, always including the first and last token."""
    T = ex.shape[0]
    routed = [set(int(e) for e in ex[t, :cnt[t]]) for t in range(T)]
    todo = set().union(*routed)
    chosen = []
    while todo:
        best = max(range(T), key=lambda t: (len(routed[t] & todo), -t))
        chosen.append(best)
        todo -= routed[best]
    for t in np.linspace(0, T - 1, minimum).astype(int):
        if len(chosen) >= minimum and t not in (0, T - 1):
            continue
        if int(t) not in chosen:
            chosen.append(int(t))
    return np.array(sorted(chosen), np.int32)


def fullshape(only=None):
    from concurrent.futures import ThreadPoolExecutor
    path = os.path.join(HERE, "fullshape.npz")
    out = dict(np.load(path, allow_pickle=False)) if os.path.exists(path) else {}
    pool = ThreadPoolExecutor(8)
    for name, sid, T, fmt, E, H, F, k, Fs, score, zipf in FULLSHAPE:
        if only and name not in only:
            continue
        print("fullshape", name, flush=True)
        x, router = workload_inputs(sid, T, H, E)
        logits = np.stack(list(pool.map(lambda t: oracle.matvec(router, E, H, x[t]), range(T))))
        logits = zipf_bias(logits, E, zipf)
        ex, w, cnt, _ = oracle.route(logits, T, E, k, score)
        sel = covering_tokens(ex, cnt, E)
        need = sorted({int(e) for t in sel for e in ex[t, :cnt[t]]})
        print(f"  {len(sel)} tokens, {len(need)} experts", flush=True)

        def quant(job):
            e, r, rows, cols = job
            return (e, r), oracle.quantize(fmt, weight(sid, e, r, rows, cols), nthreads=1)

        jobs = [(e, r, *shp) for e in need for r, shp in enumerate(shapes(H, F))]
        if Fs:
            jobs += [(SHARED, r, *shp) for r, shp in enumerate(shapes(H, Fs))]
        payload = dict(pool.map(quant, jobs))
        shared = None
        if Fs:
            shared = [oracle.dequantize(fmt, payload[(SHARED, r)], int(np.prod(shp)))
                      for r, shp in enumerate(shapes(H, Fs))]

        def row(t):
            mats = [[None] * E for _ in range(3)]
            for e in ex[t, :cnt[t]]:
                for r, shp in enumerate(shapes(H, F)):
                    mats[r][int(e)] = oracle.dequantize(fmt, payload[(int(e), r)],
                                                        int(np.prod(shp)), nthreads=1)
            return oracle.moe_layer(x[t:t + 1], logits[t:t + 1], mats[0], mats[1], mats[2], k,
                                    score, shared=shared, nthreads=1)[0]

        rows = np.stack(list(ThreadPoolExecutor(4).map(row, sel)))
        out[f"{name}/logits_sha256"] = np.array(sha(logits))
        out[f"{name}/routes_sha256"] = np.array(sha(ex, cnt))
        out[f"{name}/expert_counts"] = np.bincount(ex[ex >= 0], minlength=E).astype(np.int32)
        out[f"{name}/tokens"] = sel
        out[f"{name}/route_weights"] = w[sel]
        out[f"{name}/rows"] = rows.astype(np.float32)
        del payload
    np.savez(path, **out)


if __name__ == "__main__":
    what = sys.argv[1:] or ["crafted", "tiny", "configs", "fullshape"]
    if "crafted" in what:
        crafted()
    if "tiny" in what:
        tiny()
    if "configs" in what:
        configs()
    if "fullshape" in what:
        names = [a for a in what if a not in ("crafted", "tiny", "configs", "fullshape")]
        fullshape(names or None)
