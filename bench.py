"""Benchmark: Mixtral-8x7B-shaped MoE layer (Q4_K experts) on one MI355X.

One step = one pass of the MoE layer (router -> permutation -> gate/up GEMV
with fused SwiGLU -> down GEMV -> combine) over one batch of synthetic tokens
whose activations, router logits and quantized experts are already resident
in HBM.  Weights ~N(0, 0.02) are quantized to Q4_K on the device by the
library's quantizer; activations ~N(0, 1); logits = x . W_r^T with
W_r ~N(0, 0.02).  Several replicas of the expert set (more than twice the
~256 MB Infinity Cache in the bytes a step touches) are rotated step by step
so the weight bytes come from HBM.

Extras in the same line (skipped with --no-extra): Mixtral decode at 32
tokens, Mixtral Q8_0 prefill at 2048 tokens (MFMA grouped GEMM), the Qwen3
(E=128, k=8) and DeepSeek (E=256, k=8, sigmoid, shared expert) shapes at
their decode and batch token counts, the router logits (exact and fast
mode) for the three shapes, and the whole MoE block of a Mixtral decode step
(RMSNorm, router logits, layer, residual add).

Prints one JSON line (rank 0, N=1).  `value` = tokens/s of the whole layer.
`roofline` is for the dominant kernel (the gate/up GEMV): algorithmic bytes
= quantized weight bytes of the experts the step activates, divided by the
kernel's mean duration from HIP events on the stream it runs on.
`cpu_baseline` times the CPU oracle (single-threaded restatement of
InferenceEngine::dispatch_moe_ffn, f32 weights dequantized beforehand) on a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/sec + effective HBM GB/s (Mixtral-shape Q4_K), 1 GPU"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
Q4K_BYTES_PER_WEIGHT = 144.0 / 256.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--tokens", type=int, default=1)
    p.add_argument("--replicas", type=int, default=4)
    p.add_argument("--path", default="gemv",
                   choices=["auto", "gemv", "mfma_f16", "mfma_bf16", "mfma_split"])
    p.add_argument("--cpu-tokens", type=int, default=16, help="tokens in the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the 32-token decode and 2048-token prefill measurements")
    p.add_argument("--prefill-steps", type=int, default=20)
    p.add_argument("--prefill-path", default="auto", choices=["auto", "mfma_f16", "mfma_bf16"])
    p.add_argument("--only", default=None,
                   help="run one workload alone and print its record (for profilers): "
                        "decode, prefill, block, router, dense, or a model shape "
                        "NAME[:T<tokens>] (qwen3_q4k, deepseek_q4k_sigmoid_shared, mixtral_q2k, "
                        "mixtral_q4_0, mixtral_q8_0)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="run one device-to-device copy of this size first (calibrates HBM "
                        "byte counters under rocprofv3 --pmc)")
    p.add_argument("--seed", type=int, default=0)
    return p.parse_args()


def make_expert_sets(nx, ctx, torch, fmt, E, H, F, replicas, seed, Fs=0):
    """Quantized expert sets generated on the device (N(0, 0.02) -> fmt); Fs > 0
    adds a shared expert of width Fs."""
    dev = torch.device("cuda", 0)
    sets = []
    qbuf = None
    for rep in range(replicas):
        ex = nx.Experts(ctx, fmt, E, H, F, shared_ff_dim=Fs)
        members = [(e, F) for e in range(E)] + ([(nx.EXPERT_SHARED, Fs)] if Fs else [])
        for e, f in members:
            for role, (r, c) in ((nx.ROLE_GATE, (f, H)), (nx.ROLE_UP, (f, H)), (nx.ROLE_DOWN, (H, f))):
                g = torch.Generator(device=dev)
                g.manual_seed(seed * 1000003 + rep * 10007 + e * 101 + role)
                w = torch.randn((r, c), generator=g, device=dev, dtype=torch.float32) * 0.02
                nb = nx.quant_bytes(fmt, r * c)
                if qbuf is None or qbuf.numel() < nb:
                    qbuf = torch.empty(nb, dtype=torch.uint8, device=dev)
                ctx.quantize_dev(fmt, w.data_ptr(), r * c, qbuf.data_ptr(), nb)
                ex.load_dev(e, role, qbuf.data_ptr(), nb)
                del w
        sets.append(ex)
    torch.cuda.synchronize()
    return sets


def cpu_baseline(nx, ctx, torch, x, logits, E, H, F, k, seed, ntok):
    """Single-threaded oracle dispatch_moe_ffn on `ntok` tokens (f32 weights
    dequantized from the same Q4_K payloads outside the timed region)."""
    import numpy as np

    import oracle

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 77)
    xs = torch.randn((ntok, H), generator=gen, device=dev, dtype=torch.float32)
    rw = logits["router"]
    lg = (xs @ rw.t()).contiguous()
    xs_h, lg_h = xs.cpu().numpy(), lg.cpu().numpy()
    ex_ids, _, cnt, _ = oracle.route(lg_h, ntok, E, k)
    need = sorted({int(e) for t in range(ntok) for e in ex_ids[t, :cnt[t]]})
    mats = {0: [None] * E, 1: [None] * E, 2: [None] * E}
    for e in need:
        for role, (r, c) in ((0, (F, H)), (1, (F, H)), (2, (H, F))):
            g = torch.Generator(device=dev)
            g.manual_seed(seed * 1000003 + 0 * 10007 + e * 101 + role)  # replica 0
            w = torch.randn((r, c), generator=g, device=dev, dtype=torch.float32) * 0.02
            nb = nx.quant_bytes(nx.Q4_K, r * c)
            qb = torch.empty(nb, dtype=torch.uint8, device=dev)
            ctx.quantize_dev(nx.Q4_K, w.data_ptr(), r * c, qb.data_ptr(), nb)
            torch.cuda.synchronize()
            mats[role][e] = oracle.dequantize(oracle.Q4_K, qb.cpu().numpy(), r * c)
            del w, qb
    t0 = time.perf_counter()
    for t in range(ntok):
        oracle.dispatch_moe_ffn(xs_h[t], lg_h[t], mats[0], mats[1], mats[2], k, H, F)
    dt = time.perf_counter() - t0
    # the router matvec (InferenceEngine::matvec on W_r) for the same tokens
    rw_h = rw.cpu().numpy().ravel()
    t1 = time.perf_counter()
    for t in range(ntok):
        oracle.matvec(rw_h, E, H, xs_h[t])
    dtr = time.perf_counter() - t1
    # kernel::swiglu_ffn (the reference's CPU kernel path) per routed (token,
    # expert) on one core, and the whole batch row-parallel on every host core
    t2 = time.perf_counter()
    for t in range(ntok):
        for e in ex_ids[t, :cnt[t]]:
            e = int(e)
            oracle.swiglu_ffn(xs_h[t], mats[1][e], mats[0][e], mats[2][e], H, F)
    dts = time.perf_counter() - t2
    ncores = oracle.default_threads()  # the host CPU share for one GPU
    # one-token decode in CpuBackend::matmul's pattern (src/backend/cpu.rs:23-38):
    # each product of each routed expert as C[rows x 1] = W[rows x cols] . x,
    # its rows split over every core, token by token
    ex_w = oracle.route(lg_h, ntok, E, k)[1]
    t4 = time.perf_counter()
    for t in range(ntok):
        out = np.zeros(H, np.float32)
        for r in range(int(cnt[t])):
            e = int(ex_ids[t, r])
            gv = oracle.cpu_matmul(mats[0][e], xs_h[t], F, 1, H, nthreads=ncores)
            uv = oracle.cpu_matmul(mats[1][e], xs_h[t], F, 1, H, nthreads=ncores)
            act = (gv / (np.float32(1.0) + np.exp(-gv))) * uv
            yv = oracle.cpu_matmul(mats[2][e], act, H, 1, F, nthreads=ncores)
            out += np.float32(ex_w[t, r]) * yv
    dtd = time.perf_counter() - t4
    # the whole sample at once, its tokens spread over every core
    t3 = time.perf_counter()
    oracle.moe_layer(xs_h, lg_h, mats[0], mats[1], mats[2], k, nthreads=ncores)
    dtp = time.perf_counter() - t3
    return {"value": ntok / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "router_matvec_us_per_token": dtr / ntok * 1e6,
            "swiglu_ffn_1core_tokens_per_s": ntok / dts,
            "row_parallel_decode_tokens_per_s": ntok / dtd, "row_parallel_cores": ncores,
            "token_parallel_tokens_per_s": ntok / dtp, "token_parallel_cores": ncores,
            "host": host_info(),
            "sample": f"{ntok} tokens of the same Mixtral Q4_K layer through the oracle's "
                      f"single-threaded dispatch_moe_ffn (f32 weights dequantized from the "
                      f"Q4_K payloads outside the timed region), {dt:.1f} s; the row-parallel "
                      f"decode runs the same tokens one by one, {dtd:.2f} s"}


def host_info():
    """CPU model, logical CPUs and the oracle's compiler and flags."""
    import platform
    import subprocess

    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cflags = ""
    try:
        with open(os.path.join(ROOT, "oracle", "Makefile")) as f:
            for line in f:
                if line.startswith("CFLAGS"):
                    cflags = line.split("=", 1)[1].strip()
    except OSError:
        pass
    try:
        cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.split("\n")[0]
    except OSError:
        cc = "gcc"
    return {"cpu_model": model, "nproc": os.cpu_count(), "compiler": cc, "cflags": cflags}


# Secondary cases warm up for at least this long before their timed steps.
# Right after the host-side set-up between cases the GPU clock is still low,
# and MFMA/VALU-heavy steps (the split-activation path at 32 tokens) then run
# ~15% slower for the first few ms; back-to-back windows settle.
SETTLE_MS = 30.0


def time_steps(torch, fn, steps, warmup, settle_ms=0.0):
    """Mean wall ms per step over `steps` timed steps, after `warmup` untimed
    steps and, with settle_ms, further untimed steps until that much time has
    passed since the warm-up began."""
    t_w = time.perf_counter()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    i = warmup
    while (time.perf_counter() - t_w) * 1e3 < settle_ms:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def step_distribution(torch, fn, n=200):
    """Per-step device time over n steps (a HIP event pair around each, on
    the stream the steps run on): median, 10th and 90th percentile, in ms."""
    import numpy as np

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(ev):
        a.record()
        fn(i)
        b.record()
    torch.cuda.synchronize()
    ms = np.array([a.elapsed_time(b) for a, b in ev])
    return {"iterations": n, "median_ms": float(np.median(ms)), "p10_ms": float(np.percentile(ms, 10)),
            "p90_ms": float(np.percentile(ms, 90)), "mean_ms": float(ms.mean())}


def path_of(kern):
    """The expert-product path a step ran, from its kernel names."""
    if any(n.startswith("mfv") for n in kern):
        return "mfma_split"
    if any(n.startswith("gemm") for n in kern):
        return "mfma_bf16" if "to_bf16" in kern else "mfma_f16"
    return "gemv"


def kernel_means(ctx, torch, fn, steps):
    """Mean duration per kernel (HIP events on the launch stream) over `steps` steps."""
    ctx.profile(True)
    ctx.profile_reset()
    torch.cuda.synchronize()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    stats = ctx.profile_stats()
    ctx.profile(False)
    return {name: ms / max(n, 1) for name, (n, ms) in stats.items()}


def active_experts(ctx, logits_np, T, E, k, score=0):
    ex_ids, _, cnt, _ = ctx.route_topk(logits_np, T, E, k, score_mode=score)
    counts = [0] * E
    for t in range(T):
        for e in ex_ids[t, :cnt[t]]:
            counts[int(e)] += 1
    return counts


def prefill(nx, ctx, torch, args):
    """Mixtral-shaped Q8_0 layer, 2048 tokens, Zipf(1.2)-biased router, MFMA path."""
    import math
    E, H, F, k, T = 8, 4096, 14336, 2, 2048
    dev = torch.device("cuda", 0)
    ex = make_expert_sets(nx, ctx, torch, nx.Q8_0, E, H, F, 1, args.seed + 7)[0]
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 11)
    x = torch.randn((T, H), generator=g, device=dev, dtype=torch.float32)
    router = torch.randn((E, H), generator=g, device=dev, dtype=torch.float32) * 0.02
    p = torch.tensor([(e + 1) ** -1.2 for e in range(E)], device=dev, dtype=torch.float64)
    bias = torch.log(p / p.sum()).to(torch.float32)
    logits = (x @ router.t() + bias[None, :]).contiguous()
    out = torch.empty((T, H), device=dev, dtype=torch.float32)
    counts = active_experts(ctx, logits.cpu().numpy(), T, E, k)
    flops = 2.0 * 3 * H * F * sum(counts)
    path = {"auto": nx.PATH_AUTO, "mfma_f16": nx.PATH_MFMA_F16,
            "mfma_bf16": nx.PATH_MFMA_BF16}[args.prefill_path]

    def step(i):
        ex.forward_dev(x.data_ptr(), logits.data_ptr(), T, k, out.data_ptr(), path=path)

    ms = time_steps(torch, step, args.prefill_steps, 3, SETTLE_MS)
    kern = kernel_means(ctx, torch, step, args.prefill_steps)
    gemm_ms = kern.get("gemm_gateup", 0.0) + kern.get("gemm_down", 0.0)
    ex.close()
    # the vendor library's dense bf16 GEMM on the same products, for scale:
    # the most loaded expert's gate+up and down, and all tokens as one dense
    # expert
    lib = library_gemm_reference(torch, [(counts[0], 2 * F, H), (counts[0], H, F),
                                         (T, 2 * F, H), (T, H, F)])
    return {
        "workload": "Mixtral-8x7B MoE layer, prefill, Q8_0, Zipf(1.2) router",
        "tokens": T, "path": f"{args.prefill_path}: {path_of(kern)}", "expert_tokens": counts,
        "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3),
        "layer_TFLOPs": flops / (ms * 1e-3) / 1e12,
        "gemm_TFLOPs": flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms else None,
        "gemm_frac_of_fp16_peak": flops / (gemm_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS if gemm_ms else None,
        "kernels_ms": {k_: round(v, 4) for k_, v in kern.items()},
        "torch_bf16_matmul_TFLOPs": lib,
    }


def library_gemm_reference(torch, shapes, iters=20):
    """TFLOP/s of torch.matmul (hipBLASLt) on dense bf16 operands of shape
    [M x K] . [K x N] for each (M, N, K): what the vendor library sustains on
    the plain product, with no dequantization and no grouping."""
    dev = torch.device("cuda", 0)
    res = {}
    for M, N, K in shapes:
        a = torch.randn((M, K), device=dev, dtype=torch.bfloat16)
        b = torch.randn((K, N), device=dev, dtype=torch.bfloat16)
        for _ in range(3):
            c = a @ b
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            c = a @ b
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / iters
        res[f"{M}x{N}x{K}"] = round(2.0 * M * N * K / dt / 1e12, 1)
        del a, b, c
    return res


MODEL_CONFIGS = [
    # name, weight format, E, H, F, k, shared F, score mode, token counts, replicas rotated
    ("qwen3_q4k", "Q4_K", 128, 2048, 768, 8, 0, 0, (1, 64, 512), 2),
    ("deepseek_q4k_sigmoid_shared", "Q4_K", 256, 7168, 2048, 8, 2048, 1, (1, 4096), 2),
    ("mixtral_q2k", "Q2_K", 8, 4096, 14336, 2, 0, 0, (1, 32), 4),
    ("mixtral_q4_0", "Q4_0", 8, 4096, 14336, 2, 0, 0, (1, 32), 4),
    ("mixtral_q8_0", "Q8_0", 8, 4096, 14336, 2, 0, 0, (1, 32), 2),
]


def block_case(nx, ctx, torch, sets, x, E, H, k, args):
    """The whole MoE block of a decode step (RMSNorm -> router logits -> MoE
    layer -> residual add) on the Mixtral Q4_K sets, exact and fast mode."""
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 61)
    norm_w = 1.0 + 0.1 * torch.randn(H, generator=g, device=dev, dtype=torch.float32)
    router = torch.randn((E, H), generator=g, device=dev, dtype=torch.float32) * 0.02
    hidden = x[:1].clone()
    res = {}
    for exact in (True, False):
        def step(i, exact=exact):
            sets[i % len(sets)].block_dev(hidden.data_ptr(), norm_w.data_ptr(), H, 1e-5,
                                          router.data_ptr(), E * H, 1, k, path=nx.PATH_GEMV,
                                          exact=exact)

        ms = time_steps(torch, step, args.steps, args.warmup, SETTLE_MS)
        kern = kernel_means(ctx, torch, step, args.steps)
        res["exact" if exact else "fast"] = {
            "ms_per_step": ms, "tokens_per_s": 1 / (ms * 1e-3),
            "kernels_ms": {k_: round(v, 4) for k_, v in kern.items()}}
    return res


ROUTER_SHAPES = [
    # name, E, H, token counts
    ("mixtral", 8, 4096, (1, 32, 2048)),
    ("qwen3", 128, 2048, (1, 512)),
    ("deepseek", 256, 7168, (1, 4096)),
]


DENSE_SHAPES = [
    # name, rows, cols: Mixtral 8x7B's decode-step projections and output head
    ("attn_q", 4096, 4096),
    ("attn_k", 1024, 4096),
    ("attn_output", 4096, 4096),
    ("output", 32000, 4096),
]


def dense_cases(nx, ctx, torch, args):
    """Dense quantized matvec (one token) per projection shape and format:
    kernel mean time and GB/s on the GGUF bytes of the matrix.  Replicas are
    rotated so that every call reads its matrix from HBM rather than from the
    Infinity Cache."""
    dev = torch.device("cuda", 0)
    res = {}
    for fname, fmt in (("Q4_K", nx.Q4_K), ("Q8_0", nx.Q8_0)):
        blk, bb = nx.BLOCK[fmt]
        for name, rows, cols in DENSE_SHAPES:
            g = torch.Generator(device=dev)
            g.manual_seed(args.seed + rows)
            w = torch.randn((rows * cols,), generator=g, device=dev, dtype=torch.float32) * 0.05
            nbytes = nx.quant_bytes(fmt, rows * cols)
            q = torch.empty((nbytes,), device=dev, dtype=torch.uint8)
            ctx.quantize_dev(fmt, w.data_ptr(), rows * cols, q.data_ptr(), nbytes)
            del w
            reps = max(2, min(512, (1 << 30) // nbytes))
            mats = []
            for _ in range(reps):
                m = nx.Matrix(ctx, fmt, rows, cols)
                m.load_dev(q.data_ptr(), nbytes)
                mats.append(m)
            del q
            x = torch.randn((cols,), generator=g, device=dev, dtype=torch.float32)
            y = torch.empty((rows,), device=dev, dtype=torch.float32)

            def step(i, mats=mats, x=x, y=y, cols=cols):
                mats[i % len(mats)].matvec_dev(x.data_ptr(), cols, 1, y.data_ptr())

            time_steps(torch, step, reps, 2)
            kern = kernel_means(ctx, torch, step, 4 * reps)
            ms = kern.get("gemv_matrix", float("nan"))
            res[f"{name}_{fname}"] = {"rows": rows, "cols": cols, "us": round(ms * 1e3, 2),
                                      "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                      "replicas": reps}
            for m in mats:
                m.close()
    return res


def router_cases(nx, ctx, torch, args):
    """Router logits on device (logits = x . W_r^T, fp32): kernel mean time of
    the exact mode (the reference matvec's sequential order, bit-identical)
    and of the fast mode (parallel order with fma), per model shape and token
    count."""
    dev = torch.device("cuda", 0)
    res = {}
    for name, E, H, tokens in ROUTER_SHAPES:
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + 51)
        Tm = max(tokens)
        x = torch.randn((Tm, H), generator=g, device=dev, dtype=torch.float32)
        w = torch.randn((E, H), generator=g, device=dev, dtype=torch.float32) * 0.02
        out = torch.empty((Tm, E), device=dev, dtype=torch.float32)
        cases = {}
        for T in tokens:
            row = {}
            for exact in (True, False):
                def step(i, T=T, exact=exact):
                    ctx.router_logits_dev(w.data_ptr(), E * H, x.data_ptr(), T * H, T, E, H,
                                          out.data_ptr(), exact=exact)

                n = 50 if T <= 64 else 10
                time_steps(torch, step, 3, 2)
                kern = kernel_means(ctx, torch, step, n)
                ms = sum(kern.values())
                row["exact_us" if exact else "fast_us"] = round(ms * 1e3, 2)
                row["exact_kernel" if exact else "fast_kernel"] = next(iter(kern), None)
            cases[f"T{T}"] = row
        res[name] = {"experts": E, "hidden": H, "cases": cases}
    return res


def model_config_cases(nx, ctx, torch, args, only=None):
    """The other model shapes of the hot-path survey (AUTO path; Q4_K experts,
    and Mixtral's shape on Q2_K, Q4_0 and Q8_0):
    per token count, ms/step and the fraction of HBM and dense-fp16 MFMA peak
    on algorithmic bytes / FLOPs (realised routing).  Replicas are rotated so
    that decode steps read HBM rather than the Infinity Cache."""
    dev = torch.device("cuda", 0)
    res = {}
    for name, fname, E, H, F, k, Fs, score, tokens, reps in MODEL_CONFIGS:
        if only is not None:  # (name, token count or None)
            if name != only[0]:
                continue
            if only[1] is not None:
                tokens = (only[1],)
        print(f"bench: {name}", file=sys.stderr, flush=True)
        fmt = {"Q4_K": nx.Q4_K, "Q2_K": nx.Q2_K, "Q4_0": nx.Q4_0, "Q8_0": nx.Q8_0}[fname]
        # GGUF bytes per weight; Q2_K stays resident as 16 bytes of 2-bit
        # codes and 8 scale-plane bytes per 64 weights (0.375 B/weight read
        # per step)
        bpw = {"Q4_K": Q4K_BYTES_PER_WEIGHT, "Q2_K": 84.0 / 256.0, "Q4_0": 18.0 / 32.0,
               "Q8_0": 34.0 / 32.0}[fname]
        rbpw = {"Q4_K": Q4K_BYTES_PER_WEIGHT, "Q2_K": 0.375, "Q4_0": 18.0 / 32.0,
                "Q8_0": 34.0 / 32.0}[fname]
        sets = make_expert_sets(nx, ctx, torch, fmt, E, H, F, reps, args.seed + 31, Fs)
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + 41)
        Tm = max(tokens)
        x = torch.randn((Tm, H), generator=g, device=dev, dtype=torch.float32)
        router = torch.randn((E, H), generator=g, device=dev, dtype=torch.float32) * 0.02
        logits = (x @ router.t()).contiguous()
        out = torch.empty((Tm, H), device=dev, dtype=torch.float32)
        cases = {}
        for T in tokens:
            counts = active_experts(ctx, logits[:T].cpu().numpy(), T, E, k, score)
            n_act = sum(1 for c in counts if c) + (1 if Fs else 0)
            welems = sum(1 for c in counts if c) * 3 * H * F + (3 * H * Fs if Fs else 0)
            wbytes = welems * bpw
            flops = 2.0 * 3 * H * F * sum(counts) + (2.0 * 3 * H * Fs * T if Fs else 0.0)

            def step(i, T=T):
                sets[i % len(sets)].forward_dev(x.data_ptr(), logits.data_ptr(), T, k,
                                                out.data_ptr(), score_mode=score,
                                                path=nx.PATH_AUTO)

            steps = args.steps if T <= 64 else max(10, args.prefill_steps)
            ms = time_steps(torch, step, steps, 3, SETTLE_MS)
            kern = kernel_means(ctx, torch, step, steps)
            gbps = wbytes / (ms * 1e-3) / 1e9
            tf = flops / (ms * 1e-3) / 1e12
            cases[f"T{T}"] = {
                "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3),
                "experts_active": n_act, "weight_bytes": wbytes, "flops": flops,
                "effective_GBps": gbps, "hbm_frac": gbps / HBM_PEAK_GBPS,
                "resident_GBps": welems * rbpw / (ms * 1e-3) / 1e9,
                "TFLOPs": tf, "mfma_f16_frac": tf / MFMA_F16_PEAK_TFLOPS,
                "path": path_of(kern),
                "kernels_ms": {k_: round(v, 4) for k_, v in kern.items()}}
        for s_ in sets:
            s_.close()
        res[name] = {"experts": E, "hidden": H, "ffn": F, "top_k": k, "shared_ffn": Fs,
                     "score": "sigmoid" if score else "softmax", "weights": fname,
                     "replicas_rotated": reps, "cases": cases}
    return res


def only_case(nx, ctx, torch, args):
    """One extra workload by itself (--only)."""
    if args.only == "prefill":
        return {"prefill_2048_tokens": prefill(nx, ctx, torch, args)}
    if args.only == "router":
        return {"router_logits": router_cases(nx, ctx, torch, args)}
    if args.only == "dense":
        return {"dense_matvec_1_token": dense_cases(nx, ctx, torch, args)}
    if args.only == "block":
        E, H, k = 8, 4096, 2
        sets = make_expert_sets(nx, ctx, torch, nx.Q4_K, E, H, 14336, args.replicas, args.seed)
        g = torch.Generator(device=torch.device("cuda", 0))
        g.manual_seed(args.seed + 1)
        x = torch.randn((32, H), generator=g, device=torch.device("cuda", 0), dtype=torch.float32)
        rec = {"moe_block_1_token": block_case(nx, ctx, torch, sets, x, E, H, k, args)}
        for s_ in sets:
            s_.close()
        return rec
    name, _, tok = args.only.partition(":")
    if name not in [m[0] for m in MODEL_CONFIGS]:
        raise SystemExit(f"--only: unknown workload {args.only!r}")
    T = int(tok.lstrip("T")) if tok else None
    return {"model_configs": model_config_cases(nx, ctx, torch, args, only=(name, T))}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    import torch

    import nexus_amd as nx

    E, H, F, k, T = 8, 4096, 14336, 2, args.tokens
    path = {"auto": nx.PATH_AUTO, "gemv": nx.PATH_GEMV, "mfma_f16": nx.PATH_MFMA_F16,
            "mfma_split": nx.PATH_MFMA_SPLIT,
            "mfma_bf16": nx.PATH_MFMA_BF16}[args.path]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    ctx = nx.Context(0)
    # torch and the library share one explicit stream, so every launch is
    # ordered after the tensors it reads (torch's default is the null stream)
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)

    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only and args.only != "decode":
        print(json.dumps(only_case(nx, ctx, torch, args)), flush=True)
        ctx.close()
        return
    print(f"bench: building {args.replicas} Q4_K expert replicas (E={E} H={H} F={F})",
          file=sys.stderr, flush=True)
    sets = make_expert_sets(nx, ctx, torch, nx.Q4_K, E, H, F, args.replicas, args.seed)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 1)
    x = torch.randn((max(T, 32), H), generator=g, device=dev, dtype=torch.float32)
    router = torch.randn((E, H), generator=g, device=dev, dtype=torch.float32) * 0.02
    logits = (x @ router.t()).contiguous()
    out = torch.empty((max(T, 32), H), device=dev, dtype=torch.float32)

    def decode_case(ntok, pth, settle_ms=0.0):
        def step(i):
            sets[i % len(sets)].forward_dev(x.data_ptr(), logits.data_ptr(), ntok, k,
                                            out.data_ptr(), path=pth)

        ms = time_steps(torch, step, args.steps, args.warmup, settle_ms)
        kern = kernel_means(ctx, torch, step, args.steps)
        # the bytes of the experts the steps activate (the routes are read back
        # to the host after the timed steps, so no host round trip precedes them)
        counts = active_experts(ctx, logits[:ntok].cpu().numpy(), ntok, E, k)
        n_act = sum(1 for c in counts if c)
        gu_bytes = n_act * 2 * F * H * Q4K_BYTES_PER_WEIGHT
        dn_bytes = n_act * H * F * Q4K_BYTES_PER_WEIGHT
        return ms, kern, gu_bytes, dn_bytes, step

    print("bench: decode", file=sys.stderr, flush=True)
    ms_per_step, kern, gateup_bytes, down_bytes, decode_step = decode_case(T, path)
    # after the timed region: the per-step distribution over >= 100 steps
    dist = step_distribution(torch, decode_step, max(200, args.steps))
    step_bytes = gateup_bytes + down_bytes
    print("bench: per-kernel mean ms " + json.dumps({k_: round(v, 5) for k_, v in kern.items()}),
          file=sys.stderr, flush=True)
    # the dominant kernel (gate/up) and the down kernel of the path that ran
    ran = path_of(kern)
    gu_name, dn_name = {"gemv": ("gemv_gateup", "gemv_down_combine"),
                        "mfma_split": ("mfv_gateup", "mfv_down")}.get(ran, (None, None))
    if dn_name == "gemv_down_combine" and dn_name not in kern:
        dn_name = "gemv_down"
    gu_ms, dn_ms = kern.get(gu_name), kern.get(dn_name)
    achieved = gateup_bytes / (gu_ms * 1e-3) / 1e9 if gu_ms else None

    extra = {}
    if not args.no_extra and not args.only:
        print("bench: decode, 32 tokens", file=sys.stderr, flush=True)
        ms32, kern32, gu32, dn32, _ = decode_case(32, nx.PATH_AUTO, SETTLE_MS)
        extra["decode_32_tokens"] = {
            "ms_per_step": ms32, "settle_ms": SETTLE_MS, "tokens_per_s": 32 / (ms32 * 1e-3),
            "effective_GBps": (gu32 + dn32) / (ms32 * 1e-3) / 1e9, "path": "auto: " + path_of(kern32),
            "kernels_ms": {k_: round(v, 4) for k_, v in kern32.items()}}
    if not args.no_extra and not args.only:
        print("bench: MoE block, 1 token", file=sys.stderr, flush=True)
        extra["moe_block_1_token"] = block_case(nx, ctx, torch, sets, x, E, H, k, args)
    for s_ in sets:
        s_.close()
    if not args.no_extra and not args.only:
        print("bench: prefill", file=sys.stderr, flush=True)
        extra["prefill_2048_tokens"] = prefill(nx, ctx, torch, args)
        extra["model_configs"] = model_config_cases(nx, ctx, torch, args)
        print("bench: router logits", file=sys.stderr, flush=True)
        extra["router_logits"] = router_cases(nx, ctx, torch, args)
        print("bench: dense matvec", file=sys.stderr, flush=True)
        extra["dense_matvec_1_token"] = dense_cases(nx, ctx, torch, args)

    # HBM bytes per launch measured by counters exist for the one-token GEMV
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemv_gateup_mixtral_q4k_t1_traffic.json")
    if ran == "gemv" and T == 1 and os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get("bytes_per_launch")
        except Exception:
            traffic = None

    cpu = None
    if not args.no_cpu and not args.only:
        print(f"bench: cpu baseline on {args.cpu_tokens} tokens", file=sys.stderr, flush=True)
        cpu = cpu_baseline(nx, ctx, torch, x, {"router": router}, E, H, F, k, args.seed,
                           args.cpu_tokens)

    rec = {
        "metric": METRIC,
        "value": T / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        # the secondary cases also run untimed steps for this long first
        "secondary_settle_ms": SETTLE_MS,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Mixtral-8x7B MoE layer, decode", "hidden": H, "ffn": F,
                   "experts": E, "top_k": k, "tokens": T, "weights": "Q4_K",
                   "path": args.path, "replicas_rotated": len(sets)},
        "effective_GBps": step_bytes / (ms_per_step * 1e-3) / 1e9,
        "layer_hbm_frac": step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "kernels_ms": {k_: round(v, 5) for k_, v in kern.items()},
        "step_time_stats": dist,
        "roofline": {"bound": "hbm", "kernel": gu_name, "achieved": achieved,
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS if achieved else None,
                     "traffic": traffic, "algorithmic_bytes": gateup_bytes},
        "down_GBps": down_bytes / (dn_ms * 1e-3) / 1e9 if dn_ms else None,
        "cpu_baseline": cpu,
    }
    rec.update(extra)
    ctx.close()
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
