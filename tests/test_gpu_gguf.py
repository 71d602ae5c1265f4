"""Quantized-resident expert loading from GGUF files (nx_experts_load_gguf).

A block's experts loaded from a file must run the layer exactly as the same
payloads loaded one by one through nx_experts_load (bit-identical output),
and match the oracle's dispatch over the dequantized weights within the GEMV
path's relative L2 1e-4.  The router logits come from the file's
blk.L.ffn_gate_inp.weight through the exact router kernel.  A file holding
Q4_K codes in upstream ggml's order, loaded with NX_Q4K_GGML, runs exactly as
the reference-order file.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from moe_cases import assert_same_bits, rel_l2
from test_gguf import moe_file

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def reference_to_ggml(blocks: np.ndarray) -> np.ndarray:
    """Q4_K blocks from the reference's code order to upstream ggml's."""
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 144).copy()
    qs = b[:, 16:]
    code = np.concatenate([qs & 15, qs >> 4], axis=1)  # element order 0..255
    out = np.zeros_like(qs)
    for j in range(4):
        lo = code[:, 64 * j:64 * j + 32]
        hi = code[:, 64 * j + 32:64 * j + 64]
        out[:, 32 * j:32 * j + 32] = lo | (hi << 4)
    b[:, 16:] = out
    return b.ravel()


def layer_from_payloads(ctx, fmt, E, H, F, Fs, pays):
    ex = nx.Experts(ctx, fmt, E, H, F, Fs)
    for (e, r), q in pays.items():
        ex.load(nx.EXPERT_SHARED if e == "s" else e, r, q)
    return ex


def oracle_layer(fmt, E, H, F, Fs, pays, x, logits, k):
    def deq(q, n):
        return oracle.dequantize(fmt, q, n) if fmt else q.view(np.float32)
    g = [deq(pays[(e, 0)], F * H) for e in range(E)]
    u = [deq(pays[(e, 1)], F * H) for e in range(E)]
    d = [deq(pays[(e, 2)], H * F) for e in range(E)]
    shared = None
    if Fs:
        shared = [deq(pays[("s", 0)], Fs * H), deq(pays[("s", 1)], Fs * H),
                  deq(pays[("s", 2)], H * Fs)]
    return oracle.moe_layer(x, logits, g, u, d, k, 0, shared=shared)


@pytest.mark.parametrize("fmt,naming,Fs", [
    (oracle.Q4_K, "merged", 0), (oracle.Q8_0, "gguf", 256), (oracle.Q4_0, "hf", 0),
    (0, "merged", 128), (oracle.Q2_K, "merged", 256)])
def test_gguf_layer_matches_direct_load_and_oracle(ctx, tmp_path, fmt, naming, Fs):
    E, H, F, k, T, layer = 6, 512, 768, 2, 5, 1
    print(f"gguf layer fmt={fmt} naming={naming} Fs={Fs}", flush=True)
    w, pays, router = moe_file(fmt, E, H, F, layer=layer, naming=naming, shared_F=Fs, seed=fmt + 3)
    path = tmp_path / "moe.gguf"
    w.write(path)
    x = np.random.default_rng(1).standard_normal((T, H)).astype(np.float32)
    with nx.Gguf(str(path)) as g:
        wr = g.data(g.find(f"blk.{layer}.ffn_gate_inp.weight")).view(np.float32)
        logits = ctx.router_logits(wr, x, E, H, exact=True)
        ex = nx.experts_from_gguf(ctx, g, layer)
    ref_logits = np.stack([oracle.matvec(router.ravel(), E, H, x[t]) for t in range(T)])
    assert_same_bits(logits, ref_logits)
    assert ex.device_bytes() > 0
    got = ex.forward(x, logits, k, path=nx.PATH_GEMV)
    direct = layer_from_payloads(ctx, fmt, E, H, F, Fs, pays)
    want = direct.forward(x, logits, k, path=nx.PATH_GEMV)
    assert_same_bits(got, want)
    ref = oracle_layer(fmt, E, H, F, Fs, pays, x, logits, k)
    assert rel_l2(got, ref) <= 1e-4
    ex.close()
    direct.close()


def test_gguf_q4k_ggml_order(ctx, tmp_path):
    E, H, F, k, T = 4, 512, 512, 2, 3
    w, pays, router = moe_file(oracle.Q4_K, E, H, F, naming="merged", seed=11)
    ref_path, ggml_path = tmp_path / "ref.gguf", tmp_path / "ggml.gguf"
    w.write(ref_path)
    w.tensors = [(n, d, t, reference_to_ggml(np.frombuffer(b, np.uint8)).tobytes()
                  if t == 12 else b) for n, d, t, b in w.tensors]
    w.write(ggml_path)
    x = np.random.default_rng(2).standard_normal((T, H)).astype(np.float32)
    logits = np.stack([oracle.matvec(router.ravel(), E, H, x[t]) for t in range(T)])
    with nx.Gguf(str(ref_path)) as g1, nx.Gguf(str(ggml_path)) as g2:
        a = nx.experts_from_gguf(ctx, g1, 0, nx.Q4K_REFERENCE)
        b = nx.experts_from_gguf(ctx, g2, 0, nx.Q4K_GGML)
        c = nx.experts_from_gguf(ctx, g2, 0, nx.Q4K_REFERENCE)  # misread on purpose
    ya, yb, yc = (m.forward(x, logits, k, path=nx.PATH_GEMV) for m in (a, b, c))
    assert_same_bits(yb, ya)
    assert rel_l2(yc, ya) > 1e-2
    for m in (a, b, c):
        m.close()


def test_gguf_load_errors(ctx, tmp_path):
    w, _, _ = moe_file(oracle.Q8_0, 2, 64, 64, naming="merged")
    p = tmp_path / "m.gguf"
    w.write(p)
    with nx.Gguf(str(p)) as g:
        with pytest.raises(nx.NexusError) as ei:
            nx.experts_from_gguf(ctx, g, 5)
        assert ei.value.code == nx.NX_ERR_NOT_FOUND
        with pytest.raises(nx.NexusError) as ei:
            nx.experts_from_gguf(ctx, g, 0, 7)
        assert ei.value.code == nx.NX_ERR_INVALID_ARG
    data = p.read_bytes()
    short = tmp_path / "short.gguf"
    short.write_bytes(data[:len(data) - 3000])  # cuts into the expert payloads
    with nx.Gguf(str(short)) as g:
        with pytest.raises(nx.NexusError) as ei:
            nx.experts_from_gguf(ctx, g, 0)
        assert ei.value.code == nx.NX_ERR_TRUNCATED
