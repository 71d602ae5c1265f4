"""Dense quantized matvec (nx_matvec): the q/k/v/o projections and the output
head of the decode step (src/engine/mod.rs:1108-1126, 1032-1043), with the
weight kept resident in its GGUF format.

Bar: every token row within relative L2 1e-4 of the oracle's
InferenceEngine::matvec (src/engine/mod.rs:775-801) over the oracle's
dequantization of the same payload, for F32, Q4_0, Q8_0, Q4_K and Q2_K, at
projection shapes (square, grouped-query k/v, a wide row), an output head of
32000 rows, ragged row counts, odd F32 row lengths and 1 to 9 tokens.  The
device entry point gives the blocking one's bits; a matrix loaded from a
GGUF file (reference or upstream ggml Q4_K order) gives the bits of the
same payload loaded directly; errors carry the reference's messages.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from gguf_writer import GgufWriter
from moe_cases import DeviceArray, assert_same_bits, rel_l2
from test_gpu_gguf import reference_to_ggml

pytestmark = pytest.mark.gpu

TOL = 1e-4
FMTS = [nx.F32, nx.Q4_0, nx.Q8_0, nx.Q4_K, nx.Q2_K]


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


def payload(fmt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
    if fmt == nx.F32:
        return w.view(np.uint8), w
    q = oracle.quantize(fmt, w)
    return q, oracle.dequantize(fmt, q, rows * cols)


def oracle_rows(wf, rows, cols, x):
    return np.stack([oracle.matvec(wf, rows, cols, xt) for xt in x])


def check(ctx, fmt, rows, cols, T, seed):
    print(f"matvec fmt={nx.FORMAT_NAMES[fmt]} rows={rows} cols={cols} T={T}", flush=True)
    q, wf = payload(fmt, rows, cols, seed)
    m = nx.Matrix(ctx, fmt, rows, cols)
    m.load(q)
    x = np.random.default_rng(seed + 1).standard_normal((T, cols)).astype(np.float32)
    got = m.matvec(x)
    ref = oracle_rows(wf, rows, cols, x)
    for t in range(T):
        assert rel_l2(got[t], ref[t]) <= TOL, (t, rel_l2(got[t], ref[t]))
    return m, x, got


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("rows,cols,T", [(4096, 4096, 1), (1024, 4096, 1), (512, 14336, 1),
                                         (1000, 2048, 3), (37, 512, 9)])
def test_matvec_parity(ctx, fmt, rows, cols, T):
    if fmt == nx.F32 and cols > 4096:
        # F32 rows hold 8 weights per 32-byte segment: 4096 is the longest
        # row the register-resident GEMV takes
        with pytest.raises(nx.NexusError) as ei:
            nx.Matrix(ctx, fmt, rows, cols)
        assert ei.value.code == nx.NX_ERR_UNSUPPORTED
        return
    m, _, _ = check(ctx, fmt, rows, cols, T, seed=rows + cols + T + fmt)
    m.close()


@pytest.mark.parametrize("fmt", [nx.Q4_K, nx.Q8_0])
def test_output_head(ctx, fmt):
    m, _, _ = check(ctx, fmt, 32000, 1024, 1, seed=5 + fmt)
    m.close()


@pytest.mark.parametrize("cols", [1, 13, 1000, 4095])
def test_f32_odd_rows(ctx, cols):
    m, _, _ = check(ctx, nx.F32, 77, cols, 2, seed=cols)
    m.close()


def test_matvec_dev_same_bits(ctx):
    m, x, got = check(ctx, nx.Q4_K, 768, 2048, 4, seed=11)
    dx = DeviceArray(x.size)
    dx.upload(x)
    dy = DeviceArray(4 * 768, fill=np.nan)
    m.matvec_dev(dx.ptr, x.size, 4, dy.ptr)
    assert_same_bits(dy.download().reshape(4, 768), got)
    # a single token after a batch: rows beyond it untouched
    dy.upload(np.full(4 * 768, 7.0, np.float32))
    m.matvec_dev(dx.ptr, 2048, 1, dy.ptr)
    out = dy.download().reshape(4, 768)
    assert_same_bits(out[0], got[0])
    assert np.all(out[1:] == 7.0)
    m.close()


def test_matvec_zero_tokens_and_errors(ctx):
    m = nx.Matrix(ctx, nx.Q8_0, 64, 256)
    q, _ = payload(nx.Q8_0, 64, 256, 3)
    m.load(q)
    assert m.matvec(np.zeros((0, 256), np.float32)).shape == (0, 64)
    with pytest.raises(nx.NexusError) as ei:
        m.matvec(np.zeros(255, np.float32))
    assert ei.value.code == nx.NX_ERR_SHAPE
    assert str(ei.value) == "Matvec input shape mismatch: got 255, expected 256"
    with pytest.raises(nx.NexusError) as ei:
        m.matvec(np.zeros(512, np.float32), num_tokens=3)
    assert str(ei.value) == "Matvec input shape mismatch: got 512, expected 768"
    with pytest.raises(nx.NexusError) as ei:
        m.load(q[:34 * 100])
    assert ei.value.code == nx.NX_ERR_SHAPE
    assert str(ei.value) == "Matvec weight too small: got 3200, expected at least 16384"
    m.close()
    f = nx.Matrix(ctx, nx.F32, 3, 5)
    with pytest.raises(nx.NexusError) as ei:
        f.load(np.zeros(14, np.float32))
    assert str(ei.value) == "Matvec weight too small: got 14, expected at least 15"
    f.close()
    with pytest.raises(nx.NexusError) as ei:
        nx.Matrix(ctx, nx.Q4_K, 16, 300)
    assert ei.value.code == nx.NX_ERR_UNSUPPORTED
    with pytest.raises(nx.NexusError) as ei:
        nx.Matrix(ctx, nx.Q4_K, 0, 256)
    assert ei.value.code == nx.NX_ERR_INVALID_ARG


def test_matrix_from_gguf(ctx, tmp_path):
    rows, cols = 320, 1024
    q, wf = payload(nx.Q4_K, rows, cols, 21)
    w8, _ = payload(nx.Q8_0, 96, 512, 22)
    wr = GgufWriter()
    wr.add_tensor("blk.0.attn_q.weight", [cols, rows], nx.Q4_K, q)
    wr.add_tensor("output.weight", [512, 96], nx.Q8_0, w8)
    path = tmp_path / "dense.gguf"
    wr.write(path)
    gw = GgufWriter()
    gw.add_tensor("blk.0.attn_q.weight", [cols, rows], nx.Q4_K, reference_to_ggml(q))
    gpath = tmp_path / "dense_ggml.gguf"
    gw.write(gpath)

    x = np.random.default_rng(4).standard_normal((2, cols)).astype(np.float32)
    direct = nx.Matrix(ctx, nx.Q4_K, rows, cols)
    direct.load(q)
    want = direct.matvec(x)
    direct.close()
    with nx.Gguf(str(path)) as g:
        m = nx.matrix_from_gguf(ctx, g, "blk.0.attn_q.weight")
        assert (m.fmt, m.rows, m.cols) == (nx.Q4_K, rows, cols)
        assert_same_bits(m.matvec(x), want)
        m.close()
        h = nx.matrix_from_gguf(ctx, g, "output.weight")
        assert (h.fmt, h.rows, h.cols) == (nx.Q8_0, 96, 512)
        h.close()
        with pytest.raises(nx.NexusError) as ei:
            nx.matrix_from_gguf(ctx, g, "lm_head.weight")
        assert ei.value.code == nx.NX_ERR_NOT_FOUND
        assert str(ei.value) == "Missing tensor: lm_head.weight"
    with nx.Gguf(str(gpath)) as g:
        m = nx.matrix_from_gguf(ctx, g, "blk.0.attn_q.weight", nx.Q4K_GGML)
        assert_same_bits(m.matvec(x), want)
        m.close()
    ref = oracle_rows(wf, rows, cols, x)
    assert max(rel_l2(want[t], ref[t]) for t in range(2)) <= TOL


def test_q8_0_wide_rows_several_tokens(ctx):
    """Rows of 14336 Q8_0 weights hold one token's activations in registers
    at a time: several tokens run one after another, on the dense matvec and
    on the MoE layer's GEMV path."""
    from moe_cases import Layer
    m, _, _ = check(ctx, nx.Q8_0, 256, 14336, 3, seed=9)
    m.close()
    L = Layer(nx.Q8_0, 4, 256, 14336, 2, 3, seed=12)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, 2, 0, nx.PATH_GEMV)
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL
