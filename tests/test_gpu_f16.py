"""F16 and BF16 weights on device (GgufReader::tensor_bytes_to_f32,
src/gguf/mod.rs:921-946): dequantization bit-exact against the oracle on
every bit pattern; experts and dense matrices resident as raw 16-bit values
on the GEMV path, within relative L2 1e-4 of the oracle over the same
payloads (rows that are not a whole number of 16-value segments included);
GGUF files with F16/BF16 tensors load; the MFMA paths reject these formats.
"""
import numpy as np
import pytest

import nexus_amd as nx
import oracle
from gguf_writer import GgufWriter
from moe_cases import BF16, F16, Layer, assert_same_bits, half_payload, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = nx.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("fmt", [F16, BF16])
def test_dequant_every_pattern(ctx, fmt):
    bits = np.arange(65536, dtype=np.uint16).view(np.uint8)
    assert_same_bits(ctx.dequant(fmt, bits, 65536), oracle.dequantize(fmt, bits, 65536))
    with pytest.raises(nx.NexusError) as ei:
        ctx.dequant(fmt, bits[:9], 5)
    assert str(ei.value) == f"{nx.FORMAT_NAMES[fmt]} tensor payload is truncated"


@pytest.mark.parametrize("fmt", [F16, BF16])
@pytest.mark.parametrize("E,H,F,k,T", [(8, 520, 1000, 2, 1), (8, 512, 768, 2, 3),
                                       (16, 256, 2048, 4, 9)])
def test_layer_gemv_parity(ctx, fmt, E, H, F, k, T):
    print(f"16-bit layer fmt={fmt} E={E} H={H} F={F} k={k} T={T}", flush=True)
    L = Layer(fmt, E, H, F, k, T, seed=E + H + F + T + fmt)
    ex = L.upload(nx, ctx)
    got = ex.forward(L.x, L.logits, k, 0, nx.PATH_GEMV)
    auto = ex.forward(L.x, L.logits, k, 0, nx.PATH_AUTO)
    for path in (nx.PATH_MFMA_F16, nx.PATH_MFMA_BF16, nx.PATH_MFMA_SPLIT):
        with pytest.raises(nx.NexusError) as ei:
            ex.forward(L.x, L.logits, k, 0, path)
        assert ei.value.code == nx.NX_ERR_UNSUPPORTED
    ex.close()
    assert rel_l2(got, L.oracle_out()) <= TOL
    assert_same_bits(auto, got)


@pytest.mark.parametrize("fmt", [F16, BF16])
def test_dense_matvec(ctx, fmt):
    rng = np.random.default_rng(fmt)
    for rows, cols, T in ((300, 4100, 2), (64, 8192, 1), (33, 7, 3)):
        w = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
        q = half_payload(fmt, w)
        wf = oracle.dequantize(fmt, q, rows * cols)
        m = nx.Matrix(ctx, fmt, rows, cols)
        m.load(q)
        x = rng.standard_normal((T, cols)).astype(np.float32)
        got = m.matvec(x)
        m.close()
        for t in range(T):
            assert rel_l2(got[t], oracle.matvec(wf, rows, cols, x[t])) <= TOL
    with pytest.raises(nx.NexusError) as ei:
        nx.Matrix(ctx, fmt, 8, 8193)  # longer than the register-resident GEMV takes
    assert ei.value.code == nx.NX_ERR_UNSUPPORTED


def test_gguf_f16_experts_and_head(ctx, tmp_path):
    E, H, F, k, T = 4, 256, 512, 2, 3
    L = Layer(F16, E, H, F, k, T, seed=12)
    wr = GgufWriter()
    for r, (name, rows, cols) in enumerate((("ffn_gate_exps", F, H), ("ffn_up_exps", F, H),
                                            ("ffn_down_exps", H, F))):
        data = np.concatenate([L.payload[(e, r)] for e in range(E)])
        wr.add_tensor(f"blk.0.{name}.weight", [cols, rows, E], F16, data)
    rng = np.random.default_rng(5)
    head = (rng.standard_normal(96 * H) * 0.05).astype(np.float32)
    wr.add_tensor("output.weight", [H, 96], BF16, half_payload(BF16, head))
    path = tmp_path / "f16.gguf"
    wr.write(path)
    with nx.Gguf(str(path)) as g:
        assert g.moe_info(0)["fmt"] == F16
        ex = nx.experts_from_gguf(ctx, g, 0)
        got = ex.forward(L.x, L.logits, k, 0, nx.PATH_GEMV)
        ex.close()
        m = nx.matrix_from_gguf(ctx, g, "output.weight")
        assert (m.fmt, m.rows, m.cols) == (BF16, 96, H)
        y = m.matvec(L.x[0])
        m.close()
    assert rel_l2(got, L.oracle_out()) <= TOL
    hf = oracle.dequantize(BF16, half_payload(BF16, head), head.size)
    assert rel_l2(y, oracle.matvec(hf, 96, H, L.x[0])) <= TOL
