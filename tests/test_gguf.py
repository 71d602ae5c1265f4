"""GGUF parsing and MoE tensor discovery (nx_gguf_*; no GPU).

Parity anchors: the reference's own GGUF tests (src/gguf/mod.rs:1636-1732:
a one-tensor v3 file read back value for value, a truncated tensor table
that errors without panicking), its error messages, its metadata accessor
semantics (get_usize over U64/U32/non-negative I64/I32), the alignment rule
(general.alignment as U32 or U64, default 32, at least 1) and its array
handling.  Files are produced by tests/gguf_writer.py.  The upstream-ggml
Q4_K code order is checked against a numpy statement of upstream's block
dequantization (published llama.cpp layout) through the oracle's reference
dequantizer.
"""
import struct

import numpy as np
import pytest

import nexus_amd as nx
import oracle
from gguf_writer import (ARRAY, BOOL, F32, F64, GgufWriter, I8, I16, I32, I64, STRING, U8, U16,
                         U32, U64)

GT_F32, GT_F16, GT_Q4_0, GT_Q8_0, GT_Q4_K = 0, 1, 2, 8, 12


def open_bytes(tmp_path, data: bytes, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return nx.Gguf(str(p))


def parse_error(tmp_path, data: bytes):
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    with pytest.raises(nx.NexusError) as ei:
        nx.Gguf(str(p))
    return ei.value


def test_reference_parse_file_case(tmp_path):
    # src/gguf/mod.rs:1636-1675, byte for byte
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 1, 4)
    for key, val in (("general.alignment", 32),):
        b += struct.pack("<Q", len(key)) + key.encode() + struct.pack("<II", 4, val)
    key, val = "general.architecture", "llama"
    b += struct.pack("<Q", len(key)) + key.encode() + struct.pack("<I", 8)
    b += struct.pack("<Q", len(val)) + val.encode()
    for key, val in (("llama.embedding_length", 4), ("llama.block_count", 1)):
        b += struct.pack("<Q", len(key)) + key.encode() + struct.pack("<II", 4, val)
    name = "token_embd.weight"
    b += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<IQIQ", 1, 4, 0, 0)
    while len(b) % 32:
        b.append(0)
    expected = [1.0, -2.0, 3.5, 4.25]
    b += struct.pack("<4f", *expected)
    with open_bytes(tmp_path, bytes(b)) as g:
        info = g.info()
        assert info["alignment"] == 32 and info["version"] == 3
        assert info["data_offset"] == len(b) - 16
        assert g.meta_usize("llama.embedding_length") == 4
        assert g.meta_usize("llama.block_count") == 1
        assert g.meta_str("general.architecture") == "llama"
        i = g.find("token_embd.weight")
        t = g.tensor(i)
        assert t["dims"] == [4] and t["type"] == GT_F32 and t["bytes"] == 16
        assert t["offset"] == len(b) - 16
        assert g.data(i).view(np.float32).tolist() == expected


def test_truncated_tensor_table_returns_error(tmp_path):
    # src/gguf/mod.rs:1716-1732: one tensor announced, none present
    e = parse_error(tmp_path, b"GGUF" + struct.pack("<IQQ", 3, 1, 0))
    assert str(e) == "Unexpected EOF reading tensor name length"
    assert e.code == nx.NX_ERR_TRUNCATED


@pytest.mark.parametrize("data,msg", [
    (b"GGU", "Invalid GGUF magic"),
    (b"GGML" + struct.pack("<IQQ", 3, 0, 0), "Invalid GGUF magic"),
    (b"GGUF" + struct.pack("<IQQ", 1, 0, 0), "Unsupported GGUF version: 1"),
    (b"GGUF" + struct.pack("<IQQ", 4, 0, 0), "Unsupported GGUF version: 4"),
    (b"GGUF" + struct.pack("<I", 3) + b"\0" * 4, "Unexpected EOF reading tensor count"),
    (b"GGUF" + struct.pack("<IQ", 3, 0), "Unexpected EOF reading kv count"),
    (b"GGUF" + struct.pack("<IQQ", 3, 0, 1), "Unexpected EOF reading metadata key length"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 0, 1, 9) + b"abc", "Key string exceeds file bounds"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 0, 1, 1) + b"k", "Unexpected EOF reading value type"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 0, 1, 1) + b"k" + struct.pack("<I", 13),
     "Unknown value type: 13"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 0, 1, 1) + b"k" + struct.pack("<IIQ", 9, 77, 0),
     "Unknown array type"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 0, 1, 1) + b"k" + struct.pack("<IQ", 8, 100) + b"ab",
     "Unexpected EOF reading metadata value"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 1, 0, 50) + b"t", "Tensor name exceeds file bounds"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 1, 0, 1) + b"t", "Unexpected EOF reading dims"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 1, 0, 1) + b"t" + struct.pack("<IQ", 2, 4),
     "Unexpected EOF reading shape"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 1, 0, 1) + b"t" + struct.pack("<IQ", 1, 4),
     "Unexpected EOF reading data type"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 1, 0, 1) + b"t" + struct.pack("<IQI", 1, 4, 4),
     "Unknown data type: 4"),
    (b"GGUF" + struct.pack("<IQQQ", 3, 1, 0, 1) + b"t" + struct.pack("<IQI", 1, 4, 0),
     "Unexpected EOF reading tensor offset"),
])
def test_parse_errors(tmp_path, data, msg):
    assert str(parse_error(tmp_path, data)) == msg


def test_missing_file():
    with pytest.raises(nx.NexusError) as ei:
        nx.Gguf("/nonexistent/dir/model.gguf")
    assert ei.value.code == nx.NX_ERR_IO


def test_metadata_values_and_accessors(tmp_path):
    w = GgufWriter(version=2)
    w.add("u8", U8, 200)
    w.add("i8", I8, -5)
    w.add("u16", U16, 60000)
    w.add("i16", I16, -300)
    w.add("u32", U32, 4_000_000_000)
    w.add("i32", I32, 123)
    w.add("neg_i32", I32, -7)
    w.add("f32", F32, 1.5)
    w.add("bool", BOOL, 1)
    w.add("s", STRING, "héllo")
    w.add("u64", U64, 2**40 + 3)
    w.add("i64", I64, 99)
    w.add("neg_i64", I64, -1)
    w.add("f64", F64, 2.25)
    w.add("ai32", ARRAY, (I32, [1, -2, 3]))
    w.add("af32", ARRAY, (F32, [0.5, 1.5]))
    w.add("astr", ARRAY, (STRING, ["a", "bc", ""]))
    w.add("au64", ARRAY, (U64, [7, 8]))  # skipped by the reference as 4 bytes/element
    w.add("after", U32, 42)
    w.add("i32", I32, 124)  # a repeated key keeps the last value
    w.add_tensor("t", [8], GT_F32, np.arange(8, dtype=np.float32))
    with open_bytes(tmp_path, w.tobytes()) as g:
        assert g.info()["version"] == 2
        assert g.info()["kv_count"] == 19
        assert g.meta_usize("u32") == 4_000_000_000
        assert g.meta_usize("u64") == 2**40 + 3
        assert g.meta_usize("i32") == 124
        assert g.meta_usize("i64") == 99
        assert g.meta_usize("after") == 42
        for key in ("u8", "i8", "u16", "i16", "neg_i32", "neg_i64", "f32", "bool", "s",
                    "ai32", "missing"):
            with pytest.raises(nx.NexusError) as ei:
                g.meta_usize(key)
            assert ei.value.code == nx.NX_ERR_NOT_FOUND
        assert g.meta_f32("f32") == 1.5
        with pytest.raises(nx.NexusError):
            g.meta_f32("f64")
        assert g.meta_str("s") == "héllo"
        with pytest.raises(nx.NexusError):
            g.meta_str("u32")
        assert g.data(g.find("t")).view(np.float32).tolist() == list(range(8))


@pytest.mark.parametrize("align,atype", [(None, None), (64, U32), (128, U64), (1, U32), (0, U32)])
def test_alignment_rule(tmp_path, align, atype):
    w = GgufWriter()
    if align is not None:
        w.add("general.alignment", atype, align)
        w.alignment = align
    w.add_tensor("a", [3], GT_F32, np.array([1, 2, 3], np.float32))
    w.add_tensor("b", [5], GT_F32, np.arange(5, dtype=np.float32) * 2)
    data = w.tobytes()
    with open_bytes(tmp_path, data) as g:
        a = 32 if align is None else max(align, 1)
        assert g.info()["alignment"] == a
        assert g.info()["data_offset"] % a == 0
        assert g.data(g.find("a")).view(np.float32).tolist() == [1, 2, 3]
        assert g.data(g.find("b")).view(np.float32).tolist() == [0, 2, 4, 6, 8]


def test_alignment_of_other_type_is_ignored(tmp_path):
    w = GgufWriter()
    w.add("general.alignment", I32, 64)  # not U32/U64: default 32
    w.add_tensor("a", [4], GT_F32, np.ones(4, np.float32))
    with open_bytes(tmp_path, w.tobytes()) as g:
        assert g.info()["alignment"] == 32


def test_tensor_lookup_and_payload_bounds(tmp_path):
    w = GgufWriter()
    q = oracle.quantize(oracle.Q8_0, np.linspace(-1, 1, 64, dtype=np.float32))
    w.add_tensor("q", [64], GT_Q8_0, q)
    data = w.tobytes()
    with open_bytes(tmp_path, data) as g:
        t = g.tensor(g.find("q"))
        assert t["bytes"] == 68 and t["type"] == GT_Q8_0
        np.testing.assert_array_equal(g.data(g.find("q")), q)
        with pytest.raises(nx.NexusError) as ei:
            g.find("nope")
        assert str(ei.value) == "Missing tensor: nope"
    with open_bytes(tmp_path, data[:-10], "short.gguf") as g:
        with pytest.raises(nx.NexusError) as ei:
            g.data(g.find("q"))
        assert ei.value.code == nx.NX_ERR_TRUNCATED


def moe_file(fmt, E, H, F, layer=0, naming="merged", shared_F=0, seed=0):
    rng = np.random.default_rng(seed)
    w = GgufWriter()
    w.add("general.architecture", STRING, "mixtral")
    w.add("mixtral.expert_count", U32, E)
    pays = {}
    gt = {oracle.Q4_K: GT_Q4_K, oracle.Q8_0: GT_Q8_0, oracle.Q4_0: GT_Q4_0, oracle.Q2_K: 10,
          0: GT_F32}[fmt]

    def mat(rows, cols):
        m = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        return oracle.quantize(fmt, m) if fmt else m.ravel().view(np.uint8)

    roles = ("ffn_gate", "ffn_up", "ffn_down")
    hf = ("w1", "w3", "w2")
    for r in range(3):
        rows, cols = (F, H) if r < 2 else (H, F)
        per = [mat(rows, cols) for _ in range(E)]
        for e in range(E):
            pays[(e, r)] = per[e]
        if naming == "merged":
            w.add_tensor(f"blk.{layer}.{roles[r]}_exps.weight", [cols, rows, E], gt,
                         np.concatenate(per))
        elif naming == "gguf":
            for e in range(E):
                w.add_tensor(f"blk.{layer}.{roles[r]}.{e}.weight", [cols, rows], gt, per[e])
        else:
            for e in range(E):
                w.add_tensor(f"model.layers.{layer}.block_sparse_moe.experts.{e}.{hf[r]}.weight",
                             [cols, rows], gt, per[e])
        if shared_F:
            srows, scols = (shared_F, H) if r < 2 else (H, shared_F)
            pays[("s", r)] = mat(srows, scols)
            w.add_tensor(f"blk.{layer}.{roles[r]}_shexp.weight", [scols, srows], gt, pays[("s", r)])
    router = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    w.add_tensor(f"blk.{layer}.ffn_gate_inp.weight", [H, E], GT_F32, router)
    return w, pays, router


@pytest.mark.parametrize("naming", ["merged", "gguf", "hf"])
def test_moe_info(tmp_path, naming):
    w, _, _ = moe_file(oracle.Q8_0, 4, 64, 96, layer=3, naming=naming, shared_F=32 if naming != "hf" else 0)
    with open_bytes(tmp_path, w.tobytes()) as g:
        info = g.moe_info(3)
        assert info == {"fmt": GT_Q8_0, "experts": 4, "hidden": 64, "ffn": 96,
                        "shared_ffn": 32 if naming != "hf" else 0}
        with pytest.raises(nx.NexusError) as ei:
            g.moe_info(2)
        assert ei.value.code == nx.NX_ERR_NOT_FOUND


def test_moe_info_rejects_inconsistent_layers(tmp_path):
    w, _, _ = moe_file(oracle.Q8_0, 2, 64, 96)
    w.tensors = [t for t in w.tensors if "ffn_down" not in t[0]]
    w.add_tensor("blk.0.ffn_down_exps.weight", [96, 32, 2], GT_Q8_0, np.zeros(2 * 32 * 3 * 34, np.uint8))
    with open_bytes(tmp_path, w.tobytes()) as g:
        with pytest.raises(nx.NexusError) as ei:
            g.moe_info(0)
        assert ei.value.code == nx.NX_ERR_SHAPE
    # F16 experts are resident-capable; Q5_0 (type 6, 22 B per 32) is not
    w2 = GgufWriter()
    for r in ("ffn_gate", "ffn_up"):
        w2.add_tensor(f"blk.0.{r}_exps.weight", [64, 96, 2], GT_F16, np.zeros(2 * 64 * 96, np.float16))
    w2.add_tensor("blk.0.ffn_down_exps.weight", [96, 64, 2], GT_F16, np.zeros(2 * 64 * 96, np.float16))
    with open_bytes(tmp_path, w2.tobytes(), "f16.gguf") as g:
        assert g.moe_info(0)["fmt"] == GT_F16
    w3 = GgufWriter()
    for r in ("ffn_gate", "ffn_up"):
        w3.add_tensor(f"blk.0.{r}_exps.weight", [64, 96, 2], 6, np.zeros(2 * 64 * 96 // 32 * 22, np.uint8))
    w3.add_tensor("blk.0.ffn_down_exps.weight", [96, 64, 2], 6, np.zeros(2 * 64 * 96 // 32 * 22, np.uint8))
    with open_bytes(tmp_path, w3.tobytes(), "q5_0.gguf") as g:
        with pytest.raises(nx.NexusError) as ei:
            g.moe_info(0)
        assert ei.value.code == nx.NX_ERR_UNSUPPORTED


@pytest.mark.parametrize("gate_dims", [[], [64]])
def test_moe_info_rejects_per_expert_tensors_without_two_dims(tmp_path, gate_dims):
    """An untrusted file may give a per-expert tensor fewer dims than a
    matrix has: an error, never a read past the dims it declared."""
    w, _, _ = moe_file(oracle.Q8_0, 2, 64, 96, naming="gguf")
    w.tensors = [(n, gate_dims if n == "blk.0.ffn_gate.0.weight" else d, t, p)
                 for n, d, t, p in w.tensors]
    with open_bytes(tmp_path, w.tobytes()) as g:
        with pytest.raises(nx.NexusError, match="fewer than 2 dims") as ei:
            g.moe_info(0)
        assert ei.value.code == nx.NX_ERR_SHAPE


def ggml_q4k_dequant(blocks: np.ndarray) -> np.ndarray:
    """Upstream ggml's Q4_K block dequantization (per 64 elements j: the 32
    code bytes at 32j hold elements 64j..64j+31 in their low nibbles and
    64j+32..64j+63 in their high nibbles; sub-block = element / 32), values
    rounded once to f32."""
    blocks = blocks.reshape(-1, 144)
    out = np.empty((blocks.shape[0], 256), np.float32)
    for b, blk in enumerate(blocks):
        d = float(oracle.f16_to_f32(blk[0:2].view(np.uint16))[0])
        dmin = float(oracle.f16_to_f32(blk[2:4].view(np.uint16))[0])
        sc, mn = oracle.unpack_q4k_scales(blk[4:16])
        qs = blk[16:144]
        for j in range(4):
            for l in range(64):
                byte = int(qs[32 * j + (l % 32)])
                q = (byte & 15) if l < 32 else (byte >> 4)
                s = 2 * j + (l >= 32)
                out[b, 64 * j + l] = np.float32(d * float(sc[s]) * q - dmin * float(mn[s]))
    return out.ravel()


def test_q4k_ggml_order_conversion():
    rng = np.random.default_rng(5)
    src = oracle.quantize(oracle.Q4_K, (rng.standard_normal(4 * 256) * 0.1).astype(np.float32))
    src = src.copy()
    src[16:144] = rng.integers(0, 256, 128, dtype=np.uint8)  # arbitrary codes in block 0
    conv = nx.q4k_from_ggml(src)
    np.testing.assert_array_equal(conv.reshape(-1, 144)[:, :16], src.reshape(-1, 144)[:, :16])
    got = oracle.dequantize(oracle.Q4_K, conv, 4 * 256)
    want = ggml_q4k_dequant(src)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", range(4))
def test_corrupt_files_error_or_parse(tmp_path, seed):
    """A valid MoE file, truncated at random lengths or with random bytes
    changed in its header, metadata and tensor table: every open, lookup and
    payload access either works or raises NexusError -- never reads outside
    the mapping (the CPU suite also runs under the host-sanitizer build)."""
    rng = np.random.default_rng(seed)
    w, _, _ = moe_file(oracle.Q8_0, 2, 64, 96, naming="gguf", shared_F=32)
    good = w.tobytes()
    head = len(good) - sum(len(t[3]) for t in w.tensors)  # header, metadata, tensor table
    for case in range(60):
        data = bytearray(good)
        if case % 3 == 0:
            data = data[: int(rng.integers(0, len(good)))]
        else:
            for _ in range(int(rng.integers(1, 6))):
                i = int(rng.integers(0, head))
                data[i] = int(rng.integers(0, 256))
        p = tmp_path / f"c{case}.gguf"
        p.write_bytes(bytes(data))
        try:
            g = nx.Gguf(str(p))
        except nx.NexusError:
            continue
        try:
            for t in g.tensors():
                try:
                    g.data(g.find(t["name"]))
                except nx.NexusError:
                    pass
            for layer in (0, 1):
                try:
                    g.moe_info(layer)
                except nx.NexusError:
                    pass
        finally:
            g.close()
