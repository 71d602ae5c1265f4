"""Pins the oracle's f16 conversions, quantizers and dequantizers.

Anchors: the reference's own tests (src/gguf/mod.rs:1681-1714,
src/quant/mod.rs:1287-1325), numpy's IEEE float16 conversion, and an
independent vectorised numpy statement of the GGUF block layouts
(src/quant/mod.rs:689-849), exercised on crafted blocks that cover every
6-bit scale/min value, every 4-bit code and subnormal f16 scales.
"""
import numpy as np
import pytest

Q4_0, Q8_0, Q4_K, Q2_K = 2, 8, 12, 10


# ----------------------------------------------------------------------------- f16
def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = oracle.f16_to_f32(bits)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = raw.view(np.float32)
    # every f16 value and every midpoint between neighbours (ties-to-even cases)
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 65536, 1e-8, 2.98e-8, 2.9802322e-8, 5.96e-8,
                     6.1035156e-05, 6.1e-05, 0.0, -0.0, np.inf, -np.inf], np.float32)
    x = np.concatenate([x, h.astype(np.float32), mids, -mids, edge])
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16(x)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r}"


# ----------------------------------------------------------------------------- known answers
def test_q8_0_known_answer(oracle):
    """src/gguf/mod.rs:1681-1695: scale f16(0.5), q = i - 16."""
    scale = np.array([0.5], np.float32).astype(np.float16).view(np.uint8)
    block = np.concatenate([scale, (np.arange(32) - 16).astype(np.int8).view(np.uint8)])
    v = oracle.dequantize(Q8_0, block, 32)
    assert v.size == 32
    assert v[0] == -8.0 and v[16] == 0.0 and v[31] == 7.5


@pytest.mark.parametrize("fmt,tol,n", [(Q8_0, 0.03, 64), (Q4_0, 0.3, 64), (Q4_K, 0.4, 300)])
def test_reference_roundtrip_tolerances(oracle, fmt, tol, n):
    """src/quant/mod.rs:1287-1325 (Q8_0 / Q4_0 on i/16-2, Q4_K on i/31-4)."""
    if fmt == Q4_K:
        data = np.arange(n, dtype=np.float32) / np.float32(31.0) - np.float32(4.0)
    else:
        data = np.arange(n, dtype=np.float32) / np.float32(16.0) - np.float32(2.0)
    q = oracle.quantize(fmt, data)
    if fmt == Q4_K:
        assert q.size == (n + 255) // 256 * 144  # src/quant/mod.rs:1318
    dec = oracle.dequantize(fmt, q, n)
    assert dec.size == n
    assert np.all(np.abs(dec - data) < tol)


def test_q4_k_ramp_sizes_match_gguf_test(oracle):
    """src/gguf/mod.rs:1697-1714: Q4_K payload size and decoded length."""
    data = np.arange(300, dtype=np.float32) / np.float32(31.0) - np.float32(4.0)
    q = oracle.quantize(Q4_K, data)
    assert q.size == 2 * 144
    assert oracle.dequantize(Q4_K, q, 300).size == 300


# ----------------------------------------------------------------------------- layouts
def np_dequant(fmt, data, n):
    """Independent vectorised statement of the three block layouts."""
    f16 = lambda b: b.copy().view(np.float16).astype(np.float32).ravel()  # noqa: E731
    np.seterr(invalid="ignore", over="ignore")
    if fmt == Q8_0:
        b = data.reshape(-1, 34)
        d = f16(b[:, 0:2])
        v = b[:, 2:].view(np.int8).astype(np.float32) * d[:, None]
    elif fmt == Q4_0:
        b = data.reshape(-1, 18)
        d = f16(b[:, 0:2])
        qs = b[:, 2:]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int16) - 8
        v = q.astype(np.float32) * d[:, None]
    elif fmt == Q2_K:
        b = data.reshape(-1, 84)
        d, dmin = f16(b[:, 80:82]), f16(b[:, 82:84])
        qs = b[:, 16:80]
        q = np.stack([(qs >> (2 * j)) & 3 for j in range(4)], axis=2).reshape(-1, 256)  # i = 4B + j
        sub = np.arange(256) // 16
        sc = (b[:, 0:16] & 15).astype(np.float32)[:, sub]
        mn = (b[:, 0:16] >> 4).astype(np.float32)[:, sub]
        v = (d[:, None] * sc) * q.astype(np.float32) - dmin[:, None] * mn
    else:
        b = data.reshape(-1, 144)
        d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
        p = b[:, 4:16]
        sc = np.concatenate([p[:, 0:4] & 63, (p[:, 8:12] & 15) | ((p[:, 0:4] >> 6) << 4)], axis=1)
        mn = np.concatenate([p[:, 4:8] & 63, (p[:, 8:12] >> 4) | ((p[:, 4:8] >> 6) << 4)], axis=1)
        qs = b[:, 16:]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32)  # element i, i+128
        sub = np.arange(256) // 32
        v = (d[:, None] * sc[:, sub].astype(np.float32)) * q - dmin[:, None] * mn[:, sub].astype(
            np.float32)
    return v.ravel()[:n]


def crafted_blocks(fmt, nblocks, seed):
    rng = np.random.default_rng(seed)
    bs = {Q8_0: 34, Q4_0: 18, Q4_K: 144, Q2_K: 84}[fmt]
    data = rng.integers(0, 256, size=(nblocks, bs), dtype=np.uint8)
    # scales: normal, subnormal, zero, negative zero, largest finite
    special = np.array([0x3C00, 0x0001, 0x03FF, 0x0000, 0x8000, 0x7BFF, 0x2E66, 0x8123],
                       np.uint16)
    if fmt == Q2_K:  # f16 d, dmin at bytes 80..83; every scale/min nibble pair in byte 0..15
        for off, shift in ((80, 0), (82, 3)):
            h = data[:, off:off + 2].copy().view(np.uint16).ravel()
            h[: nblocks // 2] = special[(np.arange(nblocks // 2) + shift) % special.size]
            data[:, off:off + 2] = h.view(np.uint8).reshape(-1, 2)
        for b in range(min(nblocks, 16)):
            data[b, 0:16] = (np.arange(16, dtype=np.uint8) * 16 + b) & 255
        return data.ravel()
    hdr = data[:, 0:2].copy().view(np.uint16).ravel()
    hdr[: nblocks // 2] = special[np.arange(nblocks // 2) % special.size]
    data[:, 0:2] = hdr.view(np.uint8).reshape(-1, 2)
    if fmt == Q4_K:
        dm = data[:, 2:4].copy().view(np.uint16).ravel()
        dm[: nblocks // 2] = special[(np.arange(nblocks // 2) + 3) % special.size]
        data[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
        # walk every 6-bit scale/min value through every sub-block slot
        for b in range(min(nblocks, 64)):
            sc = np.full(8, b, np.uint8)
            mn = np.full(8, 63 - b, np.uint8)
            data[b, 4:16] = (np.array(
                [(sc[i] & 63) | ((sc[i + 4] >> 4) << 6) for i in range(4)] +
                [(mn[i] & 63) | ((mn[i + 4] >> 4) << 6) for i in range(4)] +
                [(sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4) for i in range(4)], np.uint8))
    return data.ravel()


@pytest.mark.parametrize("fmt", [Q8_0, Q4_0, Q4_K])
def test_dequant_matches_layout_statement(oracle, fmt):
    blk = {Q8_0: 32, Q4_0: 32, Q4_K: 256}[fmt]
    data = crafted_blocks(fmt, 256, seed=fmt)
    n = 256 * blk
    got = oracle.dequantize(fmt, data, n)
    ref = np_dequant(fmt, data, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # output_len stops mid-block; a ragged byte tail is dropped like chunks_exact
    got2 = oracle.dequantize(fmt, data[: data.size - 5], n - 7)
    assert got2.size == (255 * blk if blk * 255 < n - 7 else n - 7)
    assert np.array_equal(got2.view(np.uint32), ref[: got2.size].view(np.uint32))


def test_q4k_every_code_and_scale(oracle):
    """Brute force: every (sc, m) in [0,63]^2 and q in [0,15] for d = dmin = 1 and
    for subnormal d/dmin: value = d*sc*q - dmin*m (products exact in f32)."""
    for d_bits, m_bits in [(0x3C00, 0x3C00), (0x0001, 0x0003), (0x7BFF, 0x0400)]:
        d = np.uint16(d_bits).view(np.float16).astype(np.float64)
        dm = np.uint16(m_bits).view(np.float16).astype(np.float64)
        blocks = []
        expect = []
        for s in range(64):
            sc = np.full(8, s, np.uint8)
            mn = (np.arange(8, dtype=np.uint8) * 9 + s) % 64
            packed = oracle.pack_q4k_scales(sc, mn)
            s2, m2 = oracle.unpack_q4k_scales(packed)
            assert np.array_equal(s2, sc) and np.array_equal(m2, mn)
            qs = (np.arange(128) % 16 | ((np.arange(128) * 7 % 16) << 4)).astype(np.uint8)
            hdr = np.array([d_bits, m_bits], np.uint16).view(np.uint8)
            blocks.append(np.concatenate([hdr, packed, qs]))
            q = np.concatenate([qs & 15, qs >> 4]).astype(np.float64)
            sub = np.arange(256) // 32
            exact = d * sc[sub] * q - dm * mn[sub]
            expect.append(exact.astype(np.float32))  # one rounding of the exact value
        got = oracle.dequantize(Q4_K, np.concatenate(blocks), 64 * 256)
        assert np.array_equal(got, np.concatenate(expect))


def test_scale_pack_roundtrip_all_values(oracle):
    for s in range(64):
        for m in range(0, 64, 7):
            sc = (np.arange(8) * 5 + s) % 64
            mn = (np.arange(8) * 3 + m) % 64
            s2, m2 = oracle.unpack_q4k_scales(oracle.pack_q4k_scales(sc, mn))
            assert np.array_equal(s2, sc) and np.array_equal(m2, mn)


# ----------------------------------------------------------------------------- quantizers
@pytest.mark.parametrize("fmt", [Q8_0, Q4_0, Q4_K])
def test_quantizer_error_bounds(oracle, fmt):
    """|x - dq(q(x))| stays within each format's step bound on N(0, 0.02) data."""
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    q = oracle.quantize(fmt, x)
    dq = oracle.dequantize(fmt, q, x.size)
    blk = {Q8_0: 32, Q4_0: 32, Q4_K: 256}[fmt]
    xb = x.reshape(-1, blk)
    err = np.abs(dq - x).reshape(-1, blk)
    amax = np.abs(xb).max(axis=1, keepdims=True)
    if fmt == Q8_0:
        bound = amax / 127 * 0.5 * 1.01 + amax * 2.0**-11
    elif fmt == Q4_0:
        bound = amax / 7 * 0.5 * 1.01 + amax * 2.0**-11 * 8
    else:
        bound = (xb.max(axis=1, keepdims=True) - xb.min(axis=1, keepdims=True)) / 15 * 1.2
    assert np.all(err <= bound)


def test_quantizer_thread_invariance(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256 * 97) * 0.02).astype(np.float32)
    for fmt in (Q8_0, Q4_0, Q4_K):
        a = oracle.quantize(fmt, x, nthreads=1)
        b = oracle.quantize(fmt, x, nthreads=7)
        assert np.array_equal(a, b)


def test_q8_0_hand_block(oracle):
    """One block worked by hand: x = (i-16)/2 -> max 8, scale 8/127 (f32), q = round(x/scale)."""
    x = ((np.arange(32) - 16) * 0.5).astype(np.float32)
    q = oracle.quantize(Q8_0, x)
    scale32 = np.float32(8.0) / np.float32(127.0)
    assert q[0:2].view(np.uint16)[0] == np.float32(scale32).astype(np.float16).view(np.uint16)
    codes = q[2:].view(np.int8).astype(np.int32)
    expect = [int(np.sign(v) * np.floor(abs(v) + 0.5)) for v in (x / scale32).astype(np.float32)]
    assert codes.tolist() == expect
    assert codes[0] == -127 and codes[16] == 0


def test_q4_k_hand_block(oracle):
    """A block whose sub-blocks are exact ramps 0..15 scaled by 2^-4: d = 1/63*(15/16)/15...
    every value must survive the round trip exactly when scales are representable."""
    x = np.zeros(256, np.float32)
    x[:] = (np.arange(256) % 16).astype(np.float32)  # each sub-block: 0..15, twice
    q = oracle.quantize(Q4_K, x)
    dq = oracle.dequantize(Q4_K, q, 256)
    # scale per sub-block = 15/15 = 1, d = 1/63 -> f16; sc = 63; offsets 0 -> dmin = 0
    d16 = np.float32(np.float32(1.0) / np.float32(63.0)).astype(np.float16).astype(np.float32)
    assert q[2:4].view(np.uint16)[0] == 0  # dmin == 0
    s, m = oracle.unpack_q4k_scales(q[4:16])
    assert s.tolist() == [63] * 8 and m.tolist() == [0] * 8
    assert np.array_equal(dq, (d16 * np.float32(63.0)) * x)


def _rust_round(v):
    """f32::round: halves away from zero."""
    v = np.float32(v)
    return np.float32(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)))


# Blocks on which the code of one element depends on whether the quantizer
# divides by the f32 d / dmin it computed or by their stored f16 roundings.
# The reference computes codes with the f32 values (src/quant/mod.rs:780-812,
# quantize_q4_k_value :1133-1141; quantize_q2_k :875-902, quantize_q2_k_value
# :1143) and only stores f16(d), f16(dmin) (:798-799, :906-907).  d is chosen as 1 + 0.75 * 2^-10,
# which f16 rounds up to 1 + 2^-10 (relative +2.4e-4), and one element sits
# just past a rounding boundary of its code by less than that.
def test_q4k_codes_use_unrounded_d(oracle):
    f = np.float32
    d_target = f(1.0 + 0.75 * 2 ** -10)
    big = f(f(d_target * f(63)) * f(15))          # sub-block 0 max: scale0 = big/15
    scale0 = f(big / f(15))
    d = f(scale0 / f(63))                          # max_scale / 63
    assert d == d_target and f(np.float16(d)) == f(1.0 + 2 ** -10)
    step = f(d * f(63))                            # scales[0] = round(scale0/d) = 63
    x1 = f(f(14.502) * step)                       # 14.502 steps above the offset 0
    x = np.zeros(256, np.float32)
    x[0], x[1] = big, x1
    q = oracle.quantize(Q4_K, x)
    sc, mn = oracle.unpack_q4k_scales(q[4:16])
    assert sc.tolist() == [63] + [0] * 7 and mn.tolist() == [0] * 8
    assert q[0:2].view(np.float16)[0] == np.float16(d)
    with_d = int(_rust_round(f(x1 / step)))                      # 15
    with_f16 = int(_rust_round(f(x1 / f(f(np.float16(d)) * f(63)))))  # 14
    assert (with_d, with_f16) == (15, 14)
    assert q[16] & 15 == 15 and q[17] & 15 == with_d


def test_q4k_codes_use_unrounded_dmin(oracle):
    f = np.float32
    m = f(f(1.0 + 0.75 * 2 ** -10) * f(63))      # sub-block 0 min is -m: offset0 = m
    top = f(900.0)
    scale0 = f(f(top + m) / f(15))
    d = f(scale0 / f(63))
    dmin = f(m / f(63))
    assert f(np.float16(dmin)) > dmin
    step = f(d * f(63))
    off = f(dmin * f(63))                          # mins[0] = 63
    y = f(f(f(7.5 - 0.0001) * step) - off)         # (y + offset)/scale = 7.4999
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2] = -m, y, top
    q = oracle.quantize(Q4_K, x)
    sc, mn = oracle.unpack_q4k_scales(q[4:16])
    assert sc[0] == 63 and mn[0] == 63
    with_dmin = int(_rust_round(f(f(y + off) / step)))
    with_f16 = int(_rust_round(f(f(y + f(f(np.float16(dmin)) * f(63))) / step)))
    assert (with_dmin, with_f16) == (7, 8)
    assert [q[16] & 15, q[17] & 15, q[18] & 15] == [0, with_dmin, 15]


def test_q2k_codes_use_unrounded_d_and_dmin(oracle):
    f = np.float32
    # d: sub-block 0 = {big, x1, 0 ...}; scale0 = big/3, d = scale0/15
    big = f(f(f(1.0 + 0.75 * 2 ** -10) * f(15)) * f(3))
    d = f(f(big / f(3)) / f(15))
    step = f(d * f(15))
    x1 = f(f(1.5001) * step)
    x = np.zeros(256, np.float32)
    x[0], x[1] = big, x1
    q = oracle.quantize(Q2_K, x)
    assert q[0] & 15 == 15 and q[80:82].view(np.float16)[0] == np.float16(d)
    with_d = int(_rust_round(f(x1 / step)))
    with_f16 = int(_rust_round(f(x1 / f(f(np.float16(d)) * f(15)))))
    assert (with_d, with_f16) == (2, 1)
    assert [q[16] & 3, (q[16] >> 2) & 3] == [3, with_d]
    # dmin: sub-block 0 = {-m, y, top}
    m = f(f(1.0 + 0.75 * 2 ** -10) * f(15))
    top = f(40.0)
    d = f(f(f(top + m) / f(3)) / f(15))
    dmin = f(m / f(15))
    step = f(d * f(15))
    off = f(dmin * f(15))
    y = f(f(f(1.5 - 0.0001) * step) - off)
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2] = -m, y, top
    q = oracle.quantize(Q2_K, x)
    assert q[0] & 15 == 15 and q[0] >> 4 == 15
    with_dmin = int(_rust_round(f(f(y + off) / step)))
    with_f16 = int(_rust_round(f(f(y + f(f(np.float16(dmin)) * f(15))) / step)))
    assert (with_dmin, with_f16) == (1, 2)
    assert [q[16] & 3, (q[16] >> 2) & 3, (q[16] >> 4) & 3] == [0, with_dmin, 3]


# ----------------------------------------------------------------------------- Q2_K
def test_q2k_reference_roundtrip(oracle):
    # src/quant/mod.rs:1327-1338 and src/gguf/mod.rs:1697-1714
    data = (np.arange(300, dtype=np.float32) / np.float32(31.0) - np.float32(4.0)).astype(np.float32)
    q = oracle.quantize(Q2_K, data)
    assert q.size == 2 * 84
    dq = oracle.dequantize(Q2_K, q, 300)
    assert dq.size == 300
    assert np.all(np.abs(dq - data) < 1.6)


def test_q2k_dequant_matches_layout_statement(oracle):
    data = crafted_blocks(Q2_K, 128, seed=10)
    n = 128 * 256
    got = oracle.dequantize(Q2_K, data, n)
    ref = np_dequant(Q2_K, data, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got2 = oracle.dequantize(Q2_K, data[: data.size - 5], n - 9)
    assert got2.size == 127 * 256
    assert np.array_equal(got2.view(np.uint32), ref[: got2.size].view(np.uint32))


def test_q2k_quantizer_invariants(oracle):
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(64 * 256) * np.exp(rng.uniform(-4, 2, 64 * 256))).astype(np.float32)
    x[:256] = 0.0                                   # an all-zero block
    x[256:512] = np.abs(x[256:512])                 # a block without negatives: mins 0
    x[512:528] = 7.0                                # a constant sub-block
    q = oracle.quantize(Q2_K, x).reshape(-1, 84)
    assert np.all(q[0] == 0)
    assert np.all((q[1, :16] >> 4) == 0)
    dq = oracle.dequantize(Q2_K, q.ravel(), x.size).reshape(-1, 256)
    xb = x.reshape(-1, 256)
    # each value lies within its sub-block's step of the reconstruction grid:
    # |x - x'| <= 2 * max over the block of (sub-block range / 3) + rounding
    sub = xb.reshape(-1, 16, 16)
    span = (sub.max(axis=2) - np.minimum(sub.min(axis=2), 0)).max(axis=1)
    err = np.abs(dq - xb).max(axis=1)
    assert np.all(err <= span * (2.0 / 3.0) + 1e-30 + span * 0.2)


def test_q2k_hand_worked_block(oracle):
    # sub-block s holds 16 values s/4 + (i%4)/4 (max 4.5 at s=15): offset 0,
    # scale (max)/3; d = max_scale/15; every scale nibble rounds from
    # scale/d; codes round (v / (d * sc)) into 0..3.  Rust's f32::round
    # rounds halves away from zero (2.5 -> 3, 12.5 -> 13), unlike np.round.
    rnd = lambda v: np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))  # noqa: E731
    x = np.array([s / 4 + (i % 4) / 4 for s in range(16) for i in range(16)], np.float32)
    q = oracle.quantize(Q2_K, x)
    sc = np.array([(x[16 * s:16 * s + 16].max()) / np.float32(3.0) for s in range(16)], np.float32)
    d = np.float32(sc.max() / np.float32(15.0))
    d16 = np.float16(d).astype(np.float32)
    assert q[80:82].view(np.float16)[0] == np.float16(d)
    assert q[82:84].view(np.uint16)[0] == 0               # dmin = 0
    sq = np.clip(rnd(sc / d), 1, 15).astype(np.uint8)
    sq[sc == 0] = 0
    np.testing.assert_array_equal(q[:16] & 15, sq)
    np.testing.assert_array_equal(q[:16] >> 4, 0)
    codes = np.stack([(q[16:80] >> (2 * j)) & 3 for j in range(4)], axis=1).ravel()
    step = (d * sq.astype(np.float32)).astype(np.float32)[np.arange(256) // 16]
    want = np.where(step > 0, np.clip(rnd(x / np.where(step > 0, step, 1)), 0, 3), 0)
    np.testing.assert_array_equal(codes, want.astype(np.uint8))
    assert d16 > 0


# ------------------------------------------------------------------ F16 / BF16
def test_f16_dequant_every_pattern(oracle):
    """F16 (src/gguf/mod.rs:921-933, half::f16::to_f32) on all 65536 bit
    patterns equals numpy's independent float16 -> float32 conversion."""
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.dequantize(oracle.F16, bits.view(np.uint8), 65536)
    want = bits.view(np.float16).astype(np.float32)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn)
    np.testing.assert_array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32))
    assert oracle.quant_bytes(oracle.F16, 77) == 154


def test_bf16_dequant_known_values_and_round_trip(oracle):
    """BF16 (src/gguf/mod.rs:934-946): known encodings, and every f32 whose low
    16 bits are zero comes back exactly from its top half."""
    cases = {0x3F80: 1.0, 0xC000: -2.0, 0x4049: 3.140625, 0x0000: 0.0, 0x8000: -0.0,
             0x7F80: np.inf, 0xFF80: -np.inf, 0x0001: 2.0 ** -133, 0x0080: 2.0 ** -126,
             0x7F7F: 3.3895313892515355e38}
    bits = np.array(list(cases), np.uint16)
    got = oracle.dequantize(oracle.BF16, bits.view(np.uint8), bits.size)
    for b, g in zip(cases, got):
        assert g == np.float32(cases[b]) and np.signbit(g) == np.signbit(np.float32(cases[b])), hex(b)
    assert np.isnan(oracle.dequantize(oracle.BF16, np.array([0x7FC0], np.uint16).view(np.uint8), 1)[0])
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-30, 30, 4096)).astype(np.float32)
    x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
    top = (x.view(np.uint32) >> 16).astype(np.uint16)
    back = oracle.dequantize(oracle.BF16, top.view(np.uint8), top.size)
    np.testing.assert_array_equal(back.view(np.uint32), x.view(np.uint32))
    # a short payload gives what it holds (chunks_exact drops the ragged byte)
    assert oracle.dequantize(oracle.BF16, top.view(np.uint8)[:7], 10).size == 3
