"""Seeded MoE layer cases shared by the parity tests.

Weights ~N(0, 0.02) quantized with the oracle's restatement of the reference
quantizer, activations ~N(0, 1), router logits = x . W_r with W_r ~N(0, 0.02)
(accumulated in float64, rounded to f32; the same logits feed both sides).
"""
from __future__ import annotations

import numpy as np

import oracle

F32, Q4_0, Q8_0, Q4_K, Q2_K, F16, BF16 = 0, 2, 8, 12, 10, 1, 28


def half_payload(fmt, w) -> np.ndarray:
    """F16 (IEEE round to nearest even, numpy) or BF16 (round to nearest even
    on the f32 bits) payload bytes of w."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    if fmt == F16:
        return w.astype(np.float16).view(np.uint8)
    b = w.view(np.uint32).astype(np.uint64)
    h = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return h.view(np.uint8)


def payload_of(fmt, w) -> np.ndarray:
    if fmt == F32:
        return np.ascontiguousarray(w, np.float32).ravel().view(np.uint8)
    if fmt in (F16, BF16):
        return half_payload(fmt, w)
    return oracle.quantize(fmt, w)


class Layer:
    def __init__(self, fmt, E, H, F, k, T, seed, shared_F=0, score_mode=0, zipf=None,
                 experts_needed=None):
        self.fmt, self.E, self.H, self.F, self.k, self.T = fmt, E, H, F, k, T
        self.score_mode = score_mode
        self.shared_F = shared_F
        rng = np.random.default_rng(seed)
        self.x = rng.standard_normal((T, H)).astype(np.float32)
        rw = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        lg = self.x.astype(np.float64) @ rw.T.astype(np.float64)
        if zipf is not None:  # expert popularity ~ Zipf(s): logit_e += ln p_e
            p = 1.0 / np.arange(1, E + 1) ** zipf
            lg = lg + np.log(p / p.sum())[None, :]
        self.logits = lg.astype(np.float32)
        ex, _, cnt, _ = oracle.route(self.logits, T, E, k, score_mode)
        self.routed = sorted({int(e) for t in range(T) for e in ex[t, :cnt[t]]})
        need = set(self.routed) if experts_needed is None else set(experts_needed)
        # payloads for every expert (device needs all); f32 copies only for routed ones
        self.payload = {}
        self.dense = {}
        wseed = rng.integers(0, 2**63)
        for e in range(E):
            for role, shape in ((0, (F, H)), (1, (F, H)), (2, (H, F))):
                r2 = np.random.default_rng([int(wseed), e, role])
                w = (r2.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
                q = payload_of(fmt, w)
                self.payload[(e, role)] = q
                if e in need:
                    self.dense[(e, role)] = (oracle.dequantize(fmt, q, w.size) if fmt != F32
                                             else w.ravel())
        self.shared_payload = None
        self.shared_dense = None
        if shared_F:
            r2 = np.random.default_rng([int(wseed), 10**6])
            mats = []
            pays = []
            for shape in ((shared_F, H), (shared_F, H), (H, shared_F)):
                w = (r2.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
                q = payload_of(fmt, w)
                pays.append(q)
                mats.append(oracle.dequantize(fmt, q, w.size) if fmt != F32 else w.ravel())
            self.shared_payload = pays
            self.shared_dense = mats

    def oracle_out(self, nthreads=None):
        g = [self.dense.get((e, 0)) for e in range(self.E)]
        u = [self.dense.get((e, 1)) for e in range(self.E)]
        d = [self.dense.get((e, 2)) for e in range(self.E)]
        if all(m is None for m in g):
            return np.zeros((self.T, self.H), np.float32)
        return oracle.moe_layer(self.x, self.logits, g, u, d, self.k, self.score_mode,
                                shared=self.shared_dense, nthreads=nthreads)

    def upload(self, nx, ctx):
        ex = nx.Experts(ctx, self.fmt, self.E, self.H, self.F, self.shared_F)
        for (e, role), q in self.payload.items():
            ex.load(e, role, q)
        if self.shared_payload is not None:
            for role, q in enumerate(self.shared_payload):
                ex.load(nx.EXPERT_SHARED, role, q)
        return ex


def rel_l2(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def assert_same_bits(got, ref):
    """Bit-for-bit equality of every non-NaN value and identical NaN positions.
    NaN payloads are not compared: x86 and gfx950 differ in the payload they
    give an invalid operation (x86's default NaN has the sign bit set)."""
    got = np.asarray(got, np.float32).ravel()
    ref = np.asarray(ref, np.float32).ravel()
    assert got.shape == ref.shape
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN positions differ at {np.nonzero(gn != rn)[0][:8]}"
    bad = np.nonzero(got[~gn].view(np.uint32) != ref[~rn].view(np.uint32))[0]
    assert bad.size == 0, (f"{bad.size} values differ; first at {bad[:4]}: "
                           f"{got[~gn][bad[:4]]} vs {ref[~rn][bad[:4]]}")


class DeviceArray:
    """float32 device buffer allocated through the same HIP runtime that
    libnexus_hip.so links (/opt/rocm's libamdhip64), for tests of the *_dev
    entry points.  (torch bundles its own HIP runtime, which cannot start once
    another runtime in the process holds the GPU.)"""

    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            import ctypes as C
            h = C.CDLL("libamdhip64.so.7")
            h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
            h.hipFree.argtypes = [C.c_void_p]
            h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            h.hipDeviceSynchronize.argtypes = []
            cls._hip = h
        return cls._hip

    def __init__(self, n: int, fill=None):
        import ctypes as C
        self.n = n
        p = C.c_void_p()
        assert self.hip().hipMalloc(C.byref(p), max(n, 1) * 4) == 0
        self.ptr = p.value
        if fill is not None:
            self.upload(np.full(n, fill, np.float32))

    def upload(self, a, offset: int = 0):
        a = np.ascontiguousarray(a, np.float32).ravel()
        assert offset + a.size <= self.n
        assert self.hip().hipMemcpy(self.ptr + 4 * offset, a.ctypes.data, a.nbytes, 1) == 0

    def download(self) -> np.ndarray:
        out = np.empty(self.n, np.float32)
        assert self.hip().hipDeviceSynchronize() == 0
        assert self.hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2) == 0
        return out

    def __del__(self):
        try:
            self.hip().hipFree(self.ptr)
        except Exception:
            pass
