"""CPU oracle for the Nexus MoE routed-FFN path (ctypes wrapper over nx_oracle.c).

TEST INFRASTRUCTURE ONLY: the oracle the HIP path is tested against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product package ``nexus_amd`` never imports it.

Each function restates a reference function (paths relative to the reference
repository root); see nx_oracle.c for the per-function citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# NEXUS_ORACLE_LIB points at another build (the sanitizer build,
# oracle/Makefile: liboracle_san.so)
_LIB_PATH = os.environ.get("NEXUS_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

F32, Q4_0, Q8_0, Q4_K, Q2_K, F16, BF16 = 0, 2, 8, 12, 10, 1, 28
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q2_K: (256, 84)}

_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i32p = C.POINTER(C.c_int32)
_u16p = C.POINTER(C.c_uint16)
_szp = C.POINTER(C.c_size_t)


def build() -> None:
    """Compile liboracle.so from nx_oracle.c (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.nxo_f16_to_f32.argtypes = [C.c_uint16]
        L.nxo_f16_to_f32.restype = C.c_float
        L.nxo_f32_to_f16.argtypes = [C.c_float]
        L.nxo_f32_to_f16.restype = C.c_uint16
        L.nxo_f32_to_f16_array.argtypes = [_fp, C.c_size_t, _u16p]
        L.nxo_quant_bytes.argtypes = [C.c_int, C.c_size_t]
        L.nxo_quant_bytes.restype = C.c_size_t
        L.nxo_quantize.argtypes = [C.c_int, _fp, C.c_size_t, _u8p, C.c_int]
        L.nxo_quantize.restype = C.c_size_t
        L.nxo_dequantize.argtypes = [C.c_int, _u8p, C.c_size_t, C.c_size_t, _fp, C.c_int]
        L.nxo_dequantize.restype = C.c_size_t
        L.nxo_unpack_q4k_scales.argtypes = [_u8p, _u8p, _u8p]
        L.nxo_pack_q4k_scales.argtypes = [_u8p, _u8p, _u8p]
        L.nxo_route.argtypes = [_fp, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int,
                                _i32p, _fp, _i32p]
        L.nxo_route.restype = C.c_size_t
        L.nxo_permute.argtypes = [_i32p, _i32p, C.c_size_t, C.c_size_t, C.c_size_t, _i32p, _i32p,
                                  _i32p, _i32p, _i32p]
        L.nxo_permute.restype = C.c_size_t
        L.nxo_matvec.argtypes = [_fp, C.c_size_t, C.c_size_t, C.c_size_t, _fp, C.c_size_t, _fp,
                                 C.c_char_p, C.c_size_t]
        L.nxo_matvec.restype = C.c_int
        L.nxo_rms_norm.argtypes = [_fp, _fp, C.c_size_t, C.c_float, _fp]
        L.nxo_dispatch_moe_ffn.argtypes = [_fp, C.c_size_t, _fp, C.c_size_t,
                                           C.POINTER(_fp), _szp, C.POINTER(_fp), _szp,
                                           C.POINTER(_fp), _szp, C.c_size_t, C.c_size_t,
                                           C.c_size_t, C.c_size_t, _fp, C.c_char_p, C.c_size_t]
        L.nxo_dispatch_moe_ffn.restype = C.c_int
        L.nxo_moe_layer.argtypes = [_fp, _fp, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int,
                                    C.POINTER(_fp), C.POINTER(_fp), C.POINTER(_fp), _fp, _fp, _fp,
                                    C.c_size_t, C.c_size_t, C.c_size_t, _fp, C.c_int]
        L.nxo_moe_layer.restype = C.c_int
        L.nxo_swiglu_ffn.argtypes = [_fp, C.c_size_t, _fp, _fp, _fp, C.c_size_t, C.c_size_t, _fp]
        L.nxo_cpu_matmul.argtypes = [_fp, _fp, C.c_size_t, C.c_size_t, C.c_size_t, _fp, C.c_int]
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


# --------------------------------------------------------------------------- f16
def f16_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    f = lib().nxo_f16_to_f32
    return np.array([f(int(b)) for b in bits], dtype=np.float32)


def f32_to_f16(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.empty(x.size, dtype=np.uint16)
    lib().nxo_f32_to_f16_array(_p(x, _fp), x.size, _p(out, _u16p))
    return out


# --------------------------------------------------------------------------- quant
def quant_bytes(fmt: int, n: int) -> int:
    return int(lib().nxo_quant_bytes(fmt, n))


def quantize(fmt: int, x, nthreads: int | None = None) -> np.ndarray:
    """QuantEngine::quantize_weights (src/quant/mod.rs:623-640) for one format."""
    x = _f32(x).ravel()
    out = np.empty(quant_bytes(fmt, x.size), dtype=np.uint8)
    lib().nxo_quantize(fmt, _p(x, _fp), x.size, _p(out, _u8p), nthreads or default_threads())
    return out


def dequantize(fmt: int, data, output_len: int, nthreads: int | None = None) -> np.ndarray:
    """QuantEngine::dequantize (src/quant/mod.rs:643-667) for one format; F16 and
    BF16 as GgufReader::tensor_bytes_to_f32 (src/gguf/mod.rs:921-946)."""
    data = np.ascontiguousarray(data, dtype=np.uint8).ravel()
    out = np.empty(max(output_len, 1), dtype=np.float32)
    n = lib().nxo_dequantize(fmt, _p(data, _u8p), data.size, output_len, _p(out, _fp),
                             nthreads or default_threads())
    return out[:n]


def unpack_q4k_scales(packed12) -> tuple[np.ndarray, np.ndarray]:
    p = np.ascontiguousarray(packed12, dtype=np.uint8)
    s = np.empty(8, np.uint8)
    m = np.empty(8, np.uint8)
    lib().nxo_unpack_q4k_scales(_p(p, _u8p), _p(s, _u8p), _p(m, _u8p))
    return s, m


def pack_q4k_scales(scales, mins) -> np.ndarray:
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    m = np.ascontiguousarray(mins, dtype=np.uint8)
    out = np.empty(12, np.uint8)
    lib().nxo_pack_q4k_scales(_p(s, _u8p), _p(m, _u8p), _p(out, _u8p))
    return out


# --------------------------------------------------------------------------- router
def route(logits, num_tokens: int, num_experts: int, top_k: int, score_mode: int = 0):
    """route_moe_experts (src/engine/mod.rs:918-966).

    Returns (experts[T,k] int32 padded with -1, weights[T,k] f32, counts[T],
    lists_produced)."""
    lg = _f32(logits).ravel()
    ex = np.full((max(num_tokens, 1), max(top_k, 1)), -1, np.int32)
    w = np.zeros((max(num_tokens, 1), max(top_k, 1)), np.float32)
    cnt = np.zeros(max(num_tokens, 1), np.int32)
    n = lib().nxo_route(_p(lg, _fp), lg.size, num_tokens, num_experts, top_k, score_mode,
                        _p(ex, _i32p), _p(w, _fp), _p(cnt, _i32p))
    return ex[:num_tokens, :top_k], w[:num_tokens, :top_k], cnt[:num_tokens], int(n)


def permute(experts, counts, num_experts: int):
    """Stable counting sort of (token, slot) pairs by expert."""
    ex = np.ascontiguousarray(experts, dtype=np.int32)
    cnt = np.ascontiguousarray(counts, dtype=np.int32)
    T, k = ex.shape
    P = max(int(cnt.sum()), 1)
    ec = np.zeros(max(num_experts, 1), np.int32)
    off = np.zeros(num_experts + 1, np.int32)
    pt = np.full(P, -1, np.int32)
    ps = np.full(P, -1, np.int32)
    inv = np.full((max(T, 1), max(k, 1)), -1, np.int32)
    lib().nxo_permute(_p(ex, _i32p), _p(cnt, _i32p), T, k, num_experts, _p(ec, _i32p),
                      _p(off, _i32p), _p(pt, _i32p), _p(ps, _i32p), _p(inv, _i32p))
    n = int(off[-1])
    return ec[:num_experts], off, pt[:n], ps[:n], inv[:T, :k]


# --------------------------------------------------------------------------- engine
class OracleError(RuntimeError):
    pass


def rms_norm(x, w, eps: float) -> np.ndarray:
    """kernel::rms_norm (src/kernel/mod.rs:199-209) applied to each row of x."""
    x2 = _f32(x)
    x2 = x2.reshape(-1, x2.shape[-1]) if x2.ndim > 1 else x2.reshape(1, -1)
    w = _f32(w).ravel()
    H = x2.shape[1]
    assert w.size >= H
    out = np.empty_like(x2)
    for t in range(x2.shape[0]):
        row = np.ascontiguousarray(x2[t])
        o = np.empty(H, np.float32)
        lib().nxo_rms_norm(_p(row, _fp), _p(w, _fp), H, eps, _p(o, _fp))
        out[t] = o
    return out


def matvec(w, rows: int, cols: int, x) -> np.ndarray:
    """InferenceEngine::matvec (src/engine/mod.rs:775-801)."""
    w = _f32(w).ravel()
    x = _f32(x).ravel()
    y = np.empty(max(rows, 1), np.float32)
    err = C.create_string_buffer(256)
    rc = lib().nxo_matvec(_p(w, _fp), w.size, rows, cols, _p(x, _fp), x.size, _p(y, _fp), err, 256)
    if rc:
        raise OracleError(err.value.decode())
    return y[:rows]


def _ptr_list(mats):
    arr = (_fp * max(len(mats), 1))()
    lens = (C.c_size_t * max(len(mats), 1))()
    keep = []
    for i, m in enumerate(mats):
        if m is None:
            arr[i] = _fp()
            lens[i] = 0
        else:
            m = _f32(m).ravel()
            keep.append(m)
            arr[i] = _p(m, _fp)
            lens[i] = m.size
    return arr, lens, keep


def dispatch_moe_ffn(hidden, router_logits, gate, up, down, top_k: int, hidden_size: int,
                     ff_dim: int) -> np.ndarray:
    """InferenceEngine::dispatch_moe_ffn (src/engine/mod.rs:969-1024), one token.

    gate/up/down are per-expert lists of flat f32 matrices (None = empty)."""
    if not (len(gate) == len(up) == len(down)) or len(gate) == 0:
        raise OracleError("MoE expert weight lists must be non-empty and aligned")
    h = _f32(hidden).ravel()
    lg = _f32(router_logits).ravel()
    g, gl, k1 = _ptr_list(gate)
    u, ul, k2 = _ptr_list(up)
    d, dl, k3 = _ptr_list(down)
    out = np.empty(max(hidden_size, 1), np.float32)
    err = C.create_string_buffer(256)
    rc = lib().nxo_dispatch_moe_ffn(_p(h, _fp), h.size, _p(lg, _fp), lg.size, g, gl, u, ul, d, dl,
                                    len(gate), top_k, hidden_size, ff_dim, _p(out, _fp), err, 256)
    if rc:
        raise OracleError(err.value.decode())
    return out[:hidden_size]


def moe_layer(x, logits, gate, up, down, top_k: int, score_mode: int = 0, shared=None,
              nthreads: int | None = None) -> np.ndarray:
    """Batched layer: row t == dispatch_moe_ffn(x[t], logits[t]) (+ shared expert).

    gate/up are lists of [F,H] f32 (None for experts never routed), down [H,F]."""
    x = _f32(x)
    T, H = x.shape
    lg = _f32(logits)
    E = lg.shape[1]
    F = next(m for m in gate if m is not None).size // H if any(m is not None for m in gate) else 0
    g, _, k1 = _ptr_list(gate)
    u, _, k2 = _ptr_list(up)
    d, _, k3 = _ptr_list(down)
    sg = su = sd = _fp()
    Fs = 0
    keep = []
    if shared is not None:
        s = [_f32(m).ravel() for m in shared]
        keep += s
        sg, su, sd = (_p(m, _fp) for m in s)
        Fs = s[0].size // H
    out = np.empty((T, H), np.float32)
    lib().nxo_moe_layer(_p(x, _fp), _p(lg, _fp), T, E, top_k, score_mode, g, u, d, sg, su, sd, H,
                        F, Fs, _p(out, _fp), nthreads or default_threads())
    return out


def swiglu_ffn(inp, w1, w3, w2, hidden_size: int, ff_dim: int) -> np.ndarray:
    """kernel::swiglu_ffn (src/kernel/mod.rs:104-157)."""
    inp = _f32(inp).ravel()
    w1, w3, w2 = (_f32(w).ravel() for w in (w1, w3, w2))
    B = inp.size // hidden_size
    out = np.empty(max(B * hidden_size, 1), np.float32)
    lib().nxo_swiglu_ffn(_p(inp, _fp), inp.size, _p(w1, _fp), _p(w3, _fp), _p(w2, _fp),
                         hidden_size, ff_dim, _p(out, _fp))
    return out[:B * hidden_size]


def cpu_matmul(a, b, m: int, n: int, k: int, nthreads: int | None = None) -> np.ndarray:
    """CpuBackend::matmul (src/backend/cpu.rs:23-38)."""
    a = _f32(a).ravel()
    b = _f32(b).ravel()
    c = np.empty(max(m * n, 1), np.float32)
    lib().nxo_cpu_matmul(_p(a, _fp), _p(b, _fp), m, n, k, _p(c, _fp), nthreads or default_threads())
    return c[:m * n]
