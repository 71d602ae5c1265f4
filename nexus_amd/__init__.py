"""nexus_amd — MI355X (gfx950) MoE routed-FFN path for Nexus.

The product is ``libnexus_hip.so`` (HIP kernels behind the C ABI declared in
``include/nexus_hip.h``).  This module is a thin ctypes binding over that ABI
for Python callers, tests and the benchmark.  There is no CPU fallback: if the
library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import sys
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# NEXUS_AMD_LIB points at another build of the same library (for example the
# host-sanitizer build, nexus_amd/csrc: make san)
LIB_PATH = os.environ.get("NEXUS_AMD_LIB") or os.path.join(_HERE, "libnexus_hip.so")
ROOT = os.path.dirname(_HERE)

# status codes / enums (include/nexus_hip.h)
NX_OK = 0
NX_ERR_INVALID_ARG, NX_ERR_SHAPE, NX_ERR_UNSUPPORTED, NX_ERR_DEVICE = 1, 2, 3, 4
NX_ERR_OOM, NX_ERR_TRUNCATED, NX_ERR_NO_ROUTES, NX_ERR_NOT_FOUND, NX_ERR_IO = 5, 6, 7, 8, 9
Q4K_REFERENCE, Q4K_GGML = 0, 1
F32, Q4_0, Q8_0, Q4_K, Q2_K, F16, BF16 = 0, 2, 8, 12, 10, 1, 28
SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1
PATH_AUTO, PATH_GEMV, PATH_MFMA_F16, PATH_MFMA_BF16, PATH_MFMA_SPLIT = 0, 1, 2, 3, 4
ROLE_GATE, ROLE_UP, ROLE_DOWN = 0, 1, 2
EXPERT_SHARED = -1
FORMAT_NAMES = {F32: "F32", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q2_K: "Q2_K", F16: "F16",
                BF16: "BF16"}
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q2_K: (256, 84), F32: (1, 4),
         F16: (1, 2), BF16: (1, 2)}

# every symbol the header declares (checked by the CPU test suite)
EXPORTS = [
    "nx_last_error", "nx_version", "nx_device_count", "nx_ctx_create", "nx_ctx_destroy",
    "nx_ctx_set_stream", "nx_ctx_get_stream", "nx_sync", "nx_mem_info", "nx_profile_enable",
    "nx_profile_reset", "nx_profile_count", "nx_profile_get", "nx_quant_bytes", "nx_dequant",
    "nx_dequant_dev", "nx_quantize", "nx_quantize_dev", "nx_router_logits",
    "nx_router_logits_dev", "nx_route_topk", "nx_permute",
    "nx_experts_create", "nx_experts_add_shared", "nx_experts_load", "nx_experts_info",
    "nx_experts_destroy", "nx_moe_forward", "nx_moe_forward_dev", "nx_gguf_open",
    "nx_gguf_close", "nx_gguf_info", "nx_gguf_tensor", "nx_gguf_find_tensor",
    "nx_gguf_tensor_data", "nx_gguf_meta_usize", "nx_gguf_meta_f32", "nx_gguf_meta_str",
    "nx_gguf_moe_info", "nx_experts_load_gguf", "nx_q4k_from_ggml", "nx_rms_norm",
    "nx_rms_norm_dev", "nx_moe_block", "nx_moe_block_dev", "nx_matrix_create",
    "nx_matrix_load", "nx_matrix_info", "nx_matrix_destroy", "nx_matvec", "nx_matvec_dev",
    "nx_matrix_load_gguf", "nx_moe_last_routes", "nx_moe_forward_noalloc",
]

_lib = None
_vp = C.c_void_p
_fp = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_ip = C.POINTER(C.c_int)


class NexusError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def build(verbose: bool = False) -> None:
    """Compile libnexus_hip.so for gfx950 with hipcc (always rebuilds)."""
    cmd = ["make", "-B", "-j8", "-C", os.path.join(_HERE, "csrc")]
    out = subprocess.run(cmd, capture_output=not verbose, text=True)
    if out.returncode != 0:
        raise RuntimeError("libnexus_hip.so build failed:\n" + (out.stdout or "") + (out.stderr or ""))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run nexus_amd.build() (there is no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    sig = {
        "nx_last_error": ([], C.c_char_p),
        "nx_version": ([], C.c_int),
        "nx_device_count": ([_ip], C.c_int),
        "nx_ctx_create": ([C.c_int, C.POINTER(_vp)], C.c_int),
        "nx_ctx_destroy": ([_vp], C.c_int),
        "nx_ctx_set_stream": ([_vp, _vp], C.c_int),
        "nx_ctx_get_stream": ([_vp, C.POINTER(_vp)], C.c_int),
        "nx_sync": ([_vp], C.c_int),
        "nx_mem_info": ([_vp, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)], C.c_int),
        "nx_profile_enable": ([_vp, C.c_int], C.c_int),
        "nx_profile_reset": ([_vp], C.c_int),
        "nx_profile_count": ([_vp, _ip], C.c_int),
        "nx_profile_get": ([_vp, C.c_int, C.c_char_p, C.c_size_t, _ip, C.POINTER(C.c_double)], C.c_int),
        "nx_quant_bytes": ([C.c_int, C.c_size_t, C.POINTER(C.c_size_t)], C.c_int),
        "nx_dequant": ([_vp, C.c_int, _vp, C.c_size_t, C.c_size_t, _fp], C.c_int),
        "nx_dequant_dev": ([_vp, C.c_int, _vp, C.c_size_t, C.c_size_t, _vp], C.c_int),
        "nx_quantize": ([_vp, C.c_int, _fp, C.c_size_t, _vp, C.c_size_t], C.c_int),
        "nx_quantize_dev": ([_vp, C.c_int, _vp, C.c_size_t, _vp, C.c_size_t], C.c_int),
        "nx_router_logits": ([_vp, _fp, C.c_size_t, _fp, C.c_size_t, C.c_int, C.c_int, C.c_int,
                              C.c_int, _fp], C.c_int),
        "nx_router_logits_dev": ([_vp, _vp, C.c_size_t, _vp, C.c_size_t, C.c_int, C.c_int,
                                  C.c_int, C.c_int, _vp], C.c_int),
        "nx_route_topk": ([_vp, _fp, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_int, _i32p, _fp,
                           _i32p, _ip], C.c_int),
        "nx_permute": ([_vp, _i32p, _i32p, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p, _i32p,
                        _i32p], C.c_int),
        "nx_experts_create": ([_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(_vp)], C.c_int),
        "nx_experts_add_shared": ([_vp, _vp, C.c_int], C.c_int),
        "nx_experts_load": ([_vp, _vp, C.c_int, C.c_int, _vp, C.c_size_t, C.c_int], C.c_int),
        "nx_experts_info": ([_vp, _ip, _ip, _ip, _ip, _ip, C.POINTER(C.c_size_t)], C.c_int),
        "nx_experts_destroy": ([_vp], C.c_int),
        "nx_moe_forward": ([_vp, _vp, _fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, _fp], C.c_int),
        "nx_moe_forward_dev": ([_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp],
                               C.c_int),
    }
    _u64p = C.POINTER(C.c_uint64)
    _u32p = C.POINTER(C.c_uint32)
    _szp = C.POINTER(C.c_size_t)
    sig.update({
        "nx_gguf_open": ([C.c_char_p, C.POINTER(_vp)], C.c_int),
        "nx_gguf_close": ([_vp], C.c_int),
        "nx_gguf_info": ([_vp, _u32p, _szp, _szp, _szp, _u64p], C.c_int),
        "nx_gguf_tensor": ([_vp, C.c_size_t, C.c_char_p, C.c_size_t, _u32p, _u32p, _u64p,
                            C.c_size_t, _u64p, _u64p], C.c_int),
        "nx_gguf_find_tensor": ([_vp, C.c_char_p, _szp], C.c_int),
        "nx_gguf_tensor_data": ([_vp, C.c_size_t, C.POINTER(_vp), _u64p], C.c_int),
        "nx_gguf_meta_usize": ([_vp, C.c_char_p, _u64p], C.c_int),
        "nx_gguf_meta_f32": ([_vp, C.c_char_p, _fp], C.c_int),
        "nx_gguf_meta_str": ([_vp, C.c_char_p, C.c_char_p, C.c_size_t, _szp], C.c_int),
        "nx_gguf_moe_info": ([_vp, C.c_int, _ip, _ip, _ip, _ip, _ip], C.c_int),
        "nx_experts_load_gguf": ([_vp, _vp, C.c_int, C.c_int, C.POINTER(_vp)], C.c_int),
        "nx_q4k_from_ggml": ([_vp, _vp, C.c_size_t], C.c_int),
        "nx_rms_norm": ([_vp, _fp, C.c_size_t, _fp, C.c_size_t, C.c_float, C.c_int, C.c_int,
                         C.c_int, _fp], C.c_int),
        "nx_rms_norm_dev": ([_vp, _vp, C.c_size_t, _vp, C.c_size_t, C.c_float, C.c_int, C.c_int,
                             C.c_int, _vp], C.c_int),
        "nx_moe_block": ([_vp, _vp, _fp, _fp, C.c_size_t, C.c_float, _fp, C.c_size_t, C.c_int,
                          C.c_int, C.c_int, C.c_int, C.c_int], C.c_int),
        "nx_moe_block_dev": ([_vp, _vp, _vp, _vp, C.c_size_t, C.c_float, _vp, C.c_size_t,
                              C.c_int, C.c_int, C.c_int, C.c_int, C.c_int], C.c_int),
        "nx_matrix_create": ([_vp, C.c_int, C.c_int, C.c_int, C.POINTER(_vp)], C.c_int),
        "nx_matrix_load": ([_vp, _vp, _vp, C.c_size_t, C.c_int], C.c_int),
        "nx_matrix_info": ([_vp, _ip, _ip, _ip, _szp], C.c_int),
        "nx_matrix_destroy": ([_vp], C.c_int),
        "nx_matvec": ([_vp, _vp, _fp, C.c_size_t, C.c_int, _fp], C.c_int),
        "nx_matvec_dev": ([_vp, _vp, _vp, C.c_size_t, C.c_int, _vp], C.c_int),
        "nx_matrix_load_gguf": ([_vp, _vp, C.c_char_p, C.c_int, C.POINTER(_vp)], C.c_int),
        "nx_moe_last_routes": ([_vp, C.c_int, C.c_int, _i32p, _fp, _i32p], C.c_int),
        "nx_moe_forward_noalloc": ([_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                    _vp], C.c_int),
    })
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != NX_OK:
        raise NexusError(rc, lib().nx_last_error().decode())


def device_count() -> int:
    n = C.c_int(0)
    check(lib().nx_device_count(C.byref(n)))
    return n.value


def quant_bytes(fmt: int, n: int) -> int:
    out = C.c_size_t(0)
    check(lib().nx_quant_bytes(fmt, n, C.byref(out)))
    return out.value


def _p(a, t):
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Context:
    """A device context (one HIP stream).  Not thread-safe."""

    def __init__(self, device: int = 0):
        h = _vp()
        check(lib().nx_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().nx_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self, _finalizing=sys.is_finalizing):
        # bound at definition: module globals may already be None at exit
        if _finalizing():  # the process is ending: leave it to the OS
            return
        try:
            self.close()
        except Exception:
            pass

    # ----------------------------------------------------------- runtime
    def sync(self):
        check(lib().nx_sync(self.h))

    def set_stream(self, stream_handle: int | None):
        check(lib().nx_ctx_set_stream(self.h, _vp(stream_handle or 0)))

    def mem_info(self):
        f, t = C.c_size_t(0), C.c_size_t(0)
        check(lib().nx_mem_info(self.h, C.byref(f), C.byref(t)))
        return f.value, t.value

    def profile(self, enable: bool):
        check(lib().nx_profile_enable(self.h, 1 if enable else 0))

    def profile_reset(self):
        check(lib().nx_profile_reset(self.h))

    def profile_stats(self) -> dict:
        n = C.c_int(0)
        check(lib().nx_profile_count(self.h, C.byref(n)))
        out = {}
        for i in range(n.value):
            name = C.create_string_buffer(64)
            cnt = C.c_int(0)
            ms = C.c_double(0)
            check(lib().nx_profile_get(self.h, i, name, 64, C.byref(cnt), C.byref(ms)))
            out[name.value.decode()] = (cnt.value, ms.value)
        return out

    # ----------------------------------------------------------- quant
    def dequant(self, fmt: int, data, n: int) -> np.ndarray:
        data = np.ascontiguousarray(data, dtype=np.uint8).ravel()
        out = np.empty(max(n, 1), np.float32)
        check(lib().nx_dequant(self.h, fmt, _vp(data.ctypes.data), data.size, n, _p(out, _fp)))
        return out[:n]

    def quantize(self, fmt: int, x) -> np.ndarray:
        x = _f32(x).ravel()
        nb = quant_bytes(fmt, x.size)
        out = np.empty(max(nb, 1), np.uint8)
        check(lib().nx_quantize(self.h, fmt, _p(x, _fp), x.size, _vp(out.ctypes.data), nb))
        return out[:nb]

    def dequant_dev(self, fmt: int, src_ptr: int, src_bytes: int, n: int, dst_ptr: int):
        check(lib().nx_dequant_dev(self.h, fmt, _vp(src_ptr), src_bytes, n, _vp(dst_ptr)))

    def quantize_dev(self, fmt: int, src_ptr: int, n: int, dst_ptr: int, dst_bytes: int):
        check(lib().nx_quantize_dev(self.h, fmt, _vp(src_ptr), n, _vp(dst_ptr), dst_bytes))

    # ----------------------------------------------------------- routing
    def router_logits(self, w_router, x, num_experts: int, hidden: int,
                      exact: bool = True) -> np.ndarray:
        """logits [T x E] = x [T x H] . w_router[E x H]^T on device.  exact=True
        reproduces InferenceEngine::matvec (src/engine/mod.rs:775-801) bit for bit."""
        w = _f32(w_router).ravel()
        xf = _f32(x).ravel()
        T = xf.size // hidden if hidden else 0
        out = np.empty(max(T * num_experts, 1), np.float32)
        check(lib().nx_router_logits(self.h, _p(w, _fp), w.size, _p(xf, _fp), xf.size, T,
                                     num_experts, hidden, 1 if exact else 0, _p(out, _fp)))
        return out[:T * num_experts].reshape(T, num_experts)

    def router_logits_raw(self, w_router, w_len: int, x, x_len: int, num_tokens: int,
                          num_experts: int, hidden: int, exact: bool = True) -> np.ndarray:
        """The C call with explicit lengths (for shape-error tests)."""
        w = _f32(w_router).ravel()
        xf = _f32(x).ravel()
        assert w.size >= w_len and xf.size >= x_len
        out = np.empty(max(num_tokens * num_experts, 1), np.float32)
        check(lib().nx_router_logits(self.h, _p(w, _fp), w_len, _p(xf, _fp), x_len, num_tokens,
                                     num_experts, hidden, 1 if exact else 0, _p(out, _fp)))
        return out[:num_tokens * num_experts].reshape(num_tokens, num_experts)

    def router_logits_dev(self, w_ptr: int, w_len: int, x_ptr: int, x_len: int,
                          num_tokens: int, num_experts: int, hidden: int, out_ptr: int,
                          exact: bool = True):
        check(lib().nx_router_logits_dev(self.h, _vp(w_ptr), w_len, _vp(x_ptr), x_len,
                                         num_tokens, num_experts, hidden, 1 if exact else 0,
                                         _vp(out_ptr)))

    def rms_norm(self, x, weight, eps: float, exact: bool = True) -> np.ndarray:
        """kernel::rms_norm (src/kernel/mod.rs:199-209) of each row of x [T x H]."""
        x2 = _f32(x)
        x2 = x2.reshape(-1, x2.shape[-1])
        w = _f32(weight).ravel()
        T, H = x2.shape
        out = np.empty((max(T, 1), max(H, 1)), np.float32)
        check(lib().nx_rms_norm(self.h, _p(x2, _fp), x2.size, _p(w, _fp), w.size, eps, T, H,
                                1 if exact else 0, _p(out, _fp)))
        return out[:T, :H]

    def rms_norm_dev(self, x_ptr: int, x_len: int, w_ptr: int, w_len: int, eps: float,
                     num_tokens: int, hidden: int, out_ptr: int, exact: bool = True):
        """nx_rms_norm_dev on device pointers (enqueued on the context's stream)."""
        check(lib().nx_rms_norm_dev(self.h, _vp(x_ptr), x_len, _vp(w_ptr), w_len, eps,
                                    num_tokens, hidden, 1 if exact else 0, _vp(out_ptr)))

    def route_topk(self, logits, num_tokens: int, num_experts: int, top_k: int,
                   score_mode: int = SCORE_SOFTMAX):
        lg = _f32(logits).ravel()
        T, k = num_tokens, top_k
        ex = np.full((max(T, 1), max(k, 1)), -1, np.int32)
        w = np.zeros((max(T, 1), max(k, 1)), np.float32)
        cnt = np.zeros(max(T, 1), np.int32)
        lists = C.c_int(0)
        check(lib().nx_route_topk(self.h, _p(lg, _fp), lg.size, T, num_experts, k, score_mode,
                                  _p(ex, _i32p), _p(w, _fp), _p(cnt, _i32p), C.byref(lists)))
        return ex[:T, :k], w[:T, :k], cnt[:T], lists.value

    def last_routes(self, num_tokens: int, top_k: int):
        """Routes of the last MoE forward on this context (experts, weights, counts)."""
        T, k = num_tokens, top_k
        ex = np.full((max(T, 1), max(k, 1)), -1, np.int32)
        w = np.zeros((max(T, 1), max(k, 1)), np.float32)
        cnt = np.zeros(max(T, 1), np.int32)
        check(lib().nx_moe_last_routes(self.h, T, k, _p(ex, _i32p), _p(w, _fp), _p(cnt, _i32p)))
        return ex[:T, :k], w[:T, :k], cnt[:T]

    def permute(self, experts, counts, num_experts: int):
        ex = np.ascontiguousarray(experts, dtype=np.int32)
        cnt = np.ascontiguousarray(counts, dtype=np.int32)
        T, k = ex.shape
        P = max(int(cnt.sum()), 1)
        ec = np.zeros(num_experts, np.int32)
        off = np.zeros(num_experts + 1, np.int32)
        pt = np.full(P, -1, np.int32)
        ps = np.full(P, -1, np.int32)
        inv = np.full((max(T, 1), max(k, 1)), -1, np.int32)
        check(lib().nx_permute(self.h, _p(ex, _i32p), _p(cnt, _i32p), T, k, num_experts,
                               _p(ec, _i32p), _p(off, _i32p), _p(pt, _i32p), _p(ps, _i32p),
                               _p(inv, _i32p)))
        n = int(off[-1])
        return ec, off, pt[:n], ps[:n], inv[:T, :k]


class Experts:
    """A device-resident expert set (quantized payloads kept in HBM)."""

    def __init__(self, ctx: Context, fmt: int, num_experts: int, hidden: int, ff_dim: int,
                 shared_ff_dim: int = 0):
        h = _vp()
        check(lib().nx_experts_create(ctx.h, fmt, num_experts, hidden, ff_dim, C.byref(h)))
        self.h = h
        self.ctx = ctx
        self.fmt, self.E, self.H, self.F, self.Fs = fmt, num_experts, hidden, ff_dim, 0
        if shared_ff_dim:
            check(lib().nx_experts_add_shared(ctx.h, h, shared_ff_dim))
            self.Fs = shared_ff_dim

    def load(self, expert: int, role: int, payload) -> None:
        """Load one GGUF payload (numpy uint8 array in host memory)."""
        data = np.ascontiguousarray(payload).view(np.uint8).ravel()
        check(lib().nx_experts_load(self.ctx.h, self.h, expert, role, _vp(data.ctypes.data),
                                    data.size, 0))

    def load_dev(self, expert: int, role: int, ptr: int, nbytes: int) -> None:
        check(lib().nx_experts_load(self.ctx.h, self.h, expert, role, _vp(ptr), nbytes, 1))

    def device_bytes(self) -> int:
        b = C.c_size_t(0)
        check(lib().nx_experts_info(self.h, None, None, None, None, None, C.byref(b)))
        return b.value

    def close(self):
        if self.h:
            lib().nx_experts_destroy(self.h)
            self.h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        # bound at definition: module globals may already be None at exit
        if _finalizing():  # the process is ending: leave it to the OS
            return
        try:
            self.close()
        except Exception:
            pass

    def forward(self, x, logits, top_k: int, score_mode: int = SCORE_SOFTMAX,
                path: int = PATH_AUTO) -> np.ndarray:
        x = _f32(x)
        T = x.shape[0]
        lg = _f32(logits)
        out = np.empty((max(T, 1), self.H), np.float32)
        check(lib().nx_moe_forward(self.ctx.h, self.h, _p(x, _fp), _p(lg, _fp), T, top_k,
                                   score_mode, path, _p(out, _fp)))
        return out[:T]

    def block(self, hidden, norm_w, eps: float, router_w, top_k: int,
              score_mode: int = SCORE_SOFTMAX, path: int = PATH_AUTO,
              exact: bool = True) -> np.ndarray:
        """One MoE block: hidden + MoE(rms_norm(hidden)) with on-device router logits."""
        h = _f32(hidden).copy()
        T = h.shape[0]
        nw = _f32(norm_w).ravel()
        rw = _f32(router_w).ravel()
        check(lib().nx_moe_block(self.ctx.h, self.h, _p(h, _fp), _p(nw, _fp), nw.size, eps,
                                 _p(rw, _fp), rw.size, T, top_k, score_mode, path,
                                 1 if exact else 0))
        return h

    def block_dev(self, hidden_ptr: int, norm_ptr: int, norm_len: int, eps: float,
                  router_ptr: int, router_len: int, num_tokens: int, top_k: int,
                  score_mode: int = SCORE_SOFTMAX, path: int = PATH_AUTO, exact: bool = True):
        check(lib().nx_moe_block_dev(self.ctx.h, self.h, _vp(hidden_ptr), _vp(norm_ptr),
                                     norm_len, eps, _vp(router_ptr), router_len, num_tokens,
                                     top_k, score_mode, path, 1 if exact else 0))

    def forward_dev(self, x_ptr: int, logits_ptr: int, num_tokens: int, top_k: int,
                    out_ptr: int, score_mode: int = SCORE_SOFTMAX, path: int = PATH_AUTO):
        check(lib().nx_moe_forward_dev(self.ctx.h, self.h, _vp(x_ptr), _vp(logits_ptr),
                                       num_tokens, top_k, score_mode, path, _vp(out_ptr)))

    def forward_noalloc(self, x_ptr: int, logits_ptr: int, num_tokens: int, top_k: int,
                        out_ptr: int, score_mode: int = SCORE_SOFTMAX, path: int = PATH_AUTO):
        """forward_dev with every intermediate in the library's static scratch array."""
        check(lib().nx_moe_forward_noalloc(self.ctx.h, self.h, _vp(x_ptr), _vp(logits_ptr),
                                           num_tokens, top_k, score_mode, path, _vp(out_ptr)))


class Matrix:
    """A device-resident dense weight matrix (rows x cols) kept in its GGUF format."""

    def __init__(self, ctx: Context, fmt: int, rows: int, cols: int):
        h = _vp()
        check(lib().nx_matrix_create(ctx.h, fmt, rows, cols, C.byref(h)))
        self.h, self.ctx = h, ctx
        self.fmt, self.rows, self.cols = fmt, rows, cols

    @classmethod
    def _wrap(cls, ctx: Context, h):
        m = cls.__new__(cls)
        m.h, m.ctx = h, ctx
        f, r, c = C.c_int(), C.c_int(), C.c_int()
        check(lib().nx_matrix_info(h, C.byref(f), C.byref(r), C.byref(c), None))
        m.fmt, m.rows, m.cols = f.value, r.value, c.value
        return m

    def load(self, payload) -> None:
        """Load a GGUF payload (numpy array in host memory)."""
        data = np.ascontiguousarray(payload).view(np.uint8).ravel()
        check(lib().nx_matrix_load(self.ctx.h, self.h, _vp(data.ctypes.data), data.size, 0))

    def load_dev(self, ptr: int, nbytes: int) -> None:
        check(lib().nx_matrix_load(self.ctx.h, self.h, _vp(ptr), nbytes, 1))

    def device_bytes(self) -> int:
        b = C.c_size_t(0)
        check(lib().nx_matrix_info(self.h, None, None, None, C.byref(b)))
        return b.value

    def matvec(self, x, num_tokens: int | None = None) -> np.ndarray:
        """y[t] = W . x[t] for x of shape [T, cols] (or [cols] for one token)."""
        x = _f32(x)
        T = (1 if x.ndim == 1 else x.shape[0]) if num_tokens is None else num_tokens
        y = np.empty((max(T, 1), self.rows), np.float32)
        xf = x.ravel()
        check(lib().nx_matvec(self.ctx.h, self.h, _p(xf, _fp), xf.size, T, _p(y, _fp)))
        return y[:T] if x.ndim != 1 else y[0]

    def matvec_dev(self, x_ptr: int, x_len: int, num_tokens: int, y_ptr: int) -> None:
        check(lib().nx_matvec_dev(self.ctx.h, self.h, _vp(x_ptr), x_len, num_tokens, _vp(y_ptr)))

    def close(self):
        if self.h:
            lib().nx_matrix_destroy(self.h)
            self.h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        # bound at definition: module globals may already be None at exit
        if _finalizing():  # the process is ending: leave it to the OS
            return
        try:
            self.close()
        except Exception:
            pass


class Gguf:
    """A memory-mapped GGUF file (GgufReader::parse_file).  No GPU needed."""

    def __init__(self, path: str):
        h = _vp()
        check(lib().nx_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().nx_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self, _finalizing=sys.is_finalizing):
        # bound at definition: module globals may already be None at exit
        if _finalizing():  # the process is ending: leave it to the OS
            return
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> dict:
        v, n, kv, al, off = C.c_uint32(), C.c_size_t(), C.c_size_t(), C.c_size_t(), C.c_uint64()
        check(lib().nx_gguf_info(self.h, C.byref(v), C.byref(n), C.byref(kv), C.byref(al),
                                 C.byref(off)))
        return {"version": v.value, "tensor_count": n.value, "kv_count": kv.value,
                "alignment": al.value, "data_offset": off.value}

    def tensor(self, index: int) -> dict:
        name = C.create_string_buffer(512)
        t, nd, off, nb = C.c_uint32(), C.c_uint32(), C.c_uint64(), C.c_uint64()
        dims = (C.c_uint64 * 8)()
        check(lib().nx_gguf_tensor(self.h, index, name, 512, C.byref(t), C.byref(nd), dims, 8,
                                   C.byref(off), C.byref(nb)))
        return {"name": name.value.decode(), "type": t.value,
                "dims": [dims[i] for i in range(min(nd.value, 8))], "offset": off.value,
                "bytes": nb.value}

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.info()["tensor_count"])]

    def find(self, name: str) -> int:
        i = C.c_size_t()
        check(lib().nx_gguf_find_tensor(self.h, name.encode(), C.byref(i)))
        return i.value

    def data(self, index: int) -> np.ndarray:
        """A copy of tensor `index`'s payload bytes."""
        p, nb = _vp(), C.c_uint64()
        check(lib().nx_gguf_tensor_data(self.h, index, C.byref(p), C.byref(nb)))
        return np.frombuffer(C.string_at(p.value, nb.value), dtype=np.uint8).copy()

    def meta_usize(self, key: str) -> int:
        v = C.c_uint64()
        check(lib().nx_gguf_meta_usize(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_f32(self, key: str) -> float:
        v = C.c_float()
        check(lib().nx_gguf_meta_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key: str) -> str:
        n = C.c_size_t()
        check(lib().nx_gguf_meta_str(self.h, key.encode(), None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        check(lib().nx_gguf_meta_str(self.h, key.encode(), buf, n.value + 1, None))
        return buf.raw[:n.value].decode()

    def moe_info(self, layer: int) -> dict:
        f, e, h, ff, fs = C.c_int(), C.c_int(), C.c_int(), C.c_int(), C.c_int()
        check(lib().nx_gguf_moe_info(self.h, layer, C.byref(f), C.byref(e), C.byref(h),
                                     C.byref(ff), C.byref(fs)))
        return {"fmt": f.value, "experts": e.value, "hidden": h.value, "ffn": ff.value,
                "shared_ffn": fs.value}


def q4k_from_ggml(blocks) -> np.ndarray:
    """Q4_K blocks from upstream ggml's code order to the reference's."""
    src = np.ascontiguousarray(blocks, dtype=np.uint8).ravel()
    dst = np.empty_like(src)
    check(lib().nx_q4k_from_ggml(_vp(src.ctypes.data), _vp(dst.ctypes.data), src.size // 144))
    return dst


def experts_from_gguf(ctx: Context, g: Gguf, layer: int, q4k_order: int = Q4K_REFERENCE):
    """Block `layer`'s experts loaded quantized-resident from a GGUF file."""
    h = _vp()
    check(lib().nx_experts_load_gguf(ctx.h, g.h, layer, q4k_order, C.byref(h)))
    info = g.moe_info(layer)
    ex = Experts.__new__(Experts)
    ex.h, ex.ctx = h, ctx
    ex.fmt, ex.E, ex.H, ex.F = info["fmt"], info["experts"], info["hidden"], info["ffn"]
    ex.Fs = info["shared_ffn"]
    return ex


def matrix_from_gguf(ctx: Context, g: Gguf, name: str, q4k_order: int = Q4K_REFERENCE) -> Matrix:
    """The tensor `name` of a GGUF file as a resident dense matrix."""
    h = _vp()
    check(lib().nx_matrix_load_gguf(ctx.h, g.h, name.encode(), q4k_order, C.byref(h)))
    return Matrix._wrap(ctx, h)
