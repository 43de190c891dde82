"""intllm — Python bindings (ctypes) of the Q16.48 forward-pass libraries.

The product is native: ``lib/libintllm_hip.so`` (HIP kernels behind the C ABI
of ``include/intllm_hip.h``) and ``lib/libq48host.so`` (the C host:
config.json / .mgw loading, llama_forward and generate over that ABI).  This
module only loads them and moves numpy int64 arrays across the boundary, for
tests and benchmarks.  It never computes a result itself: if the libraries
are missing it raises instead of falling back to anything.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_DIR = PKG_ROOT / "lib"
HIP_LIB = LIB_DIR / "libintllm_hip.so"
HOST_LIB = LIB_DIR / "libq48host.so"

Q48_OK, Q48_EINVAL, Q48_ENOMEM, Q48_EHIP, Q48_ERANGE, Q48_ESTATE = 0, -1, -2, -3, -4, -5
Q48_ETIMEOUT, Q48_ETOOBIG = -6, -7

# fp_eval function ids (include/intllm_hip.h, q48_fp_eval)
FP_MUL, FP_DIV, FP_SQRT, FP_SQRT_FAST, FP_INV_SQRT, FP_EXP, FP_LOG, FP_SINCOS, \
    FP_SIGMOID, FP_SILU, FP_SAFE_EXP, FP_EXP_DYADIC, FP_DIV_ROW = range(13)

# q48_gemm_ex kernels (include/intllm_hip.h)
GEMM_AUTO, GEMM_VALU, GEMM_I8, GEMM_I8_FUSED, GEMM_I8_PLANES = 0, 1, 2, 3, 4

# ABI entry points and their argument types (include/intllm_hip.h)
_P, _I, _SZ = C.c_void_p, C.c_int, C.c_size_t
ABI_SIGNATURES = {
    "q48_ctx_create": [C.POINTER(C.c_void_p), _I],
    "q48_ctx_destroy": [_P],
    "q48_malloc": [_P, C.POINTER(C.c_void_p), _SZ],
    "q48_free": [_P, _P],
    "q48_memcpy_h2d": [_P, _P, _P, _SZ],
    "q48_memcpy_d2h": [_P, _P, _P, _SZ],
    "q48_memcpy_d2d": [_P, _P, _P, _SZ],
    "q48_zero": [_P, _P, _SZ],
    "q48_sync": [_P],
    "q48_gemv": [_P, _P, _P, _P, _I, _I],
    "q48_gemm": [_P, _P, _P, _P, _I, _I, _I],
    "q48_gemm_ex": [_P, _P, _P, _P, _I, _I, _I, _I],
    "q48_gemm_planes_bytes": [_I, _I, C.POINTER(C.c_size_t)],
    "q48_gemm_prepare": [_P, _P, _P, _I, _I],
    "q48_gemm_prepared": [_P, _P, _P, _P, _P, _I, _I, _I],
    "q48_bf16_pack": [_P, _P, _P, _SZ, C.POINTER(C.c_int)],
    "q48_gemv_bf16": [_P, _P, _P, _P, _I, _I],
    "q48_norm_gemv_stats_bf16": [_P, _P, _P, _P, _P, _P, _I, _I],
    "q48_norm_gemv_swiglu_stats_bf16": [_P, _P, _P, _P, _P, _P, _I, _I],
    "q48_gemv_residual_stats_bf16": [_P, _P, _P, _P, _I, _I, _P],
    "q48_set_gemv_persistent": [_P, _I],

    "q48_rmsnorm": [_P, _P, _P, _P, _I],
    "q48_rope_init": [_P, _I, _I, _I],
    "q48_rope": [_P, _P, _I, _I, _I],
    "q48_attn_decode": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I],
    "q48_silu_mul": [_P, _P, _P, _P, _I],
    "q48_add": [_P, _P, _P, _I],
    "q48_embed": [_P, _P, _P, _I, _I],
    "q48_argmax": [_P, _P, _I, C.POINTER(C.c_int)],
    "q48_sample": [_P, _P, _I, C.c_int64, _I, C.c_int64, _P, C.POINTER(C.c_int)],
    "q48_sample_step": [_P, _P, _I, C.c_int64, _I, C.c_int64, _P, _P, _I],
    "q48_sample_reserve": [_P, _I],
    "q48_rope_tables": [_P, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)],
    "q48_fp_eval": [_P, _I, _P, _P, _P, _P, _I],
    "q48_rmsnorm_gemv": [_P, _P, _P, _P, _P, _I, _I],
    "q48_gemv_residual": [_P, _P, _P, _P, _I, _I],
    "q48_rmsnorm_gemv_swiglu": [_P, _P, _P, _P, _P, _I, _I],
    "q48_attn_decode_rope": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I],
    "q48_attn_split_min": [],
    "q48_set_attn_one_launch": [_P, _I],
    "q48_set_pf_attn_mfma": [_P, _I],
    "q48_set_attn_g_mfma": [_P, _I],
    "q48_attn_prefill": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I],
    "q48_attn_status": [_P],
    "q48_attn_decode_rope_prefetch": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _SZ],
    "q48_norm_gemv_rope_kv": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I],
    "q48_norm_gemv_rope_kv_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I],
    "q48_attn_decode_cached": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _SZ],
    "q48_rms_inv": [_P, _P, _P, _I],
    "q48_embed_rms": [_P, _P, _P, _I, _I, _P],
    "q48_norm_gemv": [_P, _P, _P, _P, _P, _P, _I, _I],
    "q48_norm_gemv_swiglu": [_P, _P, _P, _P, _P, _P, _I, _I],
    "q48_gemv_residual_rms": [_P, _P, _P, _P, _I, _I, _P],
    "q48_rms_stats": [_P, _P, _P, _I],
    "q48_embed_stats": [_P, _P, _P, _I, _I, _P],
    "q48_norm_gemv_stats": [_P, _P, _P, _P, _P, _P, _I, _I],
    "q48_norm_gemv_swiglu_stats": [_P, _P, _P, _P, _P, _P, _I, _I],
    "q48_gemv_residual_stats": [_P, _P, _P, _P, _I, _I, _P],
    "q48_step_mode": [_P, _I],
    "q48_step_set": [_P, _I, _I],
    "q48_step_get": [_P, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)],
    "q48_argmax_step": [_P, _P, _I, _P, _I],
    "q48_record_step": [_P, _P, _I, _P, _I],
    "q48_argmax_record_step": [_P, _P, _I, _P, _I, _P, _I],
    "q48_graph_begin": [_P],
    "q48_graph_end": [_P],
    "q48_graph_launch": [_P, _I],
    "q48_graph_drop": [_P],
    "q48_graph_capture": [_P],
    "q48_graph_instantiate": [_P, C.POINTER(C.c_void_p)],
    "q48_graph_replay": [_P, _P, _I],
    "q48_graph_destroy": [_P, _P],
    "q48_set_attn_wait": [_P, C.c_int64],
    "q48_prof_enable": [_P, _I],
    "q48_timer_start": [_P],
    "q48_timer_stop": [_P, C.POINTER(C.c_double)],
    "q48_prof_read": [_P, _P, _I],
}


class Prof(C.Structure):
    """q48_prof: HIP-event timing of q48_gemv launches."""
    _fields_ = [("launches", C.c_int), ("ms", C.c_double), ("bytes", C.c_double)]


class Q48Error(RuntimeError):
    def __init__(self, fn: str, code: int):
        self.code = code
        super().__init__(f"{fn} failed: {code} ({strerror(code)})")


_hip = None
_host = None


def _require(path: Path) -> None:
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run `make -C {PKG_ROOT}` (or __graft_entry__.build())"
        )


def hip_lib() -> C.CDLL:
    """libintllm_hip.so with typed entry points (raises if not built)."""
    global _hip
    if _hip is None:
        _require(HIP_LIB)
        lib = C.CDLL(str(HIP_LIB), mode=C.RTLD_GLOBAL)
        for name, args in ABI_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = C.c_int
        lib.q48_strerror.argtypes = [C.c_int]
        lib.q48_strerror.restype = C.c_char_p
        lib.q48_rng_seed.argtypes = [C.c_uint64, C.POINTER(C.c_uint64)]
        lib.q48_rng_seed.restype = None
        lib.q48_graph_stamp.argtypes = [_P]
        lib.q48_graph_stamp.restype = C.c_uint64
        _hip = lib
    return _hip


def strerror(code: int) -> str:
    try:
        return hip_lib().q48_strerror(code).decode()
    except Exception:  # library not loadable: message only
        return "unknown"


def check(fn: str, rc: int) -> int:
    if rc < 0:
        raise Q48Error(fn, rc)
    return rc


def stats_words(dim: int) -> int:
    """Q48_STATS_WORDS(dim): int64 words of a partial-sums statistics buffer."""
    return 2 * ((dim + 7) // 8)


def i64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int64)


class Buffer:
    """A device allocation of int64 elements owned by a Context."""

    def __init__(self, ctx: "Context", n: int, itemsize: int = 8):
        self.ctx, self.n, self.itemsize = ctx, int(n), itemsize
        p = C.c_void_p()
        check("q48_malloc", hip_lib().q48_malloc(ctx.h, C.byref(p), max(1, self.n) * itemsize))
        self.ptr = p.value

    @property
    def nbytes(self) -> int:
        return self.n * self.itemsize

    def upload(self, arr) -> "Buffer":
        a = i64(arr) if self.itemsize == 8 else np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        check("q48_memcpy_h2d", hip_lib().q48_memcpy_h2d(self.ctx.h, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def download(self, n: int | None = None) -> np.ndarray:
        n = self.n if n is None else n
        out = np.empty(n, dtype=np.int64)
        check("q48_memcpy_d2h", hip_lib().q48_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr, n * 8))
        return out

    def at(self, elem_offset: int) -> int:
        return self.ptr + 8 * int(elem_offset)

    def free(self) -> None:
        if self.ptr:
            hip_lib().q48_free(self.ctx.h, self.ptr)
            self.ptr = None


class Context:
    """q48_ctx: one HIP stream plus the device fp_math constants."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check("q48_ctx_create", hip_lib().q48_ctx_create(C.byref(h), device))
        self.h = h.value
        self._bufs: list[Buffer] = []

    def close(self) -> None:
        if self.h:
            for b in self._bufs:
                b.free()
            hip_lib().q48_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def buffer(self, n: int) -> Buffer:
        b = Buffer(self, n)
        self._bufs.append(b)
        return b

    def to_device(self, arr) -> Buffer:
        a = i64(arr).ravel()
        return self.buffer(a.size).upload(a)

    def sync(self) -> None:
        check("q48_sync", hip_lib().q48_sync(self.h))

    # ---- ops (device pointers are ints) ----
    def gemv(self, y, W, x, M, K):
        return check("q48_gemv", hip_lib().q48_gemv(self.h, y, W, x, M, K))

    def bf16_pack(self, out, inp, n) -> bool:
        """Pack n int64 at inp into bfloat16 bits at out; False if any is inexact."""
        flag = C.c_int()
        check("q48_bf16_pack", hip_lib().q48_bf16_pack(self.h, out, inp, n, C.byref(flag)))
        return flag.value == 0

    def gemv_bf16(self, y, W, x, M, K):
        return check("q48_gemv_bf16", hip_lib().q48_gemv_bf16(self.h, y, W, x, M, K))

    def norm_gemv_stats_bf16(self, y, W, x, norm_w, stats, M, K):
        return check("q48_norm_gemv_stats_bf16",
                     hip_lib().q48_norm_gemv_stats_bf16(self.h, y, W, x, norm_w, stats, M, K))

    def norm_gemv_swiglu_stats_bf16(self, out, Wgu, x, norm_w, stats, ffn, K):
        return check("q48_norm_gemv_swiglu_stats_bf16", hip_lib().q48_norm_gemv_swiglu_stats_bf16(
            self.h, out, Wgu, x, norm_w, stats, ffn, K))

    def gemv_residual_stats_bf16(self, acc, W, x, M, K, stats):
        return check("q48_gemv_residual_stats_bf16",
                     hip_lib().q48_gemv_residual_stats_bf16(self.h, acc, W, x, M, K, stats))

    def set_attn_one_launch(self, on: bool):
        return check("q48_set_attn_one_launch", hip_lib().q48_set_attn_one_launch(self.h, int(on)))

    def attn_status(self):
        """0, or Q48_ETIMEOUT (returned, not raised) when a one-launch split
        attention gave up since the last call."""
        rc = hip_lib().q48_attn_status(self.h)
        return rc if rc == Q48_ETIMEOUT else check("q48_attn_status", rc)

    def set_attn_wait(self, ticks: int):
        """k_attn_g's wait bound in wall-clock ticks; -1 restores the default,
        0 gives up at the first exchange (the timeout path, for tests)."""
        return check("q48_set_attn_wait", hip_lib().q48_set_attn_wait(self.h, int(ticks)))

    def graph_stamp(self) -> int:
        return int(hip_lib().q48_graph_stamp(self.h))

    def set_pf_attn_mfma(self, on: bool):
        return check("q48_set_pf_attn_mfma", hip_lib().q48_set_pf_attn_mfma(self.h, int(on)))

    def set_attn_g_mfma(self, on: bool):
        return check("q48_set_attn_g_mfma", hip_lib().q48_set_attn_g_mfma(self.h, int(on)))

    def attn_prefill(self, out, qkv, kc, vc, layer, p0, T, nh, nkv, hd, max_seq):
        """Causal attention of T rotated [q | k | v] rows at positions p0 .. p0 + T - 1
        over the cache rows stored before (q48_rope_store_rows)."""
        return check("q48_attn_prefill", hip_lib().q48_attn_prefill(
            self.h, out, qkv, kc, vc, layer, p0, T, nh, nkv, hd, max_seq))

    def set_gemv_persistent(self, on: bool):
        return check("q48_set_gemv_persistent", hip_lib().q48_set_gemv_persistent(self.h, int(on)))

    def gemm(self, Y, W, X, T, N, K, kernel=None):
        """kernel: None (q48_gemm's choice), GEMM_VALU, GEMM_I8 (the int8
        kernel chosen by shape), GEMM_I8_FUSED or GEMM_I8_PLANES."""
        if kernel is None:
            return check("q48_gemm", hip_lib().q48_gemm(self.h, Y, W, X, T, N, K))
        return check("q48_gemm_ex", hip_lib().q48_gemm_ex(self.h, Y, W, X, T, N, K, kernel))

    @staticmethod
    def gemm_planes_bytes(N, K) -> int:
        """Bytes of a prepared weight's digit planes (q48_gemm_prepare)."""
        out = C.c_size_t(0)
        check("q48_gemm_planes_bytes", hip_lib().q48_gemm_planes_bytes(N, K, C.byref(out)))
        return out.value

    def gemm_prepare(self, Wp, W, N, K):
        """W [N][K]'s digit planes into the device buffer Wp."""
        return check("q48_gemm_prepare", hip_lib().q48_gemm_prepare(self.h, Wp, W, N, K))

    def gemm_prepared(self, Y, W, Wp, X, T, N, K):
        """q48_gemm over W with its planes Wp from gemm_prepare."""
        return check("q48_gemm_prepared",
                     hip_lib().q48_gemm_prepared(self.h, Y, W, Wp, X, T, N, K))

    def rmsnorm(self, out, x, w, dim):
        return check("q48_rmsnorm", hip_lib().q48_rmsnorm(self.h, out, x, w, dim))

    def rope_init(self, head_dim, max_seq, theta):
        return check("q48_rope_init", hip_lib().q48_rope_init(self.h, head_dim, max_seq, theta))

    def rope(self, vec, n_heads, head_dim, pos):
        return check("q48_rope", hip_lib().q48_rope(self.h, vec, n_heads, head_dim, pos))

    def attn_decode(self, out, q, kc, vc, kn, vn, layer, pos, nh, nkv, hd, max_seq):
        return check("q48_attn_decode", hip_lib().q48_attn_decode(
            self.h, out, q, kc, vc, kn, vn, layer, pos, nh, nkv, hd, max_seq))

    def silu_mul(self, out, g, u, n):
        return check("q48_silu_mul", hip_lib().q48_silu_mul(self.h, out, g, u, n))

    def add(self, acc, d, n):
        return check("q48_add", hip_lib().q48_add(self.h, acc, d, n))

    def embed(self, out, table, token, dim):
        return check("q48_embed", hip_lib().q48_embed(self.h, out, table, token, dim))

    def argmax(self, v, n) -> int:
        r = C.c_int()
        check("q48_argmax", hip_lib().q48_argmax(self.h, v, n, C.byref(r)))
        return r.value

    def sample(self, v, n, temperature, top_k, top_p, rng) -> int:
        """sample_token (llama_int.c:2958-3039) of device logits v[0..n);
        rng: device pointer to the 2-word xoroshiro128+ state."""
        r = C.c_int()
        check("q48_sample", hip_lib().q48_sample(self.h, v, n, temperature, top_k, top_p, rng,
                                                 C.byref(r)))
        return r.value

    def zero(self, p, nbytes):
        return check("q48_zero", hip_lib().q48_zero(self.h, p, nbytes))

    def rope_tables(self):
        c, s = C.c_void_p(), C.c_void_p()
        check("q48_rope_tables", hip_lib().q48_rope_tables(self.h, C.byref(c), C.byref(s)))
        return c.value, s.value

    def rmsnorm_gemv(self, y, W, x, norm_w, M, K):
        return check("q48_rmsnorm_gemv", hip_lib().q48_rmsnorm_gemv(self.h, y, W, x, norm_w, M, K))

    def gemv_residual(self, acc, W, x, M, K):
        return check("q48_gemv_residual", hip_lib().q48_gemv_residual(self.h, acc, W, x, M, K))

    def rmsnorm_gemv_swiglu(self, out, Wgu, x, norm_w, ffn, K):
        return check("q48_rmsnorm_gemv_swiglu",
                     hip_lib().q48_rmsnorm_gemv_swiglu(self.h, out, Wgu, x, norm_w, ffn, K))

    def attn_decode_rope(self, out, q, kc, vc, kn, vn, layer, pos, nh, nkv, hd, max_seq):
        return check("q48_attn_decode_rope", hip_lib().q48_attn_decode_rope(
            self.h, out, q, kc, vc, kn, vn, layer, pos, nh, nkv, hd, max_seq))

    def attn_decode_rope_prefetch(self, out, q, kc, vc, kn, vn, layer, pos, nh, nkv, hd, max_seq,
                                  prefetch, nbytes):
        return check("q48_attn_decode_rope_prefetch", hip_lib().q48_attn_decode_rope_prefetch(
            self.h, out, q, kc, vc, kn, vn, layer, pos, nh, nkv, hd, max_seq, prefetch, nbytes))

    def norm_gemv_rope_kv(self, qkv, W, x, norm_w, stats, kc, vc, layer, pos, nh, nkv, hd,
                          max_seq, K):
        return check("q48_norm_gemv_rope_kv", hip_lib().q48_norm_gemv_rope_kv(
            self.h, qkv, W, x, norm_w, stats, kc, vc, layer, pos, nh, nkv, hd, max_seq, K))

    def norm_gemv_rope_kv_bf16(self, qkv, W, x, norm_w, stats, kc, vc, layer, pos, nh, nkv,
                               hd, max_seq, K):
        return check("q48_norm_gemv_rope_kv_bf16", hip_lib().q48_norm_gemv_rope_kv_bf16(
            self.h, qkv, W, x, norm_w, stats, kc, vc, layer, pos, nh, nkv, hd, max_seq, K))

    def attn_decode_cached(self, out, q, kc, vc, layer, pos, nh, nkv, hd, max_seq,
                           prefetch=None, nbytes=0):
        return check("q48_attn_decode_cached", hip_lib().q48_attn_decode_cached(
            self.h, out, q, kc, vc, layer, pos, nh, nkv, hd, max_seq, prefetch, nbytes))

    def rms_inv(self, r_out, x, dim):
        return check("q48_rms_inv", hip_lib().q48_rms_inv(self.h, r_out, x, dim))

    def embed_rms(self, out, table, token, dim, r_out):
        return check("q48_embed_rms", hip_lib().q48_embed_rms(self.h, out, table, token, dim, r_out))

    def norm_gemv(self, y, W, x, norm_w, r, M, K):
        return check("q48_norm_gemv", hip_lib().q48_norm_gemv(self.h, y, W, x, norm_w, r, M, K))

    def norm_gemv_swiglu(self, out, Wgu, x, norm_w, r, ffn, K):
        return check("q48_norm_gemv_swiglu",
                     hip_lib().q48_norm_gemv_swiglu(self.h, out, Wgu, x, norm_w, r, ffn, K))

    def gemv_residual_rms(self, acc, W, x, M, K, r_out):
        return check("q48_gemv_residual_rms",
                     hip_lib().q48_gemv_residual_rms(self.h, acc, W, x, M, K, r_out))

    # statistics as per-8-row partial sums (stats_words(dim) int64 words)
    def rms_stats(self, stats, x, dim):
        return check("q48_rms_stats", hip_lib().q48_rms_stats(self.h, stats, x, dim))

    def embed_stats(self, out, table, token, dim, stats):
        return check("q48_embed_stats",
                     hip_lib().q48_embed_stats(self.h, out, table, token, dim, stats))

    def norm_gemv_stats(self, y, W, x, norm_w, stats, M, K):
        return check("q48_norm_gemv_stats",
                     hip_lib().q48_norm_gemv_stats(self.h, y, W, x, norm_w, stats, M, K))

    def norm_gemv_swiglu_stats(self, out, Wgu, x, norm_w, stats, ffn, K):
        return check("q48_norm_gemv_swiglu_stats",
                     hip_lib().q48_norm_gemv_swiglu_stats(self.h, out, Wgu, x, norm_w, stats,
                                                          ffn, K))

    def gemv_residual_stats(self, acc, W, x, M, K, stats):
        return check("q48_gemv_residual_stats",
                     hip_lib().q48_gemv_residual_stats(self.h, acc, W, x, M, K, stats))

    def prof_enable(self, on: bool = True):
        check("q48_prof_enable", hip_lib().q48_prof_enable(self.h, int(on)))

    def timer_start(self):
        check("q48_timer_start", hip_lib().q48_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = C.c_double()
        check("q48_timer_stop", hip_lib().q48_timer_stop(self.h, C.byref(ms)))
        return ms.value

    def prof_read(self, reset: bool = True) -> "Prof":
        p = Prof()
        check("q48_prof_read", hip_lib().q48_prof_read(self.h, C.byref(p), int(reset)))
        return p

    def fp_eval(self, func, x, y, out0, out1, n):
        return check("q48_fp_eval", hip_lib().q48_fp_eval(self.h, func, x, y or None, out0, out1 or None, n))


# ---------------------------------------------------------------------------
# C host (libq48host.so)
# ---------------------------------------------------------------------------

class Config(C.Structure):
    """q48h_config == llama_config_t field for field (llama_int.c:788-798)."""
    _fields_ = [(n, C.c_int) for n in
                ("dim", "n_heads", "n_kv_heads", "head_dim", "n_layers", "ffn",
                 "vocab", "max_seq", "rope_theta")]

    def as_tuple(self):
        return tuple(getattr(self, n) for n, _ in self._fields_)


class Stats(C.Structure):
    _fields_ = [("prefill_s", C.c_double), ("decode_s", C.c_double),
                ("prefill_tokens", C.c_int), ("decode_tokens", C.c_int)]


TINY = Config(256, 8, 2, 32, 2, 688, 512, 2048, 10000)
TINYLLAMA = Config(2048, 32, 4, 64, 22, 5632, 32000, 2048, 10000)


def config(base: Config, **kw) -> Config:
    c = Config(*base.as_tuple())
    for k, v in kw.items():
        setattr(c, k, v)
    return c


HOST_SIGNATURES = {
    "q48h_config_from_json": ([C.c_char_p, C.POINTER(Config)], C.c_int),
    "q48h_config_from_json_text": ([C.c_char_p, C.POINTER(Config)], C.c_int),
    "q48h_config_check": ([C.POINTER(Config)], C.c_int),
    "q48h_model_create": ([C.POINTER(C.c_void_p), _P, C.POINTER(Config)], C.c_int),
    "q48h_model_free": ([_P], None),
    "q48h_upload": ([_P, C.c_char_p, _P, C.c_int64], C.c_int),
    "q48h_model_synth": ([_P, C.c_uint64, _I], C.c_int),
    "q48h_model_load_mgw": ([C.POINTER(C.c_void_p), _P, C.c_char_p, _I], C.c_int),
    "q48h_mgw_write_synth": ([C.c_char_p, C.POINTER(Config), C.c_uint64, _I], C.c_int),
    "q48h_kv_keys": ([_P], C.c_void_p),
    "q48h_kv_values": ([_P], C.c_void_p),
    "q48h_kv_reset": ([_P], C.c_int),
    "q48h_kv_fill_synth": ([_P, C.c_uint64, _I, _I], C.c_int),
    "q48h_forward": ([_P, _I, _I, _P, C.POINTER(C.c_int)], C.c_int),
    "q48h_generate": ([_P, C.POINTER(C.c_int), _I, _I, C.POINTER(C.c_int),
                       C.POINTER(C.c_uint64), C.POINTER(C.c_int), C.POINTER(Stats)], C.c_int),
    "q48h_decode_from": ([_P, _I, _I, _I, C.POINTER(C.c_int), C.POINTER(C.c_uint64),
                          C.POINTER(Stats)], C.c_int),
    "q48h_model_set_fused": ([_P, _I], None),
    "q48h_model_set_prefetch": ([_P, _I], None),
    "q48h_model_set_rope_gemv": ([_P, _I], None),
    "q48h_read_logits": ([_P, _P], C.c_int),
    "q48h_model_set_bf16": ([_P, _I], C.c_int),
    "q48h_model_set_sampling": ([_P, C.c_int64, _I, C.c_int64, C.c_uint64], C.c_int),
    "q48h_model_set_batched_prefill": ([_P, _I], None),
    "q48h_model_set_gemm_planes": ([_P, _I], None),
    "q48h_prefill": ([_P, C.POINTER(C.c_int), _I, _I, _P, C.POINTER(C.c_int)], C.c_int),

    "q48h_gemv_sweep": ([_P, _I, C.POINTER(C.c_int), C.POINTER(C.c_double)], C.c_int),
    "q48h_decode_graph": ([_P, _I, _I, _I, C.POINTER(C.c_int), C.POINTER(Stats)], C.c_int),
    "q48h_decode_graph_hashed": ([_P, _I, _I, _I, C.POINTER(C.c_int), C.POINTER(C.c_uint64),
                                  C.POINTER(Stats)], C.c_int),
    "q48s_fill_named": ([_P, C.c_int64, C.c_int64, C.c_uint64, C.c_char_p, C.c_int64, _I, _I],
                        None),
    "q48s_fnv_i64": ([C.c_uint64, _P, C.c_size_t], C.c_uint64),
}

FNV_OFFSET = 1469598103934665603


def synth(name: str, rows: int, cols: int, seed: int, sigma: int, bf16: int,
          threads: int = 8) -> np.ndarray:
    """The host library's synthetic tensor `name` (q48_synth.h), flattened."""
    a = np.empty(rows * cols, dtype=np.int64)
    host_lib().q48s_fill_named(a.ctypes.data, rows, cols, seed, name.encode(), sigma, bf16,
                               threads)
    return a


def fnv(arr) -> str:
    """FNV-1a-64 of an int64 array (the hash the golden vectors record)."""
    a = np.ascontiguousarray(arr, dtype=np.int64)
    return "%016x" % host_lib().q48s_fnv_i64(FNV_OFFSET, a.ctypes.data, a.size)


def host_lib() -> C.CDLL:
    """libq48host.so (loads libintllm_hip.so first; raises if not built)."""
    global _host
    if _host is None:
        hip_lib()
        _require(HOST_LIB)
        lib = C.CDLL(str(HOST_LIB))
        for name, (args, res) in HOST_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _host = lib
    return _host


class HostModel:
    """q48h_model: device-resident weights + KV cache driven by the C host."""

    def __init__(self, ctx: Context, cfg: Config | None = None, *, mgw: str | None = None,
                 max_seq: int = 0):
        h = C.c_void_p()
        if mgw is not None:
            check("q48h_model_load_mgw",
                  host_lib().q48h_model_load_mgw(C.byref(h), ctx.h, mgw.encode(), max_seq))
        else:
            check("q48h_model_create", host_lib().q48h_model_create(C.byref(h), ctx.h, C.byref(cfg)))
        self.h, self.ctx = h.value, ctx
        self.cfg = cfg

    def free(self):
        if self.h:
            host_lib().q48h_model_free(self.h)
            self.h = None

    def synth(self, seed: int, threads: int = 8):
        check("q48h_model_synth", host_lib().q48h_model_synth(self.h, seed, threads))

    def upload(self, name: str, arr):
        a = i64(arr).ravel()
        check("q48h_upload", host_lib().q48h_upload(self.h, name.encode(), a.ctypes.data, a.size))

    def kv_fill_synth(self, seed: int, npos: int, threads: int = 8):
        check("q48h_kv_fill_synth", host_lib().q48h_kv_fill_synth(self.h, seed, npos, threads))

    def kv_pointers(self):
        return host_lib().q48h_kv_keys(self.h), host_lib().q48h_kv_values(self.h)

    def forward(self, token: int, pos: int, vocab: int, logits: bool = True,
                choose: bool = True):
        """llama_forward; with choose, also the next token (argmax, or a
        sample_token draw when sampling is set); else next is None."""
        out = np.empty(vocab, dtype=np.int64) if logits else None
        nxt = C.c_int()
        check("q48h_forward", host_lib().q48h_forward(
            self.h, token, pos, out.ctypes.data if logits else None,
            C.byref(nxt) if choose else None))
        return (nxt.value if choose else None), out

    def prefill(self, tokens, p0: int, vocab: int, logits: bool = True, choose: bool = True):
        """q48h_prefill: tokens at positions p0.. in one batched pass; returns
        (next token or None, the T logits rows or None)."""
        T = len(tokens)
        t = (C.c_int * T)(*tokens)
        out = np.empty((T, vocab), dtype=np.int64) if logits else None
        nxt = C.c_int()
        check("q48h_prefill", host_lib().q48h_prefill(
            self.h, t, T, p0, out.ctypes.data if logits else None,
            C.byref(nxt) if choose else None))
        return (nxt.value if choose else None), out

    def set_batched_prefill(self, on: bool):
        """generate's prompt in one batched pass (default) or per token."""
        host_lib().q48h_model_set_batched_prefill(self.h, int(bool(on)))

    def set_gemm_planes(self, on: bool):
        """The batched prefill through prepared weight planes (default) or
        splitting W in each GEMM (and freeing the planes)."""
        host_lib().q48h_model_set_gemm_planes(self.h, int(bool(on)))

    def kv_reset(self):
        check("q48h_kv_reset", host_lib().q48h_kv_reset(self.h))

    def generate(self, prompt, max_new: int, hashes: bool = True):
        p = (C.c_int * len(prompt))(*prompt)
        cap = len(prompt) + max_new + 1
        out = (C.c_int * cap)()
        hs = (C.c_uint64 * cap)() if hashes else None
        n = C.c_int()
        st = Stats()
        total = check("q48h_generate", host_lib().q48h_generate(
            self.h, p, len(prompt), max_new, out, hs, C.byref(n), C.byref(st)))
        return list(out[:total]), (list(hs[:n.value]) if hashes else None), st

    def set_prefetch(self, on: bool):
        """Warm the device cache with each layer's W_o during its attention."""
        host_lib().q48h_model_set_prefetch(self.h, int(bool(on)))

    def set_rope_gemv(self, on: bool):
        """RoPE and the KV store in the q|k|v projection, attention from the
        cache (short context, mode 3); off: RoPE inside attention."""
        host_lib().q48h_model_set_rope_gemv(self.h, int(bool(on)))


    def read_logits(self) -> np.ndarray:
        """The logits of the last step run on the device."""
        out = np.empty(self.cfg.vocab, dtype=np.int64)
        check("q48h_read_logits", host_lib().q48h_read_logits(self.h, out.ctypes.data))
        return out

    def set_bf16(self, on: bool):
        """Read the projection matrices and lm_head as bfloat16 bits (mode 3)."""
        check("q48h_model_set_bf16", host_lib().q48h_model_set_bf16(self.h, int(bool(on))))

    def set_sampling(self, temperature: int, top_k: int = 0, top_p: int = 1 << 48,
                     seed: int = 0):
        """sample_token instead of argmax (temperature >= ONE / 100); the rng
        is seeded by rng_seed(seed)."""
        check("q48h_model_set_sampling", host_lib().q48h_model_set_sampling(
            self.h, int(temperature), int(top_k), int(top_p), int(seed) & ((1 << 64) - 1)))

    def set_fused(self, mode: int):
        """0: one op per reference step; 1: fused with per-block norm
        statistics; 2: fused with producer-side statistics; 3 (default):
        fused with producer partial sums finished by each consumer block."""
        host_lib().q48h_model_set_fused(self.h, int(mode))

    def decode_graph(self, token: int, start_pos: int, n: int):
        """n greedy steps replayed from a captured graph; returns (tokens up
        to and including the first EOS, all n step tokens, stats)."""
        out = (C.c_int * max(1, n))()
        st = Stats()
        k = check("q48h_decode_graph", host_lib().q48h_decode_graph(
            self.h, token, start_pos, n, out, C.byref(st)))
        return list(out[:k]), list(out[:n]), st

    def decode_graph_hashed(self, token: int, start_pos: int, n: int):
        """decode_graph with every replayed step's logits recorded on the
        device and hashed: (tokens up to and including the first EOS, all
        replayed step tokens, their logits FNVs as 16-digit hex, stats)."""
        out = (C.c_int * max(1, n))()
        hs = (C.c_uint64 * max(1, n))()
        st = Stats()
        k = check("q48h_decode_graph_hashed", host_lib().q48h_decode_graph_hashed(
            self.h, token, start_pos, n, out, hs, C.byref(st)))
        ms = self.cfg.max_seq if self.cfg is not None else start_pos + n
        ran = max(0, min(n, ms - start_pos))
        return list(out[:k]), list(out[:ran]), ["%016x" % h for h in hs[:ran]], st

    def gemv_sweep(self, reps: int):
        """Enqueue the decode GEMV sequence `reps` times: (launches, bytes)."""
        n, b = C.c_int(), C.c_double()
        check("q48h_gemv_sweep", host_lib().q48h_gemv_sweep(self.h, reps, C.byref(n), C.byref(b)))
        return n.value, b.value

    def decode_from(self, token: int, start_pos: int, n: int, hashes: bool = True):
        out = (C.c_int * max(1, n))()
        hs = (C.c_uint64 * max(1, n))() if hashes else None
        st = Stats()
        steps = check("q48h_decode_from", host_lib().q48h_decode_from(
            self.h, token, start_pos, n, out, hs, C.byref(st)))
        return list(out[:steps]), (list(hs[:steps]) if hashes else None), st


def gpu_available() -> bool:
    """True when a HIP device is visible (does not initialise HIP)."""
    if os.environ.get("HIP_VISIBLE_DEVICES", None) == "":
        return False
    return os.path.exists("/dev/kfd")


def rng_seed(seed: int) -> list:
    """rng_seed (llama_int.c:2909-2920): the 2-word xoroshiro128+ state."""
    st = (C.c_uint64 * 2)()
    hip_lib().q48_rng_seed(int(seed) & ((1 << 64) - 1), st)
    return [st[0], st[1]]
