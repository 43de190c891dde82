"""Loader of the CPU oracle (oracle/liboracle_q48.so) for tests and bench.

The oracle is test infrastructure: the checker the HIP library is compared
against.  Nothing in the product imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle_q48.so"
REF_SO = ROOT / "oracle" / "_ref" / "libq48_ref.so"
FNV_OFF = 1469598103934665603

P, I, U, I64 = C.c_void_p, C.c_int, C.c_uint64, C.c_int64


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in
                ("dim", "n_heads", "n_kv_heads", "head_dim", "n_layers", "ffn",
                 "vocab", "max_seq", "rope_theta")]


_SIG = {
    "q48o_fp_mul": ([I64, I64], I64), "q48o_fp_div": ([I64, I64], I64),
    "q48o_fp_from_int": ([I], I64), "q48o_fp_sqrt": ([I64], I64),
    "q48o_fp_sqrt_fast": ([I64], I64), "q48o_fp_inv_sqrt": ([I64], I64),
    "q48o_fp_exp_dyadic": ([I64, I], I64), "q48o_fp_exp": ([I64], I64),
    "q48o_fp_safe_exp": ([I64], I64), "q48o_fp_log": ([I64], I64),
    "q48o_fp_sincos": ([I64, C.POINTER(I64), C.POINTER(I64)], None),
    "q48o_fp_sigmoid": ([I64], I64), "q48o_fp_silu": ([I64], I64),
    "q48o_fp_consts": ([C.POINTER(I64), C.POINTER(I64), P], None),
    "q48o_determinism": ([P], U), "q48o_det_grid": ([P, I], I),
    "q48o_gemv": ([P, P, P, I, I], None), "q48o_gemm": ([P, P, P, I, I, I], None),
    "q48o_rmsnorm": ([P, P, P, I], None),
    "q48o_rope_tables": ([P, P, I, I, I], None),
    "q48o_rope_apply": ([P, P, I, P, I], None),
    "q48o_softmax": ([P, I], None),
    "q48o_attn_decode": ([P, P, P, P, P, P, I, I, I, I, I, I], None),
    "q48o_silu_mul": ([P, P, P, I], None), "q48o_argmax": ([P, I], I),
    "q48o_model_synth": ([C.POINTER(Config), U, I], P),
    "q48o_model_free": ([P], None), "q48o_model_tensor": ([P, C.c_char_p], P),
    "q48o_kv_reset": ([P], None), "q48o_kv_fill_synth": ([P, U, I, I], None),
    "q48o_kv_keys": ([P], P), "q48o_kv_values": ([P], P),
    "q48o_layer_forward": ([P, I, I, P], None),
    "q48o_forward": ([P, I, I, P], I),
    "q48o_generate": ([P, P, I, I, P, P, P], I),
    "q48o_decode_from": ([P, I, I, I, P, P], I),
    "q48o_rng_seed": ([U, P], None), "q48o_rng_next": ([P], U),
    "q48o_sample": ([P, I, I64, I, I64, P], I),
    "q48o_generate_sampled": ([P, P, I, I, P, P, P, I64, I, I64, U], I),
    "q48s_fill": ([P, I64, I64, U, I64, I, I], None),
    "q48s_tensor_seed": ([U, C.c_char_p], U),
    "q48s_fnv_i64": ([U, P, C.c_size_t], U),
    "q48s_bf16_to_q48": ([C.c_uint16], I64), "q48s_q48_to_bf16": ([I64], C.c_uint16),
    "q48s_f16_to_q48": ([C.c_uint16], I64),
}

_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            subprocess.check_call(["make", "-s", "-C", str(ROOT / "oracle"), "liboracle_q48.so"])
        lib = C.CDLL(str(ORACLE_SO))
        for name, (args, res) in _SIG.items():
            f = getattr(lib, name)
            f.argtypes, f.restype = args, res
        _lib = lib
    return _lib


def threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def synth(name: str, rows: int, cols: int, seed: int, sigma: int, bf16: int) -> np.ndarray:
    """The q48_synth.h tensor `name` (rows x cols, flattened int64)."""
    lib = load()
    a = np.empty(rows * cols, dtype=np.int64)
    lib.q48s_fill(a.ctypes.data, rows, cols, lib.q48s_tensor_seed(seed, name.encode()),
                  sigma, bf16, threads())
    return a


def fnv(arr) -> str:
    a = np.ascontiguousarray(arr, dtype=np.int64)
    return "%016x" % load().q48s_fnv_i64(FNV_OFF, a.ctypes.data, a.size)


def gemv(W, x, M, K) -> np.ndarray:
    y = np.empty(M, dtype=np.int64)
    W = np.ascontiguousarray(W, dtype=np.int64)
    x = np.ascontiguousarray(x, dtype=np.int64)
    load().q48o_gemv(y.ctypes.data, W.ctypes.data, x.ctypes.data, M, K)
    return y


class Model:
    """Oracle model with synthetic weights (q48o_model)."""

    def __init__(self, cfg_tuple, seed: int):
        self.cfg = Config(*cfg_tuple)
        self.h = load().q48o_model_synth(C.byref(self.cfg), seed, threads())

    def free(self):
        if self.h:
            load().q48o_model_free(self.h)
            self.h = None

    def tensor(self, name: str, n: int) -> np.ndarray:
        p = load().q48o_model_tensor(self.h, name.encode())
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_int64)), shape=(n,)).copy()

    def generate(self, prompt, max_new):
        cap = len(prompt) + max_new + 1
        p = (C.c_int * len(prompt))(*prompt)
        out = (C.c_int * cap)()
        hs = (C.c_uint64 * cap)()
        n = C.c_int()
        total = load().q48o_generate(self.h, p, len(prompt), max_new, out, hs, C.byref(n))
        return list(out[:total]), ["%016x" % v for v in hs[:n.value]]

    def generate_sampled(self, prompt, max_new, temperature, top_k, top_p, seed):
        cap = len(prompt) + max_new + 1
        p = (C.c_int * len(prompt))(*prompt)
        out = (C.c_int * cap)()
        hs = (C.c_uint64 * cap)()
        n = C.c_int()
        total = load().q48o_generate_sampled(self.h, p, len(prompt), max_new, out, hs,
                                             C.byref(n), temperature, top_k, top_p, seed)
        return list(out[:total]), ["%016x" % v for v in hs[:n.value]]

    def forward(self, token, pos):
        lg = np.empty(self.cfg.vocab, dtype=np.int64)
        rc = load().q48o_forward(self.h, token, pos, lg.ctypes.data)
        return rc, lg

    def decode_from(self, token, start, n):
        out = (C.c_int * n)()
        hs = (C.c_uint64 * n)()
        steps = load().q48o_decode_from(self.h, token, start, n, out, hs)
        return list(out[:steps]), ["%016x" % v for v in hs[:steps]]


def rng_seed(seed: int) -> list[int]:
    s = (C.c_uint64 * 2)()
    load().q48o_rng_seed(seed & ((1 << 64) - 1), s)
    return [s[0], s[1]]


def sample(logits: np.ndarray, temperature: int, top_k: int, top_p: int, state: list[int]):
    """sample_token on the oracle: (token, state after)."""
    s = (C.c_uint64 * 2)(*state)
    x = np.ascontiguousarray(logits, dtype=np.int64)
    tok = load().q48o_sample(x.ctypes.data, x.size, temperature, top_k, top_p, s)
    return tok, [s[0], s[1]]
