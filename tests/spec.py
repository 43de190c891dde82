"""Shared definitions of the parity workloads (seeds, shapes, inputs).

Used by the golden-vector generator (tests/golden/make_golden.py), the
tests and bench.py, so every side builds bit-identical inputs.  Weight
tensors come from the synthetic generator of int-llm_amd/host/q48_synth.h
(passed in as `synth`, a function (name, rows, cols, seed, sigma, bf16)
-> int64 array); this module holds only the parameters.

Configurations:
  1  TINY        2 layers, d=256, 8/2 heads, hd 32, ffn 688, vocab 512
  2  GEMV        TinyLlama-1.1B matrix shapes, batch 1
  3  TINYLLAMA   22 layers, d=2048, 32/4 heads, hd 64, ffn 5632, vocab 32000
  4  GEMM        config-2 shapes with T in {128, 512, 2048} tokens
  5  LONGCTX     TINYLLAMA with a KV cache pre-filled to 2048 positions,
                 then 256 greedy decode steps (max_seq 4096 >= 2304)
"""
from __future__ import annotations

import numpy as np

ONE = 1 << 48
HALF = 1 << 47
M64 = (1 << 64) - 1
INT64_MIN, INT64_MAX = -(1 << 63), (1 << 63) - 1

SIGMA_W = ONE // 50      # 0.02, weights (bf16-rounded)
SIGMA_ACT = ONE          # 1.0, activations (raw Q16.48) and KV contents (bf16)

# (dim, n_heads, n_kv_heads, head_dim, n_layers, ffn, vocab, max_seq, rope_theta)
TINY = (256, 8, 2, 32, 2, 688, 512, 2048, 10000)
TINYLLAMA = (2048, 32, 4, 64, 22, 5632, 32000, 2048, 10000)
LONGCTX = (2048, 32, 4, 64, 22, 5632, 32000, 4096, 10000)

SEED_TINY = 0x5EED0001
SEED_GEMV = 0x5EED0002
SEED_TL = 0x5EED0003
SEED_OPS = 0x5EED0009
SEED_KV = 0x5EED0055

LONG_PREFILL = 2048
LONG_STEPS = 256
LONG_TOKEN = 1            # BOS id (llama_int.c:3044)

# config 2 (M = output rows, K = input length); q/o, k/v, gate/up, down, lm_head
GEMV_SHAPES = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (32000, 2048)]
# fused projections of the decode path (q|k|v and gate|up stacked)
GEMV_FUSED = [(2560, 2048), (11264, 2048)]
GEMM_TOKENS = [128, 512, 2048]

# (head_dim, max_seq, theta) of rope_init tables pinned by golden vectors
ROPE_TABLES = [(32, 64, 10000), (32, 2048, 10000), (64, 2048, 10000), (64, 4096, 10000)]


def _splitmix64(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _xorshift(s: int) -> int:
    s ^= (s << 13) & M64
    s ^= s >> 7
    s ^= (s << 17) & M64
    return s


def prompt(seed: int, n: int, vocab: int) -> list[int]:
    """Seeded prompt of n ids in [3, vocab) (q48s_tokens with seed ^ golden)."""
    s = _splitmix64((seed ^ 0x9E3779B97F4A7C15) & M64) or 0x2545F4914F6CDD1D
    out = []
    for _ in range(n):
        s = _xorshift(s)
        out.append(3 + s % (vocab - 3))
    return out


def gemv_w_name(M: int, K: int) -> str:
    return f"gemv.W.{M}x{K}"


def gemv_x_name(K: int) -> str:
    return f"gemv.x.{K}"


def gemm_x_name(T: int, K: int) -> str:
    return f"gemm.X.{T}x{K}"


def gemv_inputs_ref(synth, M: int, K: int):
    W = synth(gemv_w_name(M, K), M, K, SEED_GEMV, SIGMA_W, 1)
    x = synth(gemv_x_name(K), 1, K, SEED_GEMV, SIGMA_ACT, 0)
    return W, x


def _rand64(rng: np.random.Generator, n: int) -> np.ndarray:
    return rng.integers(INT64_MIN, INT64_MAX, size=n, dtype=np.int64, endpoint=True)


def gemv_edge_cases():
    """Small GEMVs whose operands hit the int64 extremes, odd K, K tails.

    Products up to 2^126 and sums that wrap mod 2^128 are exactly where a
    dropped carry, a sign slip or an int64 (instead of int128) accumulator
    would show."""
    rng = np.random.default_rng(1234)
    ext = np.array([INT64_MIN, INT64_MAX, INT64_MIN + 1, -1, 1, 0, -(1 << 62), (1 << 62),
                    ONE, -ONE, (1 << 32) - 1, -(1 << 32)], dtype=np.int64)
    cases = []
    for (M, K) in [(1, 1), (3, 7), (4, 12), (2, 129), (5, 64), (7, 131), (9, 688 // 8)]:
        W = _rand64(rng, M * K)
        x = _rand64(rng, K)
        W[: min(M * K, ext.size)] = ext[: min(M * K, ext.size)]
        x[: min(K, ext.size)] = ext[::-1][: min(K, ext.size)]
        cases.append((M, K, W, x))
    # all-extreme: every product is +-2^126-ish, the sum wraps repeatedly
    K = 130
    W = np.full(4 * K, INT64_MIN, dtype=np.int64)
    W[K:2 * K] = INT64_MAX
    W[2 * K:3 * K] = np.where(np.arange(K) % 2, INT64_MIN, INT64_MAX)
    W[3 * K:] = -1
    x = np.where(np.arange(K) % 3 == 0, INT64_MIN, INT64_MAX).astype(np.int64)
    cases.append((4, K, W, x))
    return cases


def gemv_exact(W: np.ndarray, x: np.ndarray, M: int, K: int) -> np.ndarray:
    """Textbook definition with Python integers: (sum W x) >> 48, wrapped
    to int64 the way a C cast of the int128 sum does."""
    y = np.empty(M, dtype=np.int64)
    xs = [int(v) for v in x]
    for i in range(M):
        s = sum(int(w) * xv for w, xv in zip(W[i * K:(i + 1) * K], xs))
        s = ((s + (1 << 127)) % (1 << 128)) - (1 << 127)   # int128 wrap
        v = (s >> 48) & M64                                 # floor shift, low 64 bits
        y[i] = v - (1 << 64) if v >> 63 else v
    return y


def det_grid() -> list[int]:
    """build_grid of fp_determinism.c:101-137, in Python."""
    g = [0, ONE, -ONE, HALF, -HALF, 1, -1, ONE + 1, ONE - 1, 32000 << 48, -(32000 << 48),
         181 << 48, 7 << 48, -(7 << 48), 2 << 48, 10 << 48]
    for e in range(-44, 15):
        p = (ONE << e) if e >= 0 else (ONE >> (-e))
        g += [p, -p]
    st = 0x9E3779B97F4A7C15
    span = 32000 << 48
    for _ in range(4096):
        st = _xorshift(st)
        mag = st % span
        g.append(mag if st & 1 else -mag)
    return g


def wrap64(v: int) -> int:
    v &= M64
    return v - (1 << 64) if v >> 63 else v


def pos_of(x: int) -> int:
    """fp_determinism.c:141-146 (int64 arithmetic: |INT64_MIN| wraps)."""
    a = wrap64(-x if x < 0 else x)
    if a < 1024:
        a = wrap64(a + 1024)
    return a


def exp_arg(x: int) -> int:
    """fp_determinism.c:149-153"""
    forty = 40 << 48
    return ((x & M64) % forty) - (20 << 48)


def fp_inputs():
    """The determinism grid plus int64 extremes, with the gate's partner
    pairing y[i] = g[(7 i + 3) % n]."""
    g = det_grid() + [INT64_MIN, INT64_MAX, INT64_MIN + 1, INT64_MAX - 1, -(1 << 62), 1 << 62,
                      (10 << 48) + 1, -(10 << 48) - 1, 10 << 48, -(10 << 48)]
    n = len(g)
    x = np.array(g, dtype=np.int64)
    y = np.array([g[(i * 7 + 3) % n] for i in range(n)], dtype=np.int64)
    return x, y


def rmsnorm_inputs(synth, dim: int):
    x = synth(f"rmsnorm.x.{dim}", 1, dim, SEED_OPS, SIGMA_ACT, 0)
    w = synth(f"rmsnorm.w.{dim}", 1, dim, SEED_OPS, SIGMA_W, 1)
    return x, w


def softmax_inputs(synth, n: int):
    """Scores of spread ~4 so the +-10 clamp of fp_safe_exp is exercised."""
    return synth(f"softmax.x.{n}", 1, n, SEED_OPS, 4 * ONE, 0)


# ---- sampling (sample_token, llama_int.c:2958-3039) ------------------------
SAMPLE_KINDS = ("gauss", "ties", "peaked", "extreme")


def sample_logits(kind: str, seed: int, n: int) -> np.ndarray:
    """Deterministic logits for the sampling cases, from integer draws only
    (identical on every host):
      gauss    sum of four uniforms, spread about 3.0
      ties     eight distinct levels: top-k thresholds and nucleus cuts
               fall inside runs of equal values
      peaked   one dominant logit (+12) over a spread of about 1.0
      extreme  large magnitudes (up to +-30000) and the int64 extremes:
               temperature division wraps, exp clamps at +-10"""
    rng = np.random.default_rng(seed)
    u = rng.integers(-(ONE // 2), ONE // 2, size=(4, n), dtype=np.int64)
    if kind == "gauss":
        return (u.sum(axis=0) * 3).astype(np.int64)
    if kind == "ties":
        lv = rng.integers(-4 * ONE, 4 * ONE, size=8, dtype=np.int64)
        return lv[rng.integers(0, 8, size=n)]
    if kind == "peaked":
        v = u.sum(axis=0)
        v[rng.integers(0, n)] += 12 * ONE
        return v.astype(np.int64)
    v = (u.sum(axis=0) * 30000).astype(np.int64)
    v[rng.integers(0, n, size=4)] = [INT64_MAX, INT64_MIN, INT64_MAX - 1, 1]
    return v


# (temperature, top_k, top_p) in Q16.48 / counts; None top_k = n - 1
SAMPLE_TEMPS = [0, ONE // 200, ONE // 100, ONE * 3 // 10, ONE * 7 // 10, ONE,
                ONE * 3 // 2, 3 * ONE]
SAMPLE_TOPK = [0, 1, 2, 10, 50, None]
SAMPLE_TOPP = [0, ONE // 20, ONE // 2, ONE * 9 // 10, ONE - ONE // 1000, ONE]

# generate() with sampling on the tiny model: (temperature, top_k, top_p, seed)
SAMPLE_GEN = [(ONE * 8 // 10, 40, ONE * 9 // 10, 7), (ONE, 0, ONE, 11),
              (ONE // 2, 5, ONE // 2, 3), (ONE * 3 // 2, 0, ONE * 95 // 100, 12345)]
SAMPLE_GEN_TL = (ONE * 8 // 10, 40, ONE * 9 // 10, 2024)
