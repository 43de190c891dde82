/*
 * q48_oracle.c — CPU oracle (TEST INFRASTRUCTURE ONLY; see q48_oracle.h).
 *
 * A plain-C restatement of the reference's exact Q16.48 arithmetic:
 *   fp_math.h          (native __int128 backend semantics, fp_math.h:184-290)
 *   llama_int.c        matmul_vec, rmsnorm, rope, softmax, exact attention,
 *                      SwiGLU, transformer layer, llama_forward, generate
 *   fp_determinism.c   the bit-exact gate over the fixed input grid
 * Build with -fwrapv (Makefile:32-39): signed int64 adds wrap.
 *
 * Parity status (what pins each function; tests/test_oracle_*.py):
 *   fp_* primitives      determinism golden c0d933ea340452ec + 12 sub-hashes
 *   gemv / gemm          Python big-int brute force + reference harness
 *   rmsnorm, rope, softmax, attention, silu_mul
 *                        reference harness (oracle/_ref) on seeded inputs
 *   forward / generate   reference harness: per-step logits FNV + tokens
 */
#include "q48_oracle.h"
#include "../int-llm_amd/host/q48_synth.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

#define ONE  ((int64_t)1 << 48)
#define HALF ((int64_t)1 << 47)

/* ======================================================================
 * fp_math.h
 * ==================================================================== */

/* fp_mul, fp_math.h:491-506: (int128)a*b >> 48 (arithmetic), truncated. */
int64_t q48o_fp_mul(int64_t a, int64_t b)
{
    return (int64_t)(((i128)a * b) >> 48);
}

/* fp_w_divs, fp_math.h:249-256: truncating signed division, b == -1 wraps. */
static i128 w_divs(i128 a, i128 b)
{
    if (b == -1)
        return (i128)(0 - (u128)a);
    return a / b;
}

/* fp_div, fp_math.h:508-524: sign(a) * ((|a| << 48) / b), truncating. */
int64_t q48o_fp_div(int64_t a, int64_t b)
{
    uint64_t mag = a < 0 ? (uint64_t)0 - (uint64_t)a : (uint64_t)a;
    i128 num = (i128)((u128)mag << 48);
    if (a < 0)
        num = (i128)(0 - (u128)num);
    return (int64_t)w_divs(num, (i128)b);
}

/* fp_from_int, fp_math.h:530-538. */
int64_t q48o_fp_from_int(int x)
{
    uint64_t mag = x < 0 ? (uint64_t)0 - (uint64_t)(int64_t)x : (uint64_t)x;
    u128 r = (u128)mag << 48;
    if (x < 0)
        r = 0 - r;
    return (int64_t)r;
}

static int64_t fp_abs(int64_t a) { return a >= 0 ? a : -a; }

/* fp_sqrt_fast, fp_math.h:605-622: 64-bit Newton isqrt, r << 24. */
int64_t q48o_fp_sqrt_fast(int64_t x)
{
    if (x <= 0)
        return 0;
    uint64_t ux = (uint64_t)x;
    int bw = 64 - __builtin_clzll(ux);
    uint64_t r = (uint64_t)1 << ((bw + 1) / 2);
    for (int i = 0; i < 5; ++i) {
        uint64_t nr = (r + ux / r) >> 1;
        if (nr >= r)
            break;
        r = nr;
    }
    return (int64_t)(r << 24);
}

/* fp_sqrt, fp_math.h:626-652: Newton on isqrt(x << 48), then r^2 <= n. */
int64_t q48o_fp_sqrt(int64_t x)
{
    if (x <= 0)
        return 0;
    i128 n = (i128)((u128)(uint64_t)x << 48);
    uint64_t hi = (uint64_t)((u128)n >> 64), lo = (uint64_t)n;
    int bw = hi ? 128 - __builtin_clzll(hi) : (lo ? 64 - __builtin_clzll(lo) : 0);
    uint64_t r = (uint64_t)1 << ((bw + 1) / 2);
    for (int i = 0; i < 7; ++i) {
        if (r == 0)
            return 0;
        uint64_t q = (uint64_t)(int64_t)w_divs(n, (i128)r);
        uint64_t nr = (r + q) >> 1;
        if (nr >= r)
            break;
        r = nr;
    }
    while ((i128)(int64_t)r * (int64_t)r > n)
        r--;
    return (int64_t)r;
}

/* fp_inv_sqrt, fp_math.h:658-707: range reduction to [2^48, 2^50),
 * sub-octave initial guess, 8 Newton steps y*(3 - x*y^2)/2, y <= 0 -> 1,
 * rescale by 2^-k with saturation. */
int64_t q48o_fp_inv_sqrt(int64_t x)
{
    if (x <= 0)
        return 0;
    int msb = 63 - __builtin_clzll((uint64_t)x);
    int k = (msb - 48) >> 1;
    int64_t xn = k >= 0 ? (x >> (2 * k)) : (int64_t)((uint64_t)x << (-2 * k));
    int msb_n = 63 - __builtin_clzll((uint64_t)xn);
    int64_t y = msb_n == 48 ? ONE : HALF;
    int64_t three = q48o_fp_from_int(3);
    for (int i = 0; i < 8; ++i) {
        int64_t y2 = (int64_t)(((i128)y * y) >> 48);
        int64_t xy2 = (int64_t)(((i128)xn * y2) >> 48);
        int64_t factor = three - xy2;
        y = (int64_t)(((i128)y * factor) >> 49);
        if (y <= 0) {
            y = 1;
            break;
        }
    }
    if (k >= 0) {
        int64_t r = y >> k;
        return r < 0 ? 0 : r;
    }
    i128 r = (i128)((u128)(i128)y << (-k));
    if (r > (i128)INT64_MAX)
        return INT64_MAX;
    if (r < 0)
        return 0;
    return (int64_t)r;
}

/* fp_exp_dyadic, fp_math.h:714-720: (1 + x/2^k)^(2^k) by k squarings. */
int64_t q48o_fp_exp_dyadic(int64_t x, int k)
{
    int64_t base = ONE + (x >> k);
    int64_t r = base;
    for (int i = 0; i < k; ++i)
        r = q48o_fp_mul(r, r);
    return r;
}

/* fp_exp, fp_math.h:724-732: k = 14; negatives through fp_div(ONE, e^-x). */
int64_t q48o_fp_exp(int64_t x)
{
    if (x >= 0)
        return q48o_fp_exp_dyadic(x, 14);
    int64_t pos = q48o_fp_exp_dyadic(-x, 14);
    if (pos == 0)
        return 0;
    return q48o_fp_div(ONE, pos);
}

/* fp_safe_exp, fp_math.h:739-744: clamp to 10, below -10 -> 0. */
int64_t q48o_fp_safe_exp(int64_t x)
{
    int64_t max_x = q48o_fp_from_int(10);
    if (x > max_x)
        x = max_x;
    if (x < -max_x)
        return 0;
    return q48o_fp_exp(x);
}

/* fp_log, fp_math.h:752-773: CLZ guess, Newton y - 1 + x/e^y, 10 steps. */
int64_t q48o_fp_log(int64_t x)
{
    if (x <= 0)
        return -q48o_fp_from_int(50);
    const int64_t ln2 = 195103586505167LL;
    int lz = __builtin_clzll((uint64_t)x);
    int log2_approx = 63 - lz - 48;
    int64_t y = (int64_t)log2_approx * ln2;
    for (int i = 0; i < 10; ++i) {
        int64_t ey = q48o_fp_exp(y);
        if (ey == 0)
            break;
        int64_t y_new = y - ONE + q48o_fp_div(x, ey);
        int64_t diff = fp_abs(y_new - y);
        if (diff < 2)
            break;
        y = y_new;
    }
    return y;
}

/* fp_atan_taylor, fp_math.h:789-800 (C truncating int64 division). */
static int64_t fp_atan_taylor(int64_t x, int max_terms)
{
    int64_t x_sq = q48o_fp_mul(x, x);
    int64_t term = x, sum = x;
    for (int n = 1; n <= max_terms; ++n) {
        term = -q48o_fp_mul(term, x_sq);
        int64_t c = term / (2 * n + 1);
        if (c == 0)
            break;
        sum += c;
    }
    return sum;
}

static int64_t g_pi, g_gain, g_angles[48];
static int g_init;

/* fp_compute_pi (fp_math.h:804-812), fp_atan_pow2 (:823-827) and
 * fp_math_init (:833-858): Machin pi, CORDIC angles, gain 1/sqrt(K^2). */
static void fp_math_init(void)
{
    if (g_init)
        return;
    int64_t atan5 = fp_atan_taylor(ONE / 5, 40);
    int64_t atan239 = fp_atan_taylor(ONE / 239, 15);
    g_pi = (int64_t)((uint64_t)atan5 << 4) - (int64_t)((uint64_t)atan239 << 2);
    g_angles[0] = g_pi >> 2;
    for (int i = 1; i < 48; ++i)
        g_angles[i] = i >= 25 ? (ONE >> i) : fp_atan_taylor(ONE >> i, 40);
    int64_t k_sq = ONE;
    for (int i = 0; i < 48; ++i) {
        int64_t sv = (2 * i < 63) ? (ONE >> (2 * i)) : 0;
        k_sq = q48o_fp_mul(k_sq, ONE + sv);
    }
    g_gain = q48o_fp_div(ONE, q48o_fp_sqrt(k_sq));
    g_init = 1;
}

void q48o_fp_consts(int64_t *pi, int64_t *gain, int64_t *angles48)
{
    fp_math_init();
    if (pi)
        *pi = g_pi;
    if (gain)
        *gain = g_gain;
    if (angles48)
        memcpy(angles48, g_angles, sizeof g_angles);
}

/* fp_sincos, fp_math.h:861-902: reduce to [-pi, pi], fold to |a| <= pi/2,
 * 48 CORDIC rotations from x = gain, y = 0. */
void q48o_fp_sincos(int64_t angle, int64_t *c, int64_t *s)
{
    fp_math_init();
    int64_t two_pi = (int64_t)((uint64_t)g_pi << 1);
    while (angle > g_pi)
        angle -= two_pi;
    while (angle < -g_pi)
        angle += two_pi;
    int64_t pi_half = g_pi >> 1;
    int neg_cos = 0;
    if (angle > pi_half) {
        angle = g_pi - angle;
        neg_cos = 1;
    } else if (angle < -pi_half) {
        angle = -g_pi - angle;
        neg_cos = 1;
    }
    int64_t x = g_gain, y = 0, z = angle;
    for (int i = 0; i < 48; ++i) {
        int64_t xs = x >> i, ys = y >> i;
        if (z >= 0) {
            int64_t xn = x - ys, yn = y + xs;
            z -= g_angles[i];
            x = xn;
            y = yn;
        } else {
            int64_t xn = x + ys, yn = y - xs;
            z += g_angles[i];
            x = xn;
            y = yn;
        }
    }
    *c = neg_cos ? -x : x;
    *s = y;
}

/* fp_sigmoid, fp_math.h:911-916. */
int64_t q48o_fp_sigmoid(int64_t x)
{
    if (x > q48o_fp_from_int(10))
        return ONE;
    if (x < -q48o_fp_from_int(10))
        return 0;
    int64_t en = q48o_fp_safe_exp(-x);
    return q48o_fp_div(ONE, ONE + en);
}

/* fp_silu, fp_math.h:919-921. */
int64_t q48o_fp_silu(int64_t x)
{
    return q48o_fp_mul(x, q48o_fp_sigmoid(x));
}

/* ======================================================================
 * fp_determinism.c
 * ==================================================================== */

#define FNV_OFF   1469598103934665603ULL
#define FNV_PRIME 1099511628211ULL

static uint64_t fnv_mix(uint64_t h, int64_t v)
{
    uint64_t u = (uint64_t)v;
    for (int b = 0; b < 8; ++b) {
        h ^= u & 0xff;
        h *= FNV_PRIME;
        u >>= 8;
    }
    return h;
}

/* build_grid, fp_determinism.c:101-137: 16 specials, +-2^e for
 * e in [-44, 14], 4096 xorshift values in [-32000, 32000]. */
int q48o_det_grid(int64_t *g, int cap)
{
    int n = 0;
#define PUSH(v) do { if (n < cap) g[n] = (v); n++; } while (0)
    uint64_t st = 0x9E3779B97F4A7C15ULL;
    PUSH(0); PUSH(ONE); PUSH(-ONE); PUSH(HALF); PUSH(-HALF);
    PUSH(1); PUSH(-1); PUSH(ONE + 1); PUSH(ONE - 1);
    PUSH((int64_t)32000 << 48); PUSH(-((int64_t)32000 << 48));
    PUSH((int64_t)181 << 48);
    PUSH(q48o_fp_from_int(7)); PUSH(q48o_fp_from_int(-7));
    PUSH(q48o_fp_from_int(2)); PUSH(q48o_fp_from_int(10));
    for (int e = -44; e <= 14; ++e) {
        int64_t p = e >= 0 ? (ONE << e) : (ONE >> (-e));
        PUSH(p);
        PUSH(-p);
    }
    const int64_t span = (int64_t)32000 << 48;
    for (int i = 0; i < 4096; ++i) {
        st ^= st << 13;
        st ^= st >> 7;
        st ^= st << 17;
        int64_t mag = (int64_t)(st % (uint64_t)span);
        PUSH((st & 1) ? mag : -mag);
    }
#undef PUSH
    return n;
}

/* pos_of / exp_arg, fp_determinism.c:141-153. */
static int64_t pos_of(int64_t x)
{
    int64_t a = fp_abs(x);
    if (a < 1024)
        a += 1024;
    return a;
}

static int64_t exp_arg(int64_t x)
{
    const int64_t forty = (int64_t)40 << 48;
    int64_t m = (int64_t)((uint64_t)x % (uint64_t)forty);
    return m - ((int64_t)20 << 48);
}

/* fp_det_compute, fp_determinism.c:162-244. */
uint64_t q48o_determinism(uint64_t subs[12])
{
    static int64_t grid[4352];
    int gn = q48o_det_grid(grid, 4352);
    uint64_t h[12];
    for (int i = 0; i < 12; ++i)
        h[i] = FNV_OFF;
    for (int i = 0; i < gn; ++i) {
        int j = (i * 7 + 3) % gn;
        int64_t x = grid[i], y = grid[j];
        h[0] = fnv_mix(h[0], q48o_fp_mul(x, y));
        if (y != 0)
            h[1] = fnv_mix(h[1], q48o_fp_div(x, y));
        int64_t xp = pos_of(x);
        h[2] = fnv_mix(h[2], q48o_fp_sqrt(xp));
        h[3] = fnv_mix(h[3], q48o_fp_sqrt_fast(xp));
        h[4] = fnv_mix(h[4], q48o_fp_inv_sqrt(xp));
        h[6] = fnv_mix(h[6], q48o_fp_log(xp));
        h[5] = fnv_mix(h[5], q48o_fp_exp(exp_arg(x)));
        int64_t c, s;
        q48o_fp_sincos(x, &c, &s);
        h[7] = fnv_mix(h[7], c);
        h[8] = fnv_mix(h[8], s);
        h[9] = fnv_mix(h[9], q48o_fp_sigmoid(x));
        h[10] = fnv_mix(h[10], q48o_fp_silu(x));
    }
    /* fp_rng_next / fp_rng_uniform (fp_math.h:929-940) from 0x123456789ABCDEF */
    uint64_t st = 0x123456789ABCDEFULL;
    for (int i = 0; i < 1024; ++i) {
        st ^= st << 13; st ^= st >> 7; st ^= st << 17;
        h[11] = fnv_mix(h[11], (int64_t)st);
        st ^= st << 13; st ^= st >> 7; st ^= st << 17;
        h[11] = fnv_mix(h[11], (int64_t)(st >> 16));
    }
    uint64_t comb = FNV_OFF;
    for (int i = 0; i < 12; ++i) {
        comb = fnv_mix(comb, (int64_t)h[i]);
        if (subs)
            subs[i] = h[i];
    }
    return comb;
}

/* ======================================================================
 * llama_int.c tensor ops
 * ==================================================================== */

/* matmul_vec, llama_int.c:1014-1046: out[i] = (int64)(sum_j (int128)
 * W[i][j] * in[j] >> 48).  The reference's 4-row unroll does not change
 * the sum; int128 adds wrap. */
void q48o_gemv(int64_t *y, const int64_t *W, const int64_t *x, int M, int K)
{
    for (int i = 0; i < M; ++i) {
        const int64_t *w = W + (int64_t)i * K;
        u128 acc = 0;
        for (int j = 0; j < K; ++j)
            acc += (u128)((i128)w[j] * x[j]);
        y[i] = (int64_t)((i128)acc >> 48);
    }
}

/* Batched prefill: every token row is matmul_vec of that row. */
void q48o_gemm(int64_t *Y, const int64_t *W, const int64_t *X,
               int T, int N, int K)
{
    for (int t = 0; t < T; ++t)
        q48o_gemv(Y + (int64_t)t * N, W, X + (int64_t)t * K, N, K);
}

/* rmsnorm, llama_int.c:1048-1058: ss = sum x^2 (int128); ms = (ss >> 48)
 * / dim (int128 division, truncating), + 2814749767 (1e-5); r = inv_sqrt;
 * out = fp_mul(fp_mul(x, r), w). */
void q48o_rmsnorm(int64_t *out, const int64_t *x, const int64_t *w, int dim)
{
    u128 ss = 0;
    for (int i = 0; i < dim; ++i)
        ss += (u128)((i128)x[i] * x[i]);
    int64_t ms = (int64_t)(((i128)ss >> 48) / dim);
    ms += (int64_t)2814749767LL;
    int64_t r = q48o_fp_inv_sqrt(ms);
    for (int i = 0; i < dim; ++i)
        out[i] = q48o_fp_mul(q48o_fp_mul(x[i], r), w[i]);
}

/* rope_init, llama_int.c:960-986: theta_i = exp(-(2i/hd) * ln(theta)),
 * angle = pos * theta_i, tables [max_seq][hd/2]. */
void q48o_rope_tables(int64_t *cos_t, int64_t *sin_t, int head_dim,
                      int max_seq, int theta)
{
    fp_math_init();
    int half = head_dim / 2;
    int64_t lt = q48o_fp_log(q48o_fp_from_int(theta));
    for (int i = 0; i < half; ++i) {
        int64_t nf = -q48o_fp_div(q48o_fp_from_int(2 * i), q48o_fp_from_int(head_dim));
        int64_t th = q48o_fp_exp(q48o_fp_mul(nf, lt));
        for (int p = 0; p < max_seq; ++p) {
            int64_t c, s;
            q48o_fp_sincos(q48o_fp_mul(q48o_fp_from_int(p), th), &c, &s);
            cos_t[(int64_t)p * half + i] = c;
            sin_t[(int64_t)p * half + i] = s;
        }
    }
}

/* rope_apply, llama_int.c:997-1008: half-split rotation of (i, i+half). */
void q48o_rope_apply(const int64_t *cos_t, const int64_t *sin_t, int half,
                     int64_t *vec, int pos)
{
    const int64_t *c = cos_t + (int64_t)pos * half;
    const int64_t *s = sin_t + (int64_t)pos * half;
    for (int i = 0; i < half; ++i) {
        int64_t x0 = vec[i], x1 = vec[i + half];
        vec[i] = q48o_fp_mul(x0, c[i]) - q48o_fp_mul(x1, s[i]);
        vec[i + half] = q48o_fp_mul(x1, c[i]) + q48o_fp_mul(x0, s[i]);
    }
}

/* softmax, llama_int.c:1060-1072: max, safe_exp(x - max), int64 sum,
 * fp_div by the sum only when it is positive. */
void q48o_softmax(int64_t *x, int n)
{
    int64_t mx = x[0];
    for (int i = 1; i < n; ++i)
        if (x[i] > mx)
            mx = x[i];
    int64_t sum = 0;
    for (int i = 0; i < n; ++i) {
        x[i] = q48o_fp_safe_exp(x[i] - mx);
        sum += x[i];
    }
    if (sum > 0)
        for (int i = 0; i < n; ++i)
            x[i] = q48o_fp_div(x[i], sum);
}

/* KV store (llama_int.c:1414-1416) + exact GQA attention
 * (llama_int.c:1433, 1502-1529).  Cache layout [L][max_seq][n_kv][hd]
 * (kv_key_at, llama_int.c:1185-1195). */
void q48o_attn_decode(int64_t *out, const int64_t *q, int64_t *kcache,
                      int64_t *vcache, const int64_t *k_new,
                      const int64_t *v_new, int layer, int pos, int n_heads,
                      int n_kv, int head_dim, int max_seq)
{
    int hd = head_dim, kvd = n_kv * hd, group = n_heads / n_kv;
    int64_t base = (int64_t)layer * max_seq;
    memcpy(kcache + (base + pos) * kvd, k_new, (size_t)kvd * 8);
    memcpy(vcache + (base + pos) * kvd, v_new, (size_t)kvd * 8);
    int64_t scale = q48o_fp_inv_sqrt(q48o_fp_from_int(hd));
    int S = pos + 1;
    int64_t *sc = (int64_t *)malloc((size_t)S * 8);
    for (int h = 0; h < n_heads; ++h) {
        int kh = h / group;
        const int64_t *qh = q + (int64_t)h * hd;
        for (int t = 0; t < S; ++t) {
            const int64_t *kt = kcache + (base + t) * kvd + (int64_t)kh * hd;
            u128 dot = 0;
            for (int d = 0; d < hd; ++d)
                dot += (u128)((i128)qh[d] * kt[d]);
            sc[t] = q48o_fp_mul((int64_t)((i128)dot >> 48), scale);
        }
        q48o_softmax(sc, S);
        int64_t *oh = out + (int64_t)h * hd;
        for (int d = 0; d < hd; ++d)
            oh[d] = 0;
        for (int t = 0; t < S; ++t) {
            const int64_t *vt = vcache + (base + t) * kvd + (int64_t)kh * hd;
            for (int d = 0; d < hd; ++d)
                oh[d] += q48o_fp_mul(sc[t], vt[d]);
        }
    }
    free(sc);
}

/* SwiGLU, llama_int.c:1549-1552: fp_mul(fp_silu(g), u). */
void q48o_silu_mul(int64_t *out, const int64_t *gate, const int64_t *up, int n)
{
    for (int i = 0; i < n; ++i)
        out[i] = q48o_fp_mul(q48o_fp_silu(gate[i]), up[i]);
}

/* argmax, llama_int.c:2888-2893: first index of the maximum. */
int q48o_argmax(const int64_t *v, int n)
{
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (v[i] > v[best])
            best = i;
    return best;
}

/* ======================================================================
 * Model (llama_model_t, llama_int.c:1575-1605) with synthetic weights
 * ==================================================================== */

typedef struct {
    int64_t *attn_norm, *wq, *wk, *wv, *wo, *ffn_norm, *wg, *wu, *wd;
} layer_w;

struct q48o_model {
    q48o_config c;
    int64_t *embed, *final_norm, *lm_head;
    layer_w *L;
    int64_t *rope_cos, *rope_sin;
    int64_t *kc, *vc;
    int64_t *buf;   /* scratch: hidden, normed, q, k, v, attn, o, gate, up, mlp, gu */
};

static int64_t *alloc_fill(const char *name, int64_t rows, int64_t cols,
                           uint64_t seed, int threads)
{
    int64_t *p = (int64_t *)malloc((size_t)(rows * cols) * 8);
    if (!p)
        return NULL;
    q48s_fill_named(p, rows, cols, seed, name, Q48_SIGMA_W, 1, threads);
    return p;
}

q48o_model *q48o_model_synth(const q48o_config *cfg, uint64_t seed, int threads)
{
    q48o_model *m = (q48o_model *)calloc(1, sizeof *m);
    if (!m)
        return NULL;
    m->c = *cfg;
    const q48o_config *c = &m->c;
    int dim = c->dim, kvd = c->n_kv_heads * c->head_dim, ffn = c->ffn;
    char nm[128];
    m->embed = alloc_fill("model.embed_tokens.weight", c->vocab, dim, seed, threads);
    m->final_norm = alloc_fill("model.norm.weight", 1, dim, seed, threads);
    m->lm_head = alloc_fill("lm_head.weight", c->vocab, dim, seed, threads);
    m->L = (layer_w *)calloc((size_t)c->n_layers, sizeof(layer_w));
    for (int l = 0; l < c->n_layers; ++l) {
        layer_w *w = &m->L[l];
#define LW(f, fmt, r, k) snprintf(nm, sizeof nm, fmt, l); w->f = alloc_fill(nm, r, k, seed, threads)
        LW(attn_norm, "model.layers.%d.input_layernorm.weight", 1, dim);
        LW(wq, "model.layers.%d.self_attn.q_proj.weight", dim, dim);
        LW(wk, "model.layers.%d.self_attn.k_proj.weight", kvd, dim);
        LW(wv, "model.layers.%d.self_attn.v_proj.weight", kvd, dim);
        LW(wo, "model.layers.%d.self_attn.o_proj.weight", dim, dim);
        LW(ffn_norm, "model.layers.%d.post_attention_layernorm.weight", 1, dim);
        LW(wg, "model.layers.%d.mlp.gate_proj.weight", ffn, dim);
        LW(wu, "model.layers.%d.mlp.up_proj.weight", ffn, dim);
        LW(wd, "model.layers.%d.mlp.down_proj.weight", dim, ffn);
#undef LW
    }
    int half = c->head_dim / 2;
    m->rope_cos = (int64_t *)malloc((size_t)c->max_seq * half * 8);
    m->rope_sin = (int64_t *)malloc((size_t)c->max_seq * half * 8);
    q48o_rope_tables(m->rope_cos, m->rope_sin, c->head_dim, c->max_seq, c->rope_theta);
    size_t kvn = (size_t)c->n_layers * c->max_seq * kvd;
    m->kc = (int64_t *)calloc(kvn, 8);
    m->vc = (int64_t *)calloc(kvn, 8);
    m->buf = (int64_t *)calloc((size_t)(8 * dim + 2 * kvd + 3 * ffn), 8);
    return m;
}

void q48o_model_free(q48o_model *m)
{
    if (!m)
        return;
    for (int l = 0; l < m->c.n_layers; ++l) {
        layer_w *w = &m->L[l];
        free(w->attn_norm); free(w->wq); free(w->wk); free(w->wv); free(w->wo);
        free(w->ffn_norm); free(w->wg); free(w->wu); free(w->wd);
    }
    free(m->L);
    free(m->embed); free(m->final_norm); free(m->lm_head);
    free(m->rope_cos); free(m->rope_sin);
    free(m->kc); free(m->vc); free(m->buf);
    free(m);
}

const int64_t *q48o_model_tensor(q48o_model *m, const char *name)
{
    if (!strcmp(name, "model.embed_tokens.weight")) return m->embed;
    if (!strcmp(name, "model.norm.weight")) return m->final_norm;
    if (!strcmp(name, "lm_head.weight")) return m->lm_head;
    if (!strcmp(name, "rope.cos")) return m->rope_cos;
    if (!strcmp(name, "rope.sin")) return m->rope_sin;
    int l;
    char rest[96];
    if (sscanf(name, "model.layers.%d.%95s", &l, rest) == 2 && l >= 0 &&
        l < m->c.n_layers) {
        layer_w *w = &m->L[l];
        if (!strcmp(rest, "input_layernorm.weight")) return w->attn_norm;
        if (!strcmp(rest, "self_attn.q_proj.weight")) return w->wq;
        if (!strcmp(rest, "self_attn.k_proj.weight")) return w->wk;
        if (!strcmp(rest, "self_attn.v_proj.weight")) return w->wv;
        if (!strcmp(rest, "self_attn.o_proj.weight")) return w->wo;
        if (!strcmp(rest, "post_attention_layernorm.weight")) return w->ffn_norm;
        if (!strcmp(rest, "mlp.gate_proj.weight")) return w->wg;
        if (!strcmp(rest, "mlp.up_proj.weight")) return w->wu;
        if (!strcmp(rest, "mlp.down_proj.weight")) return w->wd;
    }
    return NULL;
}

void q48o_kv_reset(q48o_model *m)
{
    size_t n = (size_t)m->c.n_layers * m->c.max_seq * m->c.n_kv_heads * m->c.head_dim;
    memset(m->kc, 0, n * 8);
    memset(m->vc, 0, n * 8);
}

int64_t *q48o_kv_keys(q48o_model *m) { return m->kc; }
int64_t *q48o_kv_values(q48o_model *m) { return m->vc; }

void q48o_kv_fill_synth(q48o_model *m, uint64_t seed, int npos, int threads)
{
    int kvd = m->c.n_kv_heads * m->c.head_dim;
    char nm[64];
    for (int l = 0; l < m->c.n_layers; ++l) {
        int64_t off = (int64_t)l * m->c.max_seq * kvd;
        snprintf(nm, sizeof nm, "kv.key.%d", l);
        q48s_fill_named(m->kc + off, npos, kvd, seed, nm, Q48_SIGMA_ACT, 1, threads);
        snprintf(nm, sizeof nm, "kv.value.%d", l);
        q48s_fill_named(m->vc + off, npos, kvd, seed, nm, Q48_SIGMA_ACT, 1, threads);
    }
}

/* transformer_layer_forward, llama_int.c:1326-1569 (exact-cache path). */
static void layer_forward(q48o_model *m, int l, int pos, int64_t *hidden)
{
    const q48o_config *c = &m->c;
    const layer_w *w = &m->L[l];
    int dim = c->dim, hd = c->head_dim, kvd = c->n_kv_heads * hd, ffn = c->ffn;
    int64_t *p = m->buf + dim;
    int64_t *normed = p; p += dim;
    int64_t *q = p; p += dim;
    int64_t *k = p; p += kvd;
    int64_t *v = p; p += kvd;
    int64_t *attn = p; p += dim;
    int64_t *o = p; p += dim;
    int64_t *gate = p; p += ffn;
    int64_t *up = p; p += ffn;
    int64_t *mlp = p; p += dim;
    int64_t *gu = p;

    q48o_rmsnorm(normed, hidden, w->attn_norm, dim);
    q48o_gemv(q, w->wq, normed, dim, dim);
    q48o_gemv(k, w->wk, normed, kvd, dim);
    q48o_gemv(v, w->wv, normed, kvd, dim);
    for (int h = 0; h < c->n_heads; ++h)
        q48o_rope_apply(m->rope_cos, m->rope_sin, hd / 2, q + h * hd, pos);
    for (int h = 0; h < c->n_kv_heads; ++h)
        q48o_rope_apply(m->rope_cos, m->rope_sin, hd / 2, k + h * hd, pos);
    q48o_attn_decode(attn, q, m->kc, m->vc, k, v, l, pos, c->n_heads,
                     c->n_kv_heads, hd, c->max_seq);
    q48o_gemv(o, w->wo, attn, dim, dim);
    for (int i = 0; i < dim; ++i)
        hidden[i] += o[i];
    q48o_rmsnorm(normed, hidden, w->ffn_norm, dim);
    q48o_gemv(gate, w->wg, normed, ffn, dim);
    q48o_gemv(up, w->wu, normed, ffn, dim);
    q48o_silu_mul(gu, gate, up, ffn);
    q48o_gemv(mlp, w->wd, gu, dim, ffn);
    for (int i = 0; i < dim; ++i)
        hidden[i] += mlp[i];
}

void q48o_layer_forward(q48o_model *m, int layer, int pos, int64_t *hidden)
{
    layer_forward(m, layer, pos, hidden);
}

/* llama_forward, llama_int.c:2807-2886. */
int q48o_forward(q48o_model *m, int token, int pos, int64_t *logits)
{
    const q48o_config *c = &m->c;
    if (token < 0 || token >= c->vocab || pos < 0 || pos >= c->max_seq)
        return -1;
    int dim = c->dim;
    int64_t *hidden = m->buf;
    memcpy(hidden, m->embed + (int64_t)token * dim, (size_t)dim * 8);
    for (int l = 0; l < c->n_layers; ++l)
        layer_forward(m, l, pos, hidden);
    int64_t *normed = m->buf + dim;
    q48o_rmsnorm(normed, hidden, m->final_norm, dim);
    q48o_gemv(logits, m->lm_head, normed, c->vocab, dim);
    return 0;
}

#define LLAMA_EOS 2

/* generate, llama_int.c:3067-3135 with sp == NULL (greedy argmax). */
int q48o_generate(q48o_model *m, const int *prompt, int prompt_len,
                  int max_new, int *out_tokens, uint64_t *step_hash,
                  int *n_steps)
{
    int vocab = m->c.vocab, steps = 0;
    int64_t *logits = (int64_t *)malloc((size_t)vocab * 8);
    q48o_kv_reset(m);
    memcpy(out_tokens, prompt, (size_t)prompt_len * sizeof(int));
    int total = prompt_len;
    for (int pos = 0; pos < prompt_len; ++pos) {
        if (q48o_forward(m, out_tokens[pos], pos, logits) != 0) {
            free(logits);
            return -1;
        }
        if (step_hash)
            step_hash[steps] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        if (pos == prompt_len - 1)
            out_tokens[total++] = q48o_argmax(logits, vocab);
    }
    for (int i = 1; i < max_new; ++i) {
        int pos = prompt_len + i - 1;
        if (q48o_forward(m, out_tokens[pos], pos, logits) != 0)
            break;
        if (step_hash)
            step_hash[steps] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        int next = q48o_argmax(logits, vocab);
        if (next == LLAMA_EOS)
            break;
        out_tokens[total++] = next;
    }
    free(logits);
    if (n_steps)
        *n_steps = steps;
    return total;
}

int q48o_decode_from(q48o_model *m, int token, int start_pos, int n,
                     int *out_tokens, uint64_t *step_hash)
{
    int vocab = m->c.vocab, steps = 0;
    int64_t *logits = (int64_t *)malloc((size_t)vocab * 8);
    int tok = token;
    for (int i = 0; i < n; ++i) {
        if (q48o_forward(m, tok, start_pos + i, logits) != 0)
            break;
        if (step_hash)
            step_hash[i] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        tok = q48o_argmax(logits, vocab);
        if (out_tokens)
            out_tokens[i] = tok;
        if (tok == LLAMA_EOS)
            break;
    }
    free(logits);
    return steps;
}

/* ======================================================================
 * Sampling (llama_int.c:2895-3039)
 * ==================================================================== */

static uint64_t splitmix_step(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* rng_seed, llama_int.c:2909-2920 */
void q48o_rng_seed(uint64_t seed, uint64_t s[2])
{
    s[0] = splitmix_step(seed);
    s[1] = splitmix_step(seed + 0x9E3779B97F4A7C15ULL);
    if (s[0] == 0 && s[1] == 0)
        s[0] = 1;
}

static uint64_t rotl64(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }

/* rng_next, llama_int.c:2922-2929 (xoroshiro128+) */
uint64_t q48o_rng_next(uint64_t s[2])
{
    const uint64_t a = s[0];
    uint64_t b = s[1];
    const uint64_t out = a + b;
    b ^= a;
    s[0] = rotl64(a, 55) ^ b ^ (b << 14);
    s[1] = rotl64(b, 36);
    return out;
}

static int cmp_desc_i64(const void *pa, const void *pb)
{
    const int64_t a = *(const int64_t *)pa, b = *(const int64_t *)pb;
    return (a < b) - (a > b);
}

typedef struct {
    int64_t p;
    int i;
} prob_idx;

/* descending probability, ascending index among equal ones: the order in
 * which the reference's repeated first-maximum search (llama_int.c:2998-
 * 3007) takes the entries */
static int cmp_prob_idx(const void *pa, const void *pb)
{
    const prob_idx *a = (const prob_idx *)pa, *b = (const prob_idx *)pb;
    if (a->p != b->p)
        return a->p > b->p ? -1 : 1;
    return (a->i > b->i) - (a->i < b->i);
}

/* sample_token, llama_int.c:2958-3039 */
int q48o_sample(const int64_t *logits, int n, int64_t temperature, int top_k,
                int64_t top_p, uint64_t s[2])
{
    /* 2963-2964: greedy below a temperature of 0.01 */
    if (temperature <= 0 || temperature < Q48_ONE / 100)
        return q48o_argmax(logits, n);
    int64_t *w = (int64_t *)malloc((size_t)n * 8);
    /* 2970-2971: logits / T */
    for (int i = 0; i < n; ++i)
        w[i] = q48o_fp_div(logits[i], temperature);
    /* 2974-2987: the k-th largest value (duplicates counted) is the
     * threshold; smaller values become INT64_MIN / 2 */
    if (top_k > 0 && top_k < n) {
        int64_t *srt = (int64_t *)malloc((size_t)n * 8);
        memcpy(srt, w, (size_t)n * 8);
        qsort(srt, (size_t)n, 8, cmp_desc_i64);
        const int64_t thr = srt[top_k - 1];
        free(srt);
        for (int i = 0; i < n; ++i)
            if (w[i] < thr)
                w[i] = INT64_MIN / 2;
    }
    /* 2990: softmax in place */
    q48o_softmax(w, n);
    /* 2993-3023: nucleus.  The reference takes, while the running sum is
     * below top_p, the largest remaining positive probability (first index
     * among equals); the same entries in the same order are the prefix of
     * the positive probabilities sorted by (value desc, index asc).  Kept
     * entries are renormalised by their (wrapping) sum, the rest zeroed. */
    if (top_p > 0 && top_p < Q48_ONE) {
        prob_idx *o = (prob_idx *)malloc((size_t)n * sizeof(prob_idx));
        int np = 0;
        for (int i = 0; i < n; ++i)
            if (w[i] > 0) {
                o[np].p = w[i];
                o[np].i = i;
                np++;
            }
        qsort(o, (size_t)np, sizeof(prob_idx), cmp_prob_idx);
        uint8_t *keep = (uint8_t *)calloc((size_t)n, 1);
        int64_t cum = 0;
        for (int k = 0; k < np && cum < top_p; ++k) {
            cum = (int64_t)((uint64_t)cum + (uint64_t)o[k].p);
            keep[o[k].i] = 1;
        }
        free(o);
        int64_t sum = 0;
        for (int i = 0; i < n; ++i) {
            if (!keep[i])
                w[i] = 0;
            sum = (int64_t)((uint64_t)sum + (uint64_t)w[i]);
        }
        free(keep);
        if (sum > 0)
            for (int i = 0; i < n; ++i)
                if (w[i] > 0)
                    w[i] = q48o_fp_div(w[i], sum);
    }
    /* 3027-3036: r in [0, ONE) from the top 48 bits of one draw; the first
     * index whose running (wrapping) sum exceeds r, else the argmax */
    const int64_t r = (int64_t)(q48o_rng_next(s) >> 16);
    int64_t cum = 0;
    int sel = -1;
    for (int i = 0; i < n; ++i) {
        cum = (int64_t)((uint64_t)cum + (uint64_t)w[i]);
        if (cum > r) {
            sel = i;
            break;
        }
    }
    if (sel < 0)
        sel = q48o_argmax(w, n);
    free(w);
    return sel;
}

/* generate, llama_int.c:3067-3135 with sampling parameters */
int q48o_generate_sampled(q48o_model *m, const int *prompt, int prompt_len,
                          int max_new, int *out_tokens, uint64_t *step_hash,
                          int *n_steps, int64_t temperature, int top_k,
                          int64_t top_p, uint64_t seed)
{
    uint64_t s[2];
    q48o_rng_seed(seed, s);
    int vocab = m->c.vocab, steps = 0;
    int64_t *logits = (int64_t *)malloc((size_t)vocab * 8);
    q48o_kv_reset(m);
    memcpy(out_tokens, prompt, (size_t)prompt_len * sizeof(int));
    int total = prompt_len;
    for (int pos = 0; pos < prompt_len; ++pos) {
        if (q48o_forward(m, out_tokens[pos], pos, logits) != 0) {
            free(logits);
            return -1;
        }
        if (step_hash)
            step_hash[steps] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        if (pos == prompt_len - 1)
            out_tokens[total++] = q48o_sample(logits, vocab, temperature, top_k, top_p, s);
    }
    for (int i = 1; i < max_new; ++i) {
        int pos = prompt_len + i - 1;
        if (q48o_forward(m, out_tokens[pos], pos, logits) != 0)
            break;
        if (step_hash)
            step_hash[steps] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        int next = q48o_sample(logits, vocab, temperature, top_k, top_p, s);
        if (next == LLAMA_EOS)
            break;
        out_tokens[total++] = next;
    }
    free(logits);
    if (n_steps)
        *n_steps = steps;
    return total;
}
