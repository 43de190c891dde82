/*
 * q48_synth.c — synthetic Q16.48 inputs (definition in q48_synth.h).
 *
 * Pure integer code: the same bits on every host, in any thread count.
 */
#include "q48_synth.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define FNV_OFF   1469598103934665603ULL
#define FNV_PRIME 1099511628211ULL

uint64_t q48s_fnv1a_str(const char *s)
{
    uint64_t h = FNV_OFF;
    for (; *s; ++s) {
        h ^= (uint8_t)*s;
        h *= FNV_PRIME;
    }
    return h;
}

uint64_t q48s_fnv_i64(uint64_t h, const int64_t *v, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        uint64_t u = (uint64_t)v[i];
        for (int b = 0; b < 8; ++b) {
            h ^= u & 0xff;
            h *= FNV_PRIME;
            u >>= 8;
        }
    }
    return h;
}

uint64_t q48s_tensor_seed(uint64_t base_seed, const char *name)
{
    return q48s_fnv1a_str(name) ^ base_seed;
}

/* Exact bf16 -> Q16.48: value (128 + m) * 2^(e - 134), scaled by 2^48.
 * e = 0 (zero / subnormal) -> 0; e = 255 (inf / nan) -> +-32000.
 * Follows safetensors.h:115-152, sign applied last. */
int64_t q48s_bf16_to_q48(uint16_t bits)
{
    int sign = bits >> 15;
    int e = (bits >> 7) & 0xff;
    int m = bits & 0x7f;
    int64_t r;
    if (e == 0)
        return 0;
    if (e == 0xff) {
        r = (int64_t)32000 << 48;
        return sign ? -r : r;
    }
    int sh = e - 86;
    int64_t sig = 128 + m;
    if (sh >= 0 && sh < 64)
        r = (int64_t)((uint64_t)sig << sh);
    else if (sh < 0 && sh > -64)
        r = sig >> (-sh);
    else
        r = 0;
    return sign ? -r : r;
}

/* Exact IEEE half -> Q16.48: normal values (1024 + m) * 2^(e - 25), subnormal
 * m * 2^-24, scaled by 2^48 (shifts of e + 23 and 24); +-0 -> 0; e = 31 (inf /
 * nan) -> +-32000.  Follows safetensors.h:74-111, sign applied last; the left
 * shift and the negation wrap (e = 30 reaches bit 63). */
int64_t q48s_f16_to_q48(uint16_t bits)
{
    int sign = bits >> 15;
    int e = (bits >> 10) & 0x1f;
    int m = bits & 0x3ff;
    uint64_t r;
    if (e == 0 && m == 0)
        return 0;
    if (e == 0x1f)
        r = (uint64_t)32000 << 48;
    else if (e == 0)
        r = (uint64_t)m << 24;
    else
        r = (uint64_t)(1024 + m) << (e + 23);
    return (int64_t)(sign ? (uint64_t)0 - r : r);
}

uint16_t q48s_q48_to_bf16(int64_t v)
{
    if (v == 0)
        return 0;
    uint16_t sign = v < 0 ? 0x8000 : 0;
    uint64_t mag = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
    int p = 63 - __builtin_clzll(mag);
    int sh = p - 7;            /* keep 8 significant bits */
    if (sh <= 0) {
        /* at most 8 significant bits: exact.  q = mag << (7 - p) is in
         * [128, 256) and value = q * 2^(p - 7 - 48), so E = p + 79. */
        return (uint16_t)(sign | (uint16_t)((p + 79) << 7) |
                          (uint16_t)((mag << (7 - p)) & 0x7f));
    }
    uint64_t q = mag >> sh;
    uint64_t rem = mag & (((uint64_t)1 << sh) - 1);
    uint64_t half = (uint64_t)1 << (sh - 1);
    if (rem > half || (rem == half && (q & 1)))
        q += 1;
    if (q == 256) {
        q = 128;
        sh += 1;
    }
    /* value = q * 2^sh * 2^-48 = (128 + m) * 2^(E - 134)  =>  E = sh + 86 */
    return (uint16_t)(sign | (uint16_t)((sh + 86) << 7) | (uint16_t)(q - 128));
}

static inline uint64_t xorshift64(uint64_t *s)
{
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}

static inline uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t q48s_row_state(uint64_t seed, uint64_t row)
{
    uint64_t s = splitmix64(seed + row * 0x9E3779B97F4A7C15ULL);
    return s ? s : 0x2545F4914F6CDD1DULL;
}

int64_t q48s_gaussian(uint64_t *state, int64_t sigma)
{
    int64_t sum = 0;
    for (int i = 0; i < 12; ++i)
        sum += (int64_t)(xorshift64(state) >> 16);
    int64_t z = sum - 6 * Q48_ONE;
    return (int64_t)(((__int128)sigma * z) >> 48);
}

typedef struct {
    int64_t *dst;
    int64_t rows, cols, r0, r1;
    uint64_t seed;
    int64_t sigma;
    int bf16_round;
} fill_job;

static void fill_rows(const fill_job *j)
{
    for (int64_t r = j->r0; r < j->r1; ++r) {
        uint64_t st = q48s_row_state(j->seed, (uint64_t)r);
        int64_t *row = j->dst + r * j->cols;
        for (int64_t c = 0; c < j->cols; ++c) {
            int64_t v = q48s_gaussian(&st, j->sigma);
            row[c] = j->bf16_round ? q48s_bf16_to_q48(q48s_q48_to_bf16(v)) : v;
        }
    }
}

static void *fill_thread(void *arg)
{
    fill_rows((const fill_job *)arg);
    return NULL;
}

void q48s_fill(int64_t *dst, int64_t rows, int64_t cols, uint64_t seed,
               int64_t sigma, int bf16_round, int n_threads)
{
    if (n_threads > 64)
        n_threads = 64;
    if (n_threads <= 1 || rows < 2 * n_threads) {
        fill_job j = {dst, rows, cols, 0, rows, seed, sigma, bf16_round};
        fill_rows(&j);
        return;
    }
    pthread_t th[64];
    fill_job jobs[64];
    int ok[64];
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (fill_job){dst, rows, cols, rows * t / n_threads,
                             rows * (t + 1) / n_threads, seed, sigma, bf16_round};
        ok[t] = pthread_create(&th[t], NULL, fill_thread, &jobs[t]) == 0;
        if (!ok[t])
            fill_rows(&jobs[t]);   /* no thread available: run inline */
    }
    for (int t = 0; t < n_threads; ++t)
        if (ok[t])
            pthread_join(th[t], NULL);
}

void q48s_fill_named(int64_t *dst, int64_t rows, int64_t cols,
                     uint64_t base_seed, const char *name,
                     int64_t sigma, int bf16_round, int n_threads)
{
    q48s_fill(dst, rows, cols, q48s_tensor_seed(base_seed, name), sigma,
              bf16_round, n_threads);
}

void q48s_tokens(int *dst, int n, uint64_t seed, int lo, int hi)
{
    uint64_t st = q48s_row_state(seed, 0);
    uint64_t span = (uint64_t)(hi - lo);
    for (int i = 0; i < n; ++i)
        dst[i] = lo + (int)(xorshift64(&st) % span);
}
