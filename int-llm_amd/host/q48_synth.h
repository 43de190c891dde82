/*
 * q48_synth.h — deterministic, libm-free synthetic inputs for the Q16.48 path.
 *
 * Every configuration this library is measured on uses random-init weights
 * and activations of TinyLlama shapes (no checkpoint is available offline).
 * This header fixes exactly how those int64 values are produced, so the GPU
 * run, the CPU baseline and the golden-vector harness see the same bits:
 *
 *   stream   one xorshift64 stream per (tensor, row): state =
 *            splitmix64(tensor_seed + row * 0x9E3779B97F4A7C15), forced
 *            nonzero; xorshift64 step as fp_math.h:929-934 (13, 7, 17).
 *   sample   CLT-12 Gaussian as fp_math.h:944-952: z = sum of 12 draws
 *            (next() >> 16) - 6*ONE, value = fp_mul(sigma, z) (mean 0).
 *   rounding the Q16.48 sample is rounded to bfloat16 (round to nearest,
 *            ties to even, on the exact integer value) and converted back
 *            with the exact bf16 -> Q16.48 rule of safetensors.h:115-152,
 *            so every weight is exactly an HF-style bf16 weight.
 *   seeds    tensor_seed = FNV-1a-64(tensor name) XOR base_seed.
 *
 * sigma is Q16.48: Q48_SIGMA_W = ONE/50 (0.02) for weights, ONE for
 * activations and KV-cache contents.
 */
#ifndef Q48_SYNTH_H
#define Q48_SYNTH_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q48_ONE        ((int64_t)1 << 48)
#define Q48_SIGMA_W    (Q48_ONE / 50)
#define Q48_SIGMA_ACT  (Q48_ONE)

/* FNV-1a-64 of a NUL-terminated string (seed derivation). */
uint64_t q48s_fnv1a_str(const char *s);

/* FNV-1a-64 over raw little-endian int64 bytes, continuing from h
 * (h = 1469598103934665603 to start). Same mixing as fp_determinism.c:48-56. */
uint64_t q48s_fnv_i64(uint64_t h, const int64_t *v, size_t n);

/* Seed of the tensor called `name` under `base_seed`. */
uint64_t q48s_tensor_seed(uint64_t base_seed, const char *name);

/* bf16 bits -> exact Q16.48 (restates safetensors.h:115-152). */
int64_t q48s_bf16_to_q48(uint16_t bits);

/* IEEE half bits -> exact Q16.48 (restates safetensors.h:74-111). */
int64_t q48s_f16_to_q48(uint16_t bits);

/* Q16.48 -> bf16 bits, round to nearest, ties to even. */
uint16_t q48s_q48_to_bf16(int64_t v);

/* One Gaussian sample from the stream *state (fp_gaussian, mean 0). */
int64_t q48s_gaussian(uint64_t *state, int64_t sigma);

/* Initial stream state of row `row` of a tensor seeded `seed`. */
uint64_t q48s_row_state(uint64_t seed, uint64_t row);

/* Fill dst[rows][cols] (row-major) with the tensor `seed`.  bf16_round
 * selects the bf16 rounding step.  n_threads <= 1 runs inline; rows are
 * independent streams, so the bits do not depend on the thread count. */
void q48s_fill(int64_t *dst, int64_t rows, int64_t cols, uint64_t seed,
               int64_t sigma, int bf16_round, int n_threads);

/* Convenience: q48s_fill with the seed of `name`. */
void q48s_fill_named(int64_t *dst, int64_t rows, int64_t cols,
                     uint64_t base_seed, const char *name,
                     int64_t sigma, int bf16_round, int n_threads);

/* Uniform token ids in [lo, hi) from a seeded stream (prompt synthesis). */
void q48s_tokens(int *dst, int n, uint64_t seed, int lo, int hi);

#ifdef __cplusplus
}
#endif
#endif
