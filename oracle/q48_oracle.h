/*
 * q48_oracle.h — CPU oracle for the Q16.48 forward pass.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the
 * reference's integer algorithms (fp_math.h and the exact path of
 * llama_int.c) used as the checker for the HIP library.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product (libintllm_hip + the C host) never links it.
 *
 * Every function cites the reference file:line it restates.  Parity
 * pins (what proves this restatement equals the reference) live in
 * tests/test_oracle_*.py: the determinism golden hash and sub-hashes,
 * the compiled reference harness (oracle/_ref), and closed forms.
 */
#ifndef Q48_ORACLE_H
#define Q48_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp_math.h primitives --------------------------------------------- */
int64_t q48o_fp_mul(int64_t a, int64_t b);
int64_t q48o_fp_div(int64_t a, int64_t b);
int64_t q48o_fp_from_int(int x);
int64_t q48o_fp_sqrt(int64_t x);
int64_t q48o_fp_sqrt_fast(int64_t x);
int64_t q48o_fp_inv_sqrt(int64_t x);
int64_t q48o_fp_exp_dyadic(int64_t x, int k);
int64_t q48o_fp_exp(int64_t x);
int64_t q48o_fp_safe_exp(int64_t x);
int64_t q48o_fp_log(int64_t x);
void    q48o_fp_sincos(int64_t angle, int64_t *c, int64_t *s);
int64_t q48o_fp_sigmoid(int64_t x);
int64_t q48o_fp_silu(int64_t x);
/* FP_PI, fp_cordic_gain and the 48 CORDIC angles after fp_math_init. */
void    q48o_fp_consts(int64_t *pi, int64_t *gain, int64_t *angles48);

/* Determinism gate (fp_determinism.c:162-244): fills subs[12] and
 * returns the combined hash. */
uint64_t q48o_determinism(uint64_t subs[12]);
/* The gate's 4230-value input grid (fp_determinism.c:101-137). */
int      q48o_det_grid(int64_t *out, int cap);

/* ---- llama_int.c tensor ops -------------------------------------------- */
void q48o_gemv(int64_t *y, const int64_t *W, const int64_t *x, int M, int K);
void q48o_gemm(int64_t *Y, const int64_t *W, const int64_t *X,
               int T, int N, int K);
void q48o_rmsnorm(int64_t *out, const int64_t *x, const int64_t *w, int dim);
void q48o_rope_tables(int64_t *cos_t, int64_t *sin_t, int head_dim,
                      int max_seq, int theta);
void q48o_rope_apply(const int64_t *cos_t, const int64_t *sin_t, int half,
                     int64_t *vec, int pos);
void q48o_softmax(int64_t *x, int n);
void q48o_attn_decode(int64_t *out, const int64_t *q, int64_t *kcache,
                      int64_t *vcache, const int64_t *k_new,
                      const int64_t *v_new, int layer, int pos, int n_heads,
                      int n_kv, int head_dim, int max_seq);
void q48o_silu_mul(int64_t *out, const int64_t *gate, const int64_t *up, int n);
int  q48o_argmax(const int64_t *v, int n);

/* ---- model forward / generate ------------------------------------------ */
typedef struct {
    int dim, n_heads, n_kv_heads, head_dim, n_layers, ffn, vocab, max_seq,
        rope_theta;
} q48o_config;

typedef struct q48o_model q48o_model;

/* Synthetic random-init model (q48_synth.h) of shape cfg. */
q48o_model *q48o_model_synth(const q48o_config *cfg, uint64_t seed,
                             int threads);
void        q48o_model_free(q48o_model *m);
/* Pointer to a weight tensor by HF name (NULL if absent); for tests. */
const int64_t *q48o_model_tensor(q48o_model *m, const char *name);
/* Zero the KV cache (kv_cache_reset, llama_int.c:1170-1183). */
void q48o_kv_reset(q48o_model *m);
/* Fill KV positions [0, npos) of every layer with N(0,1) bf16 samples. */
void q48o_kv_fill_synth(q48o_model *m, uint64_t seed, int npos, int threads);
/* KV cache base pointers ([L][max_seq][n_kv][hd]). */
int64_t *q48o_kv_keys(q48o_model *m);
int64_t *q48o_kv_values(q48o_model *m);
/* transformer_layer_forward (llama_int.c:1326-1569) on hidden in place. */
void q48o_layer_forward(q48o_model *m, int layer, int pos, int64_t *hidden);
/* llama_forward (llama_int.c:2807-2886): 0 and logits[vocab], or -1. */
int q48o_forward(q48o_model *m, int token, int pos, int64_t *logits);
/* generate (llama_int.c:3067-3135), greedy.  step_hash[i] is the FNV-1a-64
 * of the logits of forward call i (prompt positions included).  Returns
 * the total token count (prompt + generated) or -1. */
int q48o_generate(q48o_model *m, const int *prompt, int prompt_len,
                  int max_new, int *out_tokens, uint64_t *step_hash,
                  int *n_steps);
/* Decode loop from a pre-filled cache (config 5): token at pos start,
 * then greedy for n steps (stops at EOS like generate).  Returns the
 * number of steps run. */
int q48o_decode_from(q48o_model *m, int token, int start_pos, int n,
                     int *out_tokens, uint64_t *step_hash);

/* ---- sampling (llama_int.c:2895-3039) ----------------------------------- */
/* rng_seed (llama_int.c:2909-2920): SplitMix64 of seed and of
 * seed + 0x9E3779B97F4A7C15 into the two state words; (0, 0) -> (1, 0). */
void     q48o_rng_seed(uint64_t seed, uint64_t s[2]);
/* rng_next (llama_int.c:2922-2929): xoroshiro128+ (55/14/36). */
uint64_t q48o_rng_next(uint64_t s[2]);
/* sample_token (llama_int.c:2958-3039): argmax when temperature < ONE/100
 * (or <= 0); otherwise temperature, top-k mask, softmax, top-p nucleus and
 * one draw of rng_next.  s is advanced in place when a draw is made. */
int q48o_sample(const int64_t *logits, int n, int64_t temperature, int top_k,
                int64_t top_p, uint64_t s[2]);
/* generate (llama_int.c:3067-3135) with sampling parameters sp (rng seeded
 * by rng_seed(seed)); step_hash as in q48o_generate. */
int q48o_generate_sampled(q48o_model *m, const int *prompt, int prompt_len,
                          int max_new, int *out_tokens, uint64_t *step_hash,
                          int *n_steps, int64_t temperature, int top_k,
                          int64_t top_p, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
