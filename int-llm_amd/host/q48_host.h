/*
 * q48_host.h — the C host of the Q16.48 Llama forward pass.
 *
 * Keeps llama_int.c's host-side behaviour (config.json parsing, .mgw
 * loading, llama_forward and the greedy generate loop) and runs every
 * tensor op through libintllm_hip (include/intllm_hip.h) on device-resident
 * int64 weights and an int64 KV cache.  Token ids in, token ids (and,
 * on request, the logits) out: the host <-> device boundary is crossed
 * once per token.
 */
#ifndef Q48_HOST_H
#define Q48_HOST_H

#include <stdint.h>
#include "../../include/intllm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* llama_config_t (llama_int.c:788-798). */
typedef struct {
    int dim;          /* hidden_size               */
    int n_heads;      /* num_attention_heads       */
    int n_kv_heads;   /* num_key_value_heads (GQA) */
    int head_dim;     /* dim / n_heads (derived)   */
    int n_layers;     /* num_hidden_layers         */
    int ffn;          /* intermediate_size         */
    int vocab;        /* vocab_size                */
    int max_seq;      /* max_position_embeddings   */
    int rope_theta;   /* rope_theta                */
} q48h_config;

/* Timing counters, named like llama_int's KPI lines (llama_int.c:248-297). */
typedef struct {
    double prefill_s, decode_s;
    int prefill_tokens, decode_tokens;
} q48h_stats;

/* load_config_json (llama_int.c:834-903): same keys, defaults
 * (num_key_value_heads = num_attention_heads, max_position_embeddings =
 * 2048, rope_theta = 10000) and checks.  0, -1 (no file) or -2 (invalid). */
int q48h_config_from_json(const char *model_dir, q48h_config *cfg);
/* The same integer extraction on a JSON text already in memory. */
int q48h_config_from_json_text(const char *json, q48h_config *cfg);

/* Shapes the device path supports (head_dim even, <= 256, divides 256). */
int q48h_config_check(const q48h_config *cfg);

typedef struct q48h_model q48h_model;

/* Allocate device weights, KV cache and activations for cfg and build the
 * RoPE tables; weights are zero until uploaded. */
int q48h_model_create(q48h_model **out, q48_ctx *ctx, const q48h_config *cfg);
void q48h_model_free(q48h_model *m);
const q48h_config *q48h_model_config(const q48h_model *m);
q48_ctx *q48h_model_ctx(q48h_model *m);

/* Upload one tensor by its HF name (the names of load_layer_weights,
 * llama_int.c:1290-1298, and llama_load_global_weights, :1640-1677);
 * n must equal the tensor's element count. */
int q48h_upload(q48h_model *m, const char *name, const int64_t *host, int64_t n);

/* Fill every weight with the synthetic random-init values of q48_synth.h
 * (sigma 0.02, bf16-rounded), generated on the host with `threads`
 * threads and uploaded tensor by tensor. */
int q48h_model_synth(q48h_model *m, uint64_t seed, int threads);

/* mgw_load (llama_int.c:2344-2560): validate and upload a native .mgw
 * file.  max_seq > 0 overrides the file's max_seq_len.  Also checks each
 * tensor's element count against the config (the device must never read
 * past a tensor). */
int q48h_model_load_mgw(q48h_model **out, q48_ctx *ctx, const char *path, int max_seq);

/* mgw_export layout (llama_int.c:1718-1904) for the synthetic model of
 * cfg (no GPU needed): 64 B header, 64 B config, 96 B index entries,
 * 8-aligned int64 data, host byte order. */
int q48h_mgw_write_synth(const char *path, const q48h_config *cfg, uint64_t seed,
                         int threads);

/* KV cache (device) pointers, layout [L][max_seq][n_kv][head_dim]. */
int64_t *q48h_kv_keys(q48h_model *m);
int64_t *q48h_kv_values(q48h_model *m);
/* kv_cache_reset (llama_int.c:1170-1183). */
int q48h_kv_reset(q48h_model *m);
/* Positions [0, npos) of every layer <- N(0,1) bf16 samples (q48_synth.h,
 * tensors "kv.key.<l>" / "kv.value.<l>"); long-context configuration. */
int q48h_kv_fill_synth(q48h_model *m, uint64_t seed, int npos, int threads);

/* llama_forward (llama_int.c:2807-2886).  logits (host, may be NULL)
 * receives logits[vocab]; next (may be NULL) the greedy token.
 * Q48_ERANGE for a token or position out of range, like the
 * reference's NULL return. */
int q48h_forward(q48h_model *m, int token, int pos, int64_t *logits, int *next);
/* The logits [vocab] of the last step run on the device (forward, prefill's
 * last row, or a decode step), copied to host memory (synchronises). */
int q48h_read_logits(q48h_model *m, int64_t *logits);

/* generate (llama_int.c:3067-3135), greedy.  step_hash (may be NULL) gets
 * FNV-1a-64 of every forward call's logits (prompt positions included);
 * n_steps the number of forward calls.  Returns the total token count or
 * a negative Q48_E* code. */
int q48h_generate(q48h_model *m, const int *prompt, int prompt_len, int max_new,
                  int *out_tokens, uint64_t *step_hash, int *n_steps,
                  q48h_stats *stats);

/* Batched prefill (no reference counterpart as a batch: llama_int's prefill
 * calls llama_forward per token, llama_int.c:3081-3092): the forward of
 * tokens[0..T) at positions p0 .. p0 + T - 1 as row ops and q48_gemm
 * projections, filling the KV cache exactly as T forward calls do.
 * logits_all (host, may be NULL) receives the T logits rows; next (may be
 * NULL) the token chosen from the last row (argmax or sample_token).  Past
 * position 4096, or for T < 3 (where forward calls are as fast), the tokens
 * go one forward call at a time. */
int q48h_prefill(q48h_model *m, const int *tokens, int T, int p0, int64_t *logits_all,
                 int *next);
/* q48h_generate's prompt through q48h_prefill (1, the default) or one
 * forward call per token (0); the bits are the same. */
void q48h_model_set_batched_prefill(q48h_model *m, int on);
/* The batched prefill multiplies through digit planes of each layer's
 * projection matrices, prepared once per set of weights (q48_gemm_prepare;
 * about 8 bytes per weight of device memory, made at the first batched
 * prefill and again after q48h_upload).  1 (the default) or 0:
 * split W in each call, and free the planes.  The bits are the same. */
void q48h_model_set_gemm_planes(q48h_model *m, int on);

/* Greedy decode from an already filled cache: forward(token, start_pos),
 * then n - 1 more steps, stopping after the step that chose EOS
 * (long-context configuration); out_tokens[i] is the token chosen by step
 * i, and the return value counts the steps run (q48h_decode_graph's
 * conventions). */
int q48h_decode_from(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                     uint64_t *step_hash, q48h_stats *stats);

/* Choose how a layer maps onto library ops (same bits in every mode):
 * 0 one op per reference step; 1 fused (5 launches per layer), every GEMV
 * that starts with a norm recomputes its statistics; 2 fused, the
 * statistics computed once by the kernel that produced the vector (its last
 * block); 3 (default) fused, the producer leaves per-block partial sums and
 * each block of the consuming GEMV finishes them. */
void q48h_model_set_fused(q48h_model *m, int fused);

/* In the fused modes with bfloat16-resident weights, have each layer's
 * attention launch also read that layer's W_o on the idle compute units
 * (q48_attn_decode_rope_prefetch), so the O projection finds it in the
 * device-side cache.  On by default; int64 weights are never warmed (the
 * GEMVs read them with non-temporal loads).  The bits do not depend on it. */
void q48h_model_set_prefetch(q48h_model *m, int on);

/* In mode 3 below the split position (q48_attn_split_min), run RoPE and the
 * KV store in the q|k|v projection's epilogue and attention from the cache
 * (q48_norm_gemv_rope_kv, q48_attn_decode_cached) instead of RoPE and the
 * store inside attention (q48_attn_decode_rope).  On by default where the
 * shapes allow it (head_dim 32, 64 or 128, max_seq <= 4096); the bits do not
 * depend on it. */
void q48h_model_set_rope_gemv(q48h_model *m, int on);

/* Mode 3 with the projection matrices and lm_head read as bfloat16 bits
 * (the reference's .mgwc representation, llama_int.c:1906-1929): on packs a
 * device copy of them (2 bytes per weight, kept until the weights change)
 * and uses it; the results are bit-identical to the int64 weights.
 * Returns Q48_EINVAL, and changes nothing, when a weight is not exactly a
 * bfloat16 value or dim or ffn is not a multiple of 512. */
int q48h_model_set_bf16(q48h_model *m, int on);

/* Token selection by sample_token (llama_int.c:2958-3039) instead of argmax
 * for q48h_forward's next, q48h_generate, q48h_decode_from and
 * q48h_decode_graph: temperature and top_p in Q16.48 (top_p >= ONE: off),
 * top_k (0: off), the rng seeded by rng_seed(seed) (llama_int.c:2909-2920)
 * and advanced by each draw.  A temperature below ONE / 100 is greedy (the
 * default). */
int q48h_model_set_sampling(q48h_model *m, int64_t temperature, int top_k, int64_t top_p,
                            uint64_t seed);

/* Decode of n steps replayed from a captured graph: step i runs
 * forward(token_i, start_pos + i) and its argmax (or, with sampling set,
 * its sample_token draw) becomes token_{i+1} on the device, with no host
 * round trip between steps.  out_tokens[i] receives the token CHOSEN by
 * step i, so an EOS choice appears as the last counted entry (generate's
 * token list, q48h_generate, leaves it out: llama_int.c:3111).  The device
 * replays all n steps; the return value, and stats->decode_tokens, count
 * the steps up to and including the first EOS choice (generate stops
 * there), or every step.  n is clipped at max_seq (llama_forward's NULL,
 * llama_int.c:2817-2820, ends generate's loop, :3106).
 * q48h_decode_from has the same conventions with one forward call per step. */
int q48h_decode_graph(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                      q48h_stats *stats);

/* q48h_decode_graph that also records every replayed step's logits on the
 * device (q48_record_step inside the captured step) and writes their
 * FNV-1a-64 to step_hash[i] for every replayed step i (all n after the
 * max_seq clip, EOS or not): the per-step logits hash of the path that the
 * decode benchmark times. */
int q48h_decode_graph_hashed(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                             uint64_t *step_hash, q48h_stats *stats);

/* Measurement helper: enqueue `reps` times the GEMV launches of one decode
 * token (the four fused projections of every layer and the lm_head, in
 * decode order, on the model's weights and activation buffers) and report
 * their number and algorithmic bytes 8 (M K + K + outputs).  Overwrites the
 * activations; run it after decoding. */
int q48h_gemv_sweep(q48h_model *m, int reps, int *launches, double *bytes);

#ifdef __cplusplus
}
#endif
#endif
