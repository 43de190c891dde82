/*
 * intllm_hip.h — C ABI of libintllm_hip: the Q16.48 (int64 fixed-point)
 * Llama forward pass of nmicic/int-llm's llama_int, on one AMD MI355X.
 *
 * The reference has no FFI for this path: its hot path is `static` C
 * functions in llama_int.c.  Each entry point below replaces one of them
 * (cited as reference file:line) with the same argument meaning and the
 * same bits: every output equals the reference's CPU result exactly.
 *
 * Conventions
 *   - Every int64_t* / int* argument of an op is a DEVICE pointer owned
 *     by the caller (allocate with q48_malloc or any HIP allocator).
 *   - Values are Q16.48 fixed point (`fixed_t`, fp_math.h:175).
 *   - Ops are enqueued on the context's stream, in call order; q48_sync
 *     waits for them.  Results are visible after q48_sync or a
 *     q48_memcpy_d2h (which is synchronous).
 *   - Return 0 (Q48_OK) or a negative Q48_E* code; nothing aborts.
 *     q48_strerror turns a code into text.
 *   - One context per host thread.  The reference is single-threaded
 *     (llama_int.c has no threads); contexts are independent.
 */
#ifndef INTLLM_HIP_H
#define INTLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q48_OK          0
#define Q48_EINVAL     (-1)   /* bad argument (null pointer, size <= 0, shape) */
#define Q48_ENOMEM     (-2)   /* device allocation failed                     */
#define Q48_EHIP       (-3)   /* HIP runtime / launch error                    */
#define Q48_ERANGE     (-4)   /* token or position out of range               */
#define Q48_ESTATE     (-5)   /* op needs state not yet set up (rope tables)  */
#define Q48_ETIMEOUT   (-6)   /* a one-launch split attention could not finish */
#define Q48_ETOOBIG    (-7)   /* size exceeds the allocation-free scratch      */

typedef struct q48_ctx q48_ctx;

/* ---- context, memory, stream -------------------------------------------- */

/* Create a context on HIP device `device`: a stream of default priority and
 * the fp_math constants (FP_PI, CORDIC angles and gain) computed on the
 * device exactly as fp_math_init does (fp_math.h:833-858). */
int q48_ctx_create(q48_ctx **out, int device);
int q48_ctx_destroy(q48_ctx *ctx);

int q48_malloc(q48_ctx *ctx, void **dptr, size_t bytes);
int q48_free(q48_ctx *ctx, void *dptr);
/* Synchronous copies (the stream is drained first). */
int q48_memcpy_h2d(q48_ctx *ctx, void *dst, const void *src, size_t bytes);
int q48_memcpy_d2h(q48_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Stream-ordered device-to-device copy. */
int q48_memcpy_d2d(q48_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Stream-ordered zero fill (a kernel, so it may be graph-captured).
 * Replaces kv_cache_reset's memset (llama_int.c:1170-1183). */
int q48_zero(q48_ctx *ctx, void *dptr, size_t bytes);
int q48_sync(q48_ctx *ctx);
const char *q48_strerror(int code);

/* ---- the six hot-path ops ------------------------------------------------ */

/* y[i] = (int64)((sum_j (int128)W[i*K + j] * x[j]) >> 48), i < M.
 * Replaces matmul_vec(out, weight, in, M, N=K)  (llama_int.c:1014-1046). */
int q48_gemv(q48_ctx *ctx, int64_t *y, const int64_t *W, const int64_t *x,
             int M, int K);

/* Batched prefill: Y[t][i] = matmul_vec row i of token t, for t < T.
 * W [N][K], X [T][K], Y [T][N].  Each element is exactly what
 * matmul_vec gives for that token (llama_int.c:1014-1046 per token; the
 * reference prefills one token at a time, llama_int.c:3081-3092). */
int q48_gemm(q48_ctx *ctx, int64_t *Y, const int64_t *W, const int64_t *X,
             int T, int N, int K);

/* q48_gemm with the kernel named: Q48_GEMM_VALU multiplies 32-bit limbs on
 * the vector ALUs; Q48_GEMM_I8 splits both operands into int8 digits and
 * multiplies them on the matrix cores (v_mfma_i32_32x32x32_i8), with the
 * split either inside the k loop (Q48_GEMM_I8_FUSED) or done once per call
 * into digit planes that the k loop reads by DMA (Q48_GEMM_I8_PLANES);
 * Q48_GEMM_I8 picks one of the two by shape, and Q48_GEMM_AUTO is q48_gemm's
 * choice (the decode GEMV for T = 1, else Q48_GEMM_I8).  All give the same
 * bits.  No reference counterpart: it exists so that callers and benchmarks
 * can compare the kernels on the same inputs. */
#define Q48_GEMM_AUTO      0
#define Q48_GEMM_VALU      1
#define Q48_GEMM_I8        2
#define Q48_GEMM_I8_FUSED  3
#define Q48_GEMM_I8_PLANES 4
int q48_gemm_ex(q48_ctx *ctx, int64_t *Y, const int64_t *W, const int64_t *X,
                int T, int N, int K, int kernel);

/* A weight matrix's digit planes, prepared once for every later q48_gemm on
 * it (the int8 kernel otherwise splits W into planes in each call that
 * takes the planes path).  q48_gemm_planes_bytes gives the size of the
 * buffer (device memory the caller owns, 16-byte aligned; about 8 bytes per
 * weight); q48_gemm_prepare fills it from W [N][K]; q48_gemm_prepared is
 * q48_gemm over W with those planes (W itself is still read where a block's
 * digits leave the int8 kernel's window, and for T = 1).  Same bits as
 * q48_gemm.  The planes describe W as it was when prepared: prepare again
 * after W changes.  No reference counterpart (the reference has no batched
 * prefill): it exists for callers that run many prefills over one model. */
int q48_gemm_planes_bytes(int N, int K, size_t *bytes);
int q48_gemm_prepare(q48_ctx *ctx, void *Wp, const int64_t *W, int N, int K);
int q48_gemm_prepared(q48_ctx *ctx, int64_t *Y, const int64_t *W, const void *Wp,
                      const int64_t *X, int T, int N, int K);

/* out = rmsnorm(x) * w.  Replaces rmsnorm (llama_int.c:1048-1058). */
int q48_rmsnorm(q48_ctx *ctx, int64_t *out, const int64_t *x,
                const int64_t *w, int dim);

/* Build the RoPE cos/sin tables [max_seq][head_dim/2] on the device.
 * Replaces rope_init (llama_int.c:960-986); same bits. */
int q48_rope_init(q48_ctx *ctx, int head_dim, int max_seq, int theta);

/* Rotate n_heads consecutive head vectors of vec in place at `pos`.
 * Replaces the rope_apply loops (llama_int.c:997-1008, 1392-1395). */
int q48_rope(q48_ctx *ctx, int64_t *vec, int n_heads, int head_dim, int pos);

/* Store k_new / v_new ([n_kv][head_dim]) at cache[layer][pos] and compute
 * exact GQA attention for all n_heads query heads over positions 0..pos.
 * Cache layout [layers][max_seq][n_kv][head_dim] (kv_key_at,
 * llama_int.c:1185-1195).  Replaces the KV store, scale, exact attention
 * and softmax of transformer_layer_forward (llama_int.c:1414-1416, 1433,
 * 1502-1529, 1060-1072).  q and k_new must already be rotated. */
int q48_attn_decode(q48_ctx *ctx, int64_t *out, const int64_t *q,
                    int64_t *kcache, int64_t *vcache, const int64_t *k_new,
                    const int64_t *v_new, int layer, int pos, int n_heads,
                    int n_kv, int head_dim, int max_seq);

/* out[i] = fp_mul(fp_silu(gate[i]), up[i]).  Replaces the SwiGLU loops
 * (llama_int.c:1549-1552, fp_math.h:911-921). */
int q48_silu_mul(q48_ctx *ctx, int64_t *out, const int64_t *gate,
                 const int64_t *up, int n);

/* ---- small ops of llama_forward ----------------------------------------- */

/* acc[i] += d[i] (int64, wrapping): the residual adds (llama_int.c:1535,
 * 1556). */
int q48_add(q48_ctx *ctx, int64_t *acc, const int64_t *d, int n);

/* out = table[token] ([dim] row): the embedding lookup
 * (llama_int.c:2822-2824).  The caller range-checks token as
 * llama_forward does (llama_int.c:2813-2820). */
int q48_embed(q48_ctx *ctx, int64_t *out, const int64_t *table, int token,
              int dim);

/* Greedy token: index of the first maximum of v[0..n) (argmax,
 * llama_int.c:2888-2893).  Writes *host_out; synchronises. */
int q48_argmax(q48_ctx *ctx, const int64_t *v, int n, int *host_out);

/* ---- introspection / parity hooks ---------------------------------------- */

/* Device pointers of the current RoPE tables (after q48_rope_init). */
int q48_rope_tables(q48_ctx *ctx, const int64_t **cos_t, const int64_t **sin_t);

/* Evaluate one fp_math function element-wise on the device (no reference
 * FFI counterpart: this is fp_determinism.c's evaluation step,
 * fp_determinism.c:175-195, exposed so the gate can run on the GPU).
 * func: 0 mul(x,y) 1 div(x,y) [0 where y==0] 2 sqrt 3 sqrt_fast
 * 4 inv_sqrt 5 exp 6 log 7 sincos (out0=cos, out1=sin) 8 sigmoid 9 silu
 * 10 safe_exp 11 exp_dyadic(x, k=y) 12 div(x,y) [0 where y==0] through the
 * prepared-divisor quotient the softmax rows use.  out1 may be NULL unless
 * func 7. */
int q48_fp_eval(q48_ctx *ctx, int func, const int64_t *x, const int64_t *y,
                int64_t *out0, int64_t *out1, int n);

/* ---- fused decode ops ------------------------------------------------------- */
/* Each is exactly the composition it names (same bits as the separate ops);
 * fusing removes launches and a round trip of the activation through HBM. */

/* y = W . rmsnorm(x, norm_w): rmsnorm (llama_int.c:1048-1058) followed by
 * matmul_vec (llama_int.c:1014-1046), K = dim of x.  Used for q|k|v
 * (llama_int.c:1384-1389) and the lm_head (llama_int.c:2876-2880). */
int q48_rmsnorm_gemv(q48_ctx *ctx, int64_t *y, const int64_t *W, const int64_t *x,
                     const int64_t *norm_w, int M, int K);

/* acc += W . x: matmul_vec then the residual add (llama_int.c:1532-1535,
 * 1553-1556). */
int q48_gemv_residual(q48_ctx *ctx, int64_t *acc, const int64_t *W, const int64_t *x,
                      int M, int K);

/* out[i] = fp_mul(fp_silu(g_i), u_i) with g = rows 0..ffn-1 and u = rows
 * ffn..2ffn-1 of Wgu . rmsnorm(x, norm_w): the post-attention norm, the
 * gate/up projections and SwiGLU (llama_int.c:1544-1552).  Wgu [2*ffn][K]
 * is gate_proj stacked on up_proj. */
int q48_rmsnorm_gemv_swiglu(q48_ctx *ctx, int64_t *out, const int64_t *Wgu,
                            const int64_t *x, const int64_t *norm_w, int ffn, int K);

/* q48_attn_decode with the RoPE of q and k_new fused in (rope_apply,
 * llama_int.c:997-1008, 1392-1395): q and k_new are given unrotated, the
 * cache receives rotated k.  Needs q48_rope_init(head_dim, >= max_seq) and
 * head_dim % 8 == 0. */
int q48_attn_decode_rope(q48_ctx *ctx, int64_t *out, const int64_t *q,
                         int64_t *kcache, int64_t *vcache, const int64_t *k_new,
                         const int64_t *v_new, int layer, int pos, int n_heads,
                         int n_kv, int head_dim, int max_seq);
/* First position at which q48_attn_decode_rope(_prefetch) serves a head with
 * the split kernels (chunks of the cache over many compute units) instead
 * of one block per head.  Kernels are chosen from the pos argument, also in
 * step mode: a graph captured below this position keeps the one-block
 * kernels as replays move past it (same bits, slower). */
int q48_attn_split_min(void);
/* Split attention as ONE launch (on: the default), whose chunk blocks hand
 * the softmax's global max and sum to each other at two barriers inside the
 * kernel, or as three launches (off).  Same bits either way.  The one-launch
 * form serves a cache whose blocks (heads x chunks of max_seq) can all be
 * resident at once; otherwise the three launches run.  No reference
 * counterpart: a scheduling choice of this library. */
int q48_set_attn_one_launch(q48_ctx *ctx, int on);
/* Batched-prefill attention (q48_attn_prefill) with the q.k and p.v products
 * on the int8 matrix cores (on: the default, for head_dim 32, 64 or 128 and
 * up to 16320 cache rows) or on the VALU, one block per (head, query row)
 * (off; up to 4096 cache rows).  Same bits either way.  No reference
 * counterpart: a kernel choice of this library. */
int q48_set_pf_attn_mfma(q48_ctx *ctx, int on);
/* Decode attention from q48_attn_split_min() (the one-launch split form, head_dim
 * 64) with its q.k scores on the int8 matrix cores (on: the default) or on
 * the VALU (off).  Same bits either way.  No reference counterpart: a kernel
 * choice of this library. */
int q48_set_attn_g_mfma(q48_ctx *ctx, int on);
/* q48_attn_decode_rope without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  q48_attn_decode_rope grows the context's workspace with
 * hipMalloc when a longer cache needs it; this entry takes the split
 * attention's workspace from a fixed per-device array of 4 MiB (its usable
 * part is q48_attn_noalloc_max_bytes()) and returns Q48_ETOOBIG, launching
 * nothing, when the call would need more.  Same arguments, same bits.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (from two contexts or two streams) race. */
int q48_attn_decode_rope_noalloc(q48_ctx *ctx, int64_t *out, const int64_t *q,
                                 int64_t *kcache, int64_t *vcache, const int64_t *k_new,
                                 const int64_t *v_new, int layer, int pos, int n_heads,
                                 int n_kv, int head_dim, int max_seq);
size_t q48_attn_noalloc_max_bytes(void);
/* Synchronises; Q48_ETIMEOUT if a one-launch split attention launched since
 * the last call could not finish (a block waited past its bound: blocks were
 * not all resident; its output is then wrong and its exchange words are
 * cleared, so the next launch starts clean), else Q48_OK.  The reference's
 * llama_forward cannot fail this way; its callers treat a failed forward
 * (NULL) as the end of generation (llama_int.c:3083-3086, 3106), and
 * q48h_forward / q48h_generate / q48h_decode_* return this code. */
int q48_attn_status(q48_ctx *ctx);
/* The one-launch split attention's wait bound in wall-clock ticks (a
 * negative value restores the default, 2^24 ticks); 0 makes every chunk
 * block give up at its first exchange without waiting, so that the timeout
 * path can be tested while every block still exits normally.  No reference
 * counterpart.  Changes q48_graph_stamp. */
int q48_set_attn_wait(q48_ctx *ctx, int64_t ticks);

/* Long normed GEMVs (more than two rounds of 8-row groups: gate|up, lm_head)
 * run as persistent blocks that loop over row groups (on: the default), or
 * one block per group (off).  Same bits either way.  No reference
 * counterpart: a scheduling choice of this library. */
int q48_set_gemv_persistent(q48_ctx *ctx, int on);
/* q48_attn_decode_rope that also reads [prefetch, prefetch + prefetch_bytes)
 * (16-byte aligned; typically the next op's weights, W_o) on the compute
 * units the heads leave idle, so that the next op finds them in the
 * device-side cache.  No reference counterpart (a scheduling hint: the
 * results are those of q48_attn_decode_rope). */
int q48_attn_decode_rope_prefetch(q48_ctx *ctx, int64_t *out, const int64_t *q,
                                  int64_t *kcache, int64_t *vcache, const int64_t *k_new,
                                  const int64_t *v_new, int layer, int pos, int n_heads,
                                  int n_kv, int head_dim, int max_seq, const void *prefetch,
                                  size_t prefetch_bytes);

/* The decode layer's first half split the other way: the projection's
 * epilogue does RoPE and the KV store, so that attention starts from the
 * cache.  q48_norm_gemv_rope_kv: qkv = W . rmsnorm(x, norm_w) (statistics as
 * partial sums, see Q48_STATS_WORDS; rmsnorm and matmul_vec,
 * llama_int.c:1048-1058, 1014-1046, 1384-1389) with W the q, k and v
 * projections stacked ([(n_heads + 2 n_kv) head_dim][K]), then rope_apply on
 * the q and k heads (llama_int.c:997-1008, 1392-1395) and k, v stored in the
 * caches at pos (llama_int.c:1414-1416).  qkv receives every row, q and k
 * rotated.  Needs q48_rope_init(head_dim, >= max_seq), head_dim 32, 64 or
 * 128.  In step mode pos is read from the device-side state. */
int q48_norm_gemv_rope_kv(q48_ctx *ctx, int64_t *qkv, const int64_t *W, const int64_t *x,
                          const int64_t *norm_w, const int64_t *stats, int64_t *kcache,
                          int64_t *vcache, int layer, int pos, int n_heads, int n_kv,
                          int head_dim, int max_seq, int K);
/* q48_norm_gemv_rope_kv on bfloat16 weights (the bfloat16 section's rules). */
int q48_norm_gemv_rope_kv_bf16(q48_ctx *ctx, int64_t *qkv, const uint16_t *W,
                               const int64_t *x, const int64_t *norm_w, const int64_t *stats,
                               int64_t *kcache, int64_t *vcache, int layer, int pos,
                               int n_heads, int n_kv, int head_dim, int max_seq, int K);
/* Attention of one token over the cache (llama_int.c:1060-1072, 1502-1529)
 * after q48_norm_gemv_rope_kv: q rotated, the key and value at pos already
 * in the caches.  max_seq <= 4096; prefetch (16-byte aligned, may be NULL)
 * as in q48_attn_decode_rope_prefetch.  Same bits as q48_attn_decode_rope on
 * the unrotated inputs. */
int q48_attn_decode_cached(q48_ctx *ctx, int64_t *out, const int64_t *q, int64_t *kcache,
                           int64_t *vcache, int layer, int pos, int n_heads, int n_kv,
                           int head_dim, int max_seq, const void *prefetch,
                           size_t prefetch_bytes);

/* The same fusions with the rmsnorm statistics computed once per vector:
 * r = fp_inv_sqrt((int64)((sum x^2 >> 48) / dim) + 2814749767), the scalar
 * of rmsnorm (llama_int.c:1049-1055), lives in device memory (*r) and the
 * consumers apply fp_mul(fp_mul(x, r), norm_w) (llama_int.c:1056-1057). */
int q48_rms_inv(q48_ctx *ctx, int64_t *r_out, const int64_t *x, int dim);
/* out = table[token] (llama_int.c:2822-2824) and *r_out = its statistics. */
int q48_embed_rms(q48_ctx *ctx, int64_t *out, const int64_t *table, int token, int dim,
                  int64_t *r_out);
/* y = W . (x * r * norm_w): q48_rmsnorm_gemv with r given. */
int q48_norm_gemv(q48_ctx *ctx, int64_t *y, const int64_t *W, const int64_t *x,
                  const int64_t *norm_w, const int64_t *r, int M, int K);
/* q48_rmsnorm_gemv_swiglu with r given. */
int q48_norm_gemv_swiglu(q48_ctx *ctx, int64_t *out, const int64_t *Wgu, const int64_t *x,
                         const int64_t *norm_w, const int64_t *r, int ffn, int K);
/* acc += W . x (residual add), then *r_out = the rmsnorm statistics of the
 * updated acc (dim M): the producer of the next norm's r. */
int q48_gemv_residual_rms(q48_ctx *ctx, int64_t *acc, const int64_t *W, const int64_t *x,
                          int M, int K, int64_t *r_out);

/* The same fusions with the statistics left as partial sums: stats[2i],
 * stats[2i + 1] (lo, hi words) hold the 128-bit sum of squares of rows
 * 8i .. 8i+7 of the vector, Q48_STATS_WORDS(dim) int64 words in all.  The
 * producer of a vector writes them with no cross-block step; every block of
 * the consumer adds them up and derives r itself while its weight loads are
 * in flight (same r, same bits as rmsnorm, llama_int.c:1048-1058). */
#define Q48_STATS_WORDS(dim) (2 * (((dim) + 7) / 8))
int q48_rms_stats(q48_ctx *ctx, int64_t *stats, const int64_t *x, int dim);
/* out = table[token] (llama_int.c:2822-2824) and the partial sums of that row. */
int q48_embed_stats(q48_ctx *ctx, int64_t *out, const int64_t *table, int token, int dim,
                    int64_t *stats);
/* y = W . rmsnorm(x, norm_w) with the statistics of x given as partial sums. */
int q48_norm_gemv_stats(q48_ctx *ctx, int64_t *y, const int64_t *W, const int64_t *x,
                        const int64_t *norm_w, const int64_t *stats, int M, int K);
/* q48_rmsnorm_gemv_swiglu with the statistics of x given as partial sums. */
int q48_norm_gemv_swiglu_stats(q48_ctx *ctx, int64_t *out, const int64_t *Wgu,
                               const int64_t *x, const int64_t *norm_w,
                               const int64_t *stats, int ffn, int K);
/* acc += W . x (residual add), then the partial sums of the updated acc
 * (dim M) into stats. */
int q48_gemv_residual_stats(q48_ctx *ctx, int64_t *acc, const int64_t *W, const int64_t *x,
                            int M, int K, int64_t *stats);

/* ---- bfloat16-resident weights ------------------------------------------
 * The reference's .mgwc format (llama_int.c:1906-1929) keeps weights as
 * their bfloat16 bits and expands them with bfloat16_to_q1648
 * (safetensors.h:115-152) at load.  These GEMVs keep the bits in device
 * memory (2 bytes per weight) and expand each one in the kernel with the
 * same rule, so for weights that are bfloat16 values the results are the
 * int64-weight results, bit for bit, from a quarter of the weight bytes.
 * W is [M][K] uint16, 16-byte aligned; x, norm_w and stats 16-byte aligned;
 * K a multiple of 512 (else Q48_EINVAL).  No reference counterpart beyond
 * the format: the reference expands at load time. */

/* out[i] = the bfloat16 bits b with bfloat16_to_q1648(b) == in[i], for n
 * elements; *inexact = 1 (host int) when some in[i] has no such b (then the
 * weights must stay int64).  Synchronises. */
int q48_bf16_pack(q48_ctx *ctx, uint16_t *out, const int64_t *in, size_t n, int *inexact);
/* q48_gemv on bfloat16 weights. */
int q48_gemv_bf16(q48_ctx *ctx, int64_t *y, const uint16_t *W, const int64_t *x, int M, int K);
/* q48_norm_gemv_stats on bfloat16 weights. */
int q48_norm_gemv_stats_bf16(q48_ctx *ctx, int64_t *y, const uint16_t *W, const int64_t *x,
                             const int64_t *norm_w, const int64_t *stats, int M, int K);
/* q48_norm_gemv_swiglu_stats on bfloat16 weights (Wgu is [2 ffn][K]). */
int q48_norm_gemv_swiglu_stats_bf16(q48_ctx *ctx, int64_t *out, const uint16_t *Wgu,
                                    const int64_t *x, const int64_t *norm_w,
                                    const int64_t *stats, int ffn, int K);
/* q48_gemv_residual_stats on bfloat16 weights. */
int q48_gemv_residual_stats_bf16(q48_ctx *ctx, int64_t *acc, const uint16_t *W,
                                 const int64_t *x, int M, int K, int64_t *stats);

/* ---- device-resident decode steps (graph replay) ---------------------------- */
/* No reference counterpart: llama_int's generate (llama_int.c:3067-3135)
 * passes token and pos as C arguments each call.  In step mode q48_embed,
 * q48_embed_rms and q48_embed_stats read the token, and q48_rope / q48_attn_decode(_rope) read pos, from a
 * device-side state {token, pos, count} instead of their arguments, and
 * q48_argmax_step writes the greedy token back into that state (pos += 1),
 * so one captured forward can be replayed for consecutive tokens with no
 * host round trip.  Kernels ignore a state position outside the cache. */
int q48_step_mode(q48_ctx *ctx, int on);
int q48_step_set(q48_ctx *ctx, int token, int pos);      /* stream-ordered */
int q48_step_get(q48_ctx *ctx, int *token, int *pos, int *count);  /* syncs */
/* argmax (llama_int.c:2888-2893) of v[0..n) into the state; the token is
 * also stored at d_tokens[count] while count < cap. */
int q48_argmax_step(q48_ctx *ctx, const int64_t *v, int n, int *d_tokens, int cap);
/* Parity hook of the replayed steps.  No reference counterpart: it keeps the
 * logits of each step (what llama_forward returns to generate,
 * llama_int.c:3082 and 3105) so that the host can hash every replayed step.
 * Copies v[0..n) to rec[count * n ..] while count < cap, count being the
 * state's number of tokens chosen so far; enqueue it before the step's
 * q48_argmax_step or q48_sample_step. */
int q48_record_step(q48_ctx *ctx, const int64_t *v, int n, int64_t *rec, int cap);
/* q48_record_step (into rec, rec_cap) followed by q48_argmax_step, as one
 * launch: the same record and the same token.  No reference counterpart
 * (as q48_record_step). */
int q48_argmax_record_step(q48_ctx *ctx, const int64_t *v, int n, int *d_tokens, int cap,
                           int64_t *rec, int rec_cap);


/* ---- batched prefill ------------------------------------------------------ */
/* No reference counterpart as a batch: llama_int's prefill calls
 * llama_forward once per prompt token (llama_int.c:3081-3092).  These are the
 * per-token ops of transformer_layer_forward over T rows (token t at
 * position p0 + t), for a prefill whose projections are q48_gemm; each row
 * gets the reference's bits for its token.  Row-major [T][...] buffers. */
/* hidden[t] = embed[d_tokens[t]] (llama_int.c:2822-2824; ids on the device,
 * range-checked by the caller). */
int q48_embed_rows(q48_ctx *ctx, int64_t *H, const int64_t *table, const int *d_tokens, int T,
                   int dim);
/* rmsnorm (llama_int.c:1048-1058) of every row. */
int q48_rmsnorm_rows(q48_ctx *ctx, int64_t *out, const int64_t *X, const int64_t *w, int T,
                     int dim);
/* RoPE (llama_int.c:997-1008, 1392-1395) of the q and k heads of every
 * [q | k | v] row in place, then the KV store (1414-1416) at p0 + t. */
int q48_rope_store_rows(q48_ctx *ctx, int64_t *QKV, int64_t *kcache, int64_t *vcache, int layer,
                        int p0, int T, int n_heads, int n_kv, int head_dim, int max_seq);
/* Exact causal attention (llama_int.c:1433, 1502-1529) of the rotated q of
 * every row over cache positions 0 .. p0 + t (stored by
 * q48_rope_store_rows); out[T][n_heads * head_dim].  p0 + T at most 16320
 * (head_dim 32, 64, 128; 4096 on the VALU kernel, see q48_set_pf_attn_mfma).
 * Uses up to 16 * 8 bytes per (head, query row, cache row) of workspace. */
int q48_attn_prefill(q48_ctx *ctx, int64_t *out, const int64_t *QKV, int64_t *kcache,
                     int64_t *vcache, int layer, int p0, int T, int n_heads, int n_kv,
                     int head_dim, int max_seq);
/* SwiGLU (llama_int.c:1549-1552) of every [gate | up] row: out[T][ffn]. */
int q48_silu_mul_rows(q48_ctx *ctx, int64_t *out, const int64_t *GU, int T, int ffn);

/* ---- sampling (sample_token, llama_int.c:2958-3039) --------------------- */
/* rng_seed (llama_int.c:2909-2920): the xoroshiro128+ state of a seed
 * (SplitMix64), computed on the host.  Upload it to a device buffer of two
 * uint64 words for q48_sample / q48_sample_step. */
void q48_rng_seed(uint64_t seed, uint64_t state[2]);
/* sample_token on device logits[0..vocab): temperature (Q16.48), top_k
 * (0 = off), top_p (Q16.48, ONE = off), and one rng_next draw from the
 * device state rng[2], advanced in place.  Below a temperature of 0.01 it is
 * argmax and draws nothing, as the reference.  The token goes to *token
 * (host; the call synchronises). */
int q48_sample(q48_ctx *ctx, const int64_t *logits, int vocab, int64_t temperature,
               int top_k, int64_t top_p, uint64_t *rng, int *token);
/* The same into the decode-step state (as q48_argmax_step): stream-ordered,
 * graph-capturable once q48_sample_reserve has sized the workspace. */
int q48_sample_step(q48_ctx *ctx, const int64_t *logits, int vocab, int64_t temperature,
                    int top_k, int64_t top_p, uint64_t *rng, int *d_tokens, int cap);
/* Size the sampling workspace for `vocab` logits (synchronises; not during
 * capture). */
int q48_sample_reserve(q48_ctx *ctx, int vocab);

/* Graph capture of stream-ordered ops (no reference counterpart: the
 * reference calls llama_forward once per token, llama_int.c:3103-3113; a
 * captured decode step replays that call's kernels with the token and
 * position read from the device step state).
 *
 * The context graph: begin captures into it (replacing any previous one),
 * end instantiates it, launch replays it, drop destroys it.  Destroying waits
 * for the stream first, so in-flight launches finish. */
int q48_graph_begin(q48_ctx *ctx);
int q48_graph_end(q48_ctx *ctx);
int q48_graph_launch(q48_ctx *ctx, int times);
int q48_graph_drop(q48_ctx *ctx);
/* Graphs the caller holds, any number at once: q48_graph_capture starts a
 * capture that q48_graph_instantiate ends into a new handle (uploaded to the
 * device before it returns); q48_graph_replay launches it `times` times;
 * q48_graph_destroy waits for the stream and frees it.  Workspaces the
 * context replaces while any graph is alive are freed only after the last
 * graph is destroyed, so a graph never replays against freed memory.
 * q48_graph_stamp changes whenever a context setting that selects the
 * kernels or kernel arguments a capture records changes (the q48_set_*
 * switches, q48_rope_init with new parameters): a caller that caches graphs
 * keys them on it. */
typedef struct q48_graph q48_graph;
int q48_graph_capture(q48_ctx *ctx);
int q48_graph_instantiate(q48_ctx *ctx, q48_graph **out);
int q48_graph_replay(q48_ctx *ctx, q48_graph *graph, int times);
int q48_graph_destroy(q48_ctx *ctx, q48_graph *graph);
uint64_t q48_graph_stamp(const q48_ctx *ctx);

/* ---- kernel timing (diagnostic) -------------------------------------------- */

/* HIP-event timing of every GEMV launch (q48_gemv and the fused GEMV entry
 * points) on the context's stream while enabled (no reference counterpart:
 * llama_int's profiler, llama_int.c:65-108, times whole forwards with
 * clock_gettime).  `bytes` is the algorithmic traffic 8*(M*K + K + outputs)
 * per launch.  Not recorded while a graph is being captured. */
typedef struct {
    int launches;
    double ms;       /* sum of launch durations */
    double bytes;    /* sum of algorithmic bytes */
} q48_prof;

int q48_prof_enable(q48_ctx *ctx, int on);
/* Elapsed time of everything enqueued between start and stop, from two HIP
 * events on the context's stream (stop synchronises). */
int q48_timer_start(q48_ctx *ctx);
int q48_timer_stop(q48_ctx *ctx, double *ms);
/* Synchronise, then report (and with reset != 0 clear) the GEMV timings. */
int q48_prof_read(q48_ctx *ctx, q48_prof *gemv, int reset);

#ifdef __cplusplus
}
#endif
#endif /* INTLLM_HIP_H */
