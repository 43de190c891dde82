// q48_internal.h — context and kernel launchers shared by the HIP sources
// of libintllm_hip (not installed; the public ABI is include/intllm_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/intllm_hip.h"
#include "q48_device.hpp"

struct q48_ctx {
    int device;
    int cu_count;                // compute units of the device
    int gemv_persistent;         // long normed GEMVs take k_gemv_p6 (default on)
    hipStream_t stream;
    q48_consts *consts;          // device: fp_math_init constants
    int64_t *rope_cos, *rope_sin; // device: [max_seq][head_dim/2]
    int rope_head_dim, rope_max_seq, rope_theta;
    void *ws;                    // device workspace (scores, row sums, partials)
    size_t ws_bytes;
    int *d_scalar;               // device: small int outputs (argmax)
    int *d_step;                 // device: decode-step state {token, pos, count}
    uint64_t *amax_part;         // device: q48_argmax_step's per-block (max, index) partials,
                                 // then its ticket (back to 0 after use); zeroed at creation
    int step_mode;               // ops read token / pos from d_step
    void *tmp;                   // device temporaries of the unfused fallbacks
    size_t tmp_bytes;
    uint64_t *rms_part;          // device: per-block partial sums of squares (EPI 3)
    int *rms_count;              // device: tickets, back to 0 after use: [0] EPI 3 blocks
                                 // finished
    int rms_blocks;
    int64_t *smp;                // device: sampling workspace (q48_sample_ws_words)
    size_t smp_words;
    unsigned *attx_sync;         // device: k_attn_g's exchange region (epoch-tagged words,
                                 // per-KV-head epochs, error word); zeroed at creation
    int attn_one_launch;         // split attention as one k_attn_g launch (default on)
    int pf_attn_mfma;            // batched-prefill attention on the matrix cores (default on)
    int attx_per_cu[4];          // k_attn_g<64/32/128>, <64, matrix scores> resident blocks
                                 // per CU (-1: not asked)
    int attn_g_mfma;             // k_attn_g's scores on the matrix cores (head_dim 64; default on)
    uint64_t attg_wait;          // k_attn_g's wait bound in wall-clock ticks (0: give up at once)
    uint64_t attg_count;         // k_attn_g launches on attx_sync since it was last zeroed
    int attg_unchecked;          // k_attn_g ran since q48_attn_status last read the error words
    int64_t *scratch;            // device address of the allocation-free scratch array
    unsigned *scratch_sync;      // ... and of its exchange region
    q48_graph *cur;              // the context graph (q48_graph_begin / end / launch / drop)
    int capturing;
    uint64_t capture_attg[2];    // k_attn_g launches recorded by the capture in progress,
                                 // on attx_sync and on the scratch's region
    int n_graphs;                // instantiated graphs alive (handles and the context graph)
    uint64_t stamp;              // changes with every setting that selects captured kernels
    // buffers replaced while graphs were alive: a graph may hold their
    // addresses, so they are freed only once no graph is left
    void **retired;
    int n_retired, cap_retired;
    // GEMV launch timing (q48_prof_*): event pairs in use, then a free pool
    int prof_on;
    struct ProfRec { hipEvent_t a, b; double bytes; };
    ProfRec *prof;
    int prof_n, prof_cap;
    hipEvent_t span_a, span_b;   // q48_timer_start / q48_timer_stop
};

// An executable graph and the k_attn_g launches one replay makes on each
// exchange region ([0] the context's, [1] the allocation-free scratch's).
struct q48_graph {
    hipGraph_t g;
    hipGraphExec_t x;
    uint64_t attg[2];
};

// Grow the context workspace to at least `bytes` (stream-synchronising).
int q48_ws_reserve(q48_ctx *c, size_t bytes);
// Give back a device buffer the context owns (stream-synchronising): freed
// now, or kept until the last graph is destroyed when graphs are alive.
int q48_release(q48_ctx *c, void *p);
// Count n k_attn_g launches on the exchange region `sync` before they are
// enqueued, zeroing the region first when its 32-bit epochs could come back
// to a value a stale word still carries (stream-synchronising then).
int q48_attg_account(q48_ctx *c, const unsigned *sync, uint64_t n);
// k_attn_g's default wait bound (wall-clock ticks).
uint64_t q48_attg_default_wait();
// Launches counted on this device's scratch exchange region.
uint64_t *q48_scratch_attg_count(int device);

// ---- launchers (return hipError_t as int; shapes already validated) ----
int q48_launch_gemv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                    int M, int K);
bool q48_gemv_v2_ok(const int64_t *W, int K);
// pro: 0 none, 1 rmsnorm(x, norm_w) computed in every block, 2 with r = *r_in,
//      3 with r from the partial sums at r_in;
// epi: 0 store, 1 add into y, 2 SwiGLU pairs, 3 add into y + rms statistics -> *r_out,
//      4 add into y + partial sums -> r_out
int q48_launch_gemv_fused(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                          const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M,
                          int K, int pro, int epi);
// the same fused GEMVs on bfloat16 weight bits (pro 0/3, epi 0/2/4; K =
// 512, 1024, 2048 or 5632: q48_gemv_bf16_ok); -1 for other K
bool q48_gemv_bf16_ok(int K);
int q48_launch_gemv_fused_bf16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                               const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M,
                               int K, int pro, int epi);
// Operands of the q|k|v projection's RoPE + KV-store epilogue (epi 5): the
// projection's rows are (n_heads + 2 n_kv) heads of hd, q then k then v.
struct q48_ropekv {
    int64_t *kc, *vc;               // caches [L][max_seq][n_kv][hd]
    const int64_t *cos_t, *sin_t;   // RoPE tables [rope_max_seq][hd / 2]
    const int *d_pos;               // device position (graph replay), or null: pos
    int pos, layer, max_seq, n_heads, n_kv, hd;
};
// rmsnorm (r from the partial sums at stats) + q|k|v projection + RoPE of
// the q and k heads + k and v stored at pos; y gets every row (q and k
// rotated).  The int64 form needs q48_gemv_v2_ok, the bfloat16 one
// q48_gemv_bf16_ok.
int q48_launch_gemv_rope_kv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                            const int64_t *norm_w, const int64_t *stats,
                            const q48_ropekv *rk, int M, int K);
int q48_launch_gemv_rope_kv_bf16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                                 const int64_t *norm_w, const int64_t *stats,
                                 const q48_ropekv *rk, int M, int K);
// out[i] = the bfloat16 bits of in[i] where exact; *inexact = 1 otherwise
int q48_launch_bf16_pack(q48_ctx *c, uint16_t *out, const int64_t *in, size_t n, int *inexact);
int q48_launch_rms_inv(q48_ctx *c, int64_t *r_out, int64_t *out, const int64_t *x,
                       const int64_t *table, const int *d_token, int token, int dim);
int q48_launch_rms_apply(q48_ctx *c, int64_t *out, const int64_t *x, const int64_t *w,
                         const int64_t *r, int dim);
int q48_launch_rms_stats(q48_ctx *c, int64_t *stats, int64_t *out, const int64_t *x,
                         const int64_t *table, const int *d_token, int token, int dim);
int q48_launch_stats_r(q48_ctx *c, int64_t *r_out, const int64_t *stats, int dim);
// Grow the per-block partial sums of the rms epilogue to `blocks` entries.
int q48_rms_reserve(q48_ctx *c, int blocks);
int q48_launch_gemm(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X,
                    int T, int N, int K);
// int8-digit GEMM on the matrix cores (q48_gemm.hip); same bits as
// q48_launch_gemm.  kernel: Q48_GEMM_I8_FUSED or Q48_GEMM_I8_PLANES, anything
// else picks one of them by shape.  Wpre: W's planes from
// q48_launch_gemm_prepare (or NULL: the planes path splits W in the call).
int q48_launch_gemm_i8(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X,
                       int T, int N, int K, int kernel, const void *Wpre);
// bytes of W's digit planes and masks for q48_launch_gemm_prepare
size_t q48_gemm_planes_size(int N, int K);
int q48_launch_gemm_prepare(q48_ctx *c, void *Wp, const int64_t *W, int N, int K);
// K splits the int8 GEMM uses for this shape on cu_count compute units
int q48_gemm_i8_splits(int T, int N, int K, int cu_count);
// Q48_GEMM_VALU or Q48_GEMM_I8: the kernel q48_gemm runs for this shape
int q48_gemm_auto_kernel(int T, int N, int K);
int q48_launch_rmsnorm(q48_ctx *c, int64_t *out, const int64_t *x,
                       const int64_t *w, int dim);
int q48_launch_rope_init(q48_ctx *c);
int q48_launch_rope(q48_ctx *c, int64_t *vec, int n_heads, int head_dim,
                    const int *d_pos, int pos);
int q48_launch_attn(q48_ctx *c, int64_t *out, const int64_t *q,
                    int64_t *kcache, int64_t *vcache, const int64_t *k_new,
                    const int64_t *v_new, int layer, const int *d_pos, int pos,
                    int n_heads, int n_kv, int head_dim, int max_seq);
int q48_att_split_min();
int q48_att_lds_max();   // positions a single-block attention keeps in LDS
int q48_launch_attn_v2(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                       int64_t *vcache, const int64_t *k_new, const int64_t *v_new,
                       int layer, const int *d_pos, int pos, int n_heads, int n_kv,
                       int head_dim, int max_seq, int rope,
                       const void *prefetch, size_t prefetch_bytes,
                       int64_t *ws_ext = nullptr, size_t ws_ext_bytes = 0,
                       unsigned *sync_ext = nullptr);
// Decode attention over the cache (k_attn_v3's ROT form): q rotated, k and v
// at pos already stored (q48_launch_gemv_rope_kv); head_dim 32, 64 or 128,
// max_seq <= q48_att_lds_max().  Spare blocks warm the cache with
// `prefetch` as in q48_launch_attn_v2.
int q48_launch_attn_cached(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                           int64_t *vcache, int layer, const int *d_pos, int pos, int n_heads,
                           int n_kv, int head_dim, int max_seq, const void *prefetch,
                           size_t prefetch_bytes);
// bytes of the split attention's workspace; of its barrier region
size_t q48_attn_ws_bytes(int n_heads, int max_seq, int head_dim);
size_t q48_attn_sync_bytes();
// the allocation-free attention's scratch on the context's device: address
// (set up once per device by q48_ctx_create), bytes, and its barrier region
int q48_scratch_init(q48_ctx *c);
size_t q48_scratch_bytes();
int q48_launch_step_set(q48_ctx *c, int token, int pos);
int q48_launch_step_argmax(q48_ctx *c, int *tokens, int cap, const int64_t *v, int n,
                           int64_t *rec, int rec_cap);
size_t q48_amax_part_bytes();
int q48_launch_step_record(q48_ctx *c, int64_t *rec, int cap, const int64_t *v, int n);
int q48_launch_silu_mul_pairs(q48_ctx *c, int64_t *out, const int64_t *t, int n);
int q48_launch_silu_mul(q48_ctx *c, int64_t *out, const int64_t *g,
                        const int64_t *u, int n);
int q48_launch_add(q48_ctx *c, int64_t *acc, const int64_t *d, int n);
int q48_launch_embed(q48_ctx *c, int64_t *out, const int64_t *table,
                     const int *d_token, int token, int dim);
int q48_launch_argmax(q48_ctx *c, int *d_out, const int64_t *v, int n);
// batched prefill rows (q48_prefill.hip)
int q48_launch_pf_embed(q48_ctx *c, int64_t *H, const int64_t *table, const int *tokens, int T,
                        int dim);
int q48_launch_pf_rmsnorm(q48_ctx *c, int64_t *out, const int64_t *X, const int64_t *w, int T,
                          int dim);
int q48_launch_pf_rope_store(q48_ctx *c, int64_t *QKV, int64_t *kcache, int64_t *vcache,
                             int layer, int p0, int T, int n_heads, int n_kv, int hd,
                             int max_seq);
// the same attention with both products on the int8 matrix cores
// (q48_pfattn.hip): head_dim 32, 64 or 128 and at most
// q48_pf_attn_mfma_max_pos() cache rows
bool q48_pf_attn_mfma_ok(int p0, int T, int hd);
int q48_pf_attn_mfma_max_pos();
int q48_launch_pf_attn_mfma(q48_ctx *c, int64_t *out, const int64_t *QKV, int64_t *kcache,
                            int64_t *vcache, int layer, int p0, int T, int n_heads, int n_kv,
                            int hd, int max_seq);
int q48_launch_pf_attn(q48_ctx *c, int64_t *out, const int64_t *QKV, int64_t *kcache,
                       int64_t *vcache, int layer, int p0, int T, int n_heads, int n_kv, int hd,
                       int max_seq);
int q48_launch_pf_silu(q48_ctx *c, int64_t *out, const int64_t *GU, int T, int ffn);
// sample_token: the sampling workspace size in int64 words for n logits, and
// the kernel chain (greedy temperatures are the caller's: argmax); with
// tokens != nullptr the token goes to the decode-step state
size_t q48_sample_ws_words(int n);
int q48_launch_sample(q48_ctx *c, int64_t *ws, const int64_t *logits, int n, int64_t temperature,
                      int top_k, int64_t top_p, uint64_t *rng, int *out_tok, int *tokens, int cap);
int q48_launch_zero(q48_ctx *c, void *p, size_t bytes);
int q48_launch_math_init(q48_ctx *c);
int q48_launch_fp_eval(q48_ctx *c, int func, const int64_t *x,
                       const int64_t *y, int64_t *out0, int64_t *out1, int n);

