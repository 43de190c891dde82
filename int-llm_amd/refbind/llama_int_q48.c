/*
 * llama_int_q48.c — libintllm_hip bound into llama_int.c itself.
 *
 * This is the reference-side binding: the code a maintainer adds to
 * llama_int.c so that its llama_forward runs on the GPU while the rest of
 * the program (config.json / .mgw loading, generate, sample_token, the CLI)
 * stays as it is.  It is compiled in ONE translation unit with the
 * unmodified llama_int.c (included below, from where it lies), so it is
 * written against the reference's own types and fields:
 *   llama_config_t   llama_int.c:788-798   (hidden_dim, num_heads, ...)
 *   layer_weights_t  llama_int.c:1250-1260 (q_proj ... down_proj)
 *   llama_model_t    llama_int.c:1575-1602
 * and replaces, call for call:
 *   transformer_layer_forward  llama_int.c:1326-1569  -> layer_forward_q48
 *   llama_forward              llama_int.c:2807-2886  -> llama_forward_q48
 *
 * Routing.  In llama_int.c the patch is one line at the top of
 * llama_forward:
 *       if (g_q48.ctx) return llama_forward_q48(m, token, pos);
 * This build leaves the file untouched and reaches the same routing with the
 * preprocessor: every use of the name llama_forward goes through the macro
 * below.  The definition (whose first parameter starts with the type name
 * llama_model_t) becomes llama_forward_cpu; the four call sites (their
 * first argument is `m`: llama_int.c:3082, 3105, 3510, 4207) become a call
 * through g_q48_forward when it is set, else to llama_forward_cpu.  So the
 * reference's own generate(), verify and benchmark loops call the device
 * forward.
 *
 * Nothing falls back to the CPU: with the binding attached, a failing
 * library call makes llama_forward_q48 print the error and return NULL,
 * which the reference's callers treat as a failed forward.
 */
#include <stdint.h>

typedef void (*q48_any_fn)(void);
static q48_any_fn g_q48_forward; /* non-NULL: llama_forward's callers run it */

#define llama_forward(first, ...) Q48_LLAMA_FORWARD_##first, __VA_ARGS__)
#define Q48_LLAMA_FORWARD_llama_model_t llama_forward_cpu(llama_model_t
#define Q48_LLAMA_FORWARD_m                                                          \
    (g_q48_forward ? (fixed_t * (*)(llama_model_t *, int, int)) g_q48_forward     \
                   : llama_forward_cpu)(m

#define main llama_int_main
#include "llama_int.c"
#undef main
#undef llama_forward

#include "intllm_hip.h"

/* ======================================================================== */
/*  The patch (what a maintainer pastes into llama_int.c after llama_forward) */
/* ======================================================================== */

/* Device copies of layer_weights_t (llama_int.c:1250-1260), same fields.
 * q_proj, k_proj and v_proj are consecutive rows of one [q; k; v] matrix
 * (qkv), gate_proj and up_proj of one [gate; up] matrix (gu): stacking rows
 * changes no row's dot product (matmul_vec is row-independent,
 * llama_int.c:1014-1046), and it lets one fused launch produce q|k|v and one
 * gate|up. */
typedef struct {
    int64_t *input_layernorm, *q_proj, *k_proj, *v_proj, *o_proj;
    int64_t *post_attn_norm, *gate_proj, *up_proj, *down_proj;
    int64_t *qkv, *gu;
} q48_layer_dev_t;

/* The device side of one llama_model_t: weights, the exact KV cache in
 * kv_cache_t's layout [layers][max_seq_len][num_kv_heads][head_dim]
 * (llama_int.c:1078-1095, 1185-1195) and the layer scratch (the buffers of
 * llama_init_scratch, llama_int.c:1607-1637, with q|k|v and gate|up
 * stacked), plus the norm statistics the fused launches hand on. */
typedef struct {
    q48_ctx *ctx;
    const llama_model_t *model;        /* the host model these copies mirror */
    int64_t *embed_tokens, *final_norm, *lm_head;
    q48_layer_dev_t *layers;
    int64_t *key_cache, *value_cache;
    int64_t *hidden, *normed, *q, *k, *v, *attn_out, *o_out;
    int64_t *gate, *up, *mlp_out, *logits;
    int64_t *s_attn, *s_ffn;           /* partial sums of squares (Q48_STATS_WORDS) */
    int fused;                         /* 1: five fused launches per layer, graph
                                          replay; 0: one library call per step
                                          of transformer_layer_forward */
    q48_graph *graph[2];               /* captured forward, below / from the split
                                          position (q48_attn_split_min) */
    uint64_t graph_stamp[2];
} q48_model_dev_t;

static q48_model_dev_t g_q48;

static int q48_check(int rc, const char *what)
{
    if (rc)
        fprintf(stderr, "libintllm_hip: %s: %s\n", what, q48_strerror(rc));
    return rc;
}

static int64_t *q48_upload(const int64_t *src, size_t n, int *rc)
{
    void *d = NULL;
    if (*rc)
        return NULL;
    *rc = q48_check(q48_malloc(g_q48.ctx, &d, n * sizeof(int64_t)), "q48_malloc");
    if (!*rc && src)
        *rc = q48_check(q48_memcpy_h2d(g_q48.ctx, d, src, n * sizeof(int64_t)), "upload");
    return (int64_t *)d;
}

/* Copy n elements to the device at dst (already allocated). */
static void q48_put(int64_t *dst, const int64_t *src, size_t n, int *rc)
{
    if (!*rc)
        *rc = q48_check(q48_memcpy_h2d(g_q48.ctx, dst, src, n * sizeof(int64_t)), "upload");
}

static void q48_detach(void);
static fixed_t *llama_forward_q48(llama_model_t *m, int token, int pos);

/* Upload a loaded model (mgw_load, or the safetensors path with its layers
 * cached) to device `device` and route llama_forward to the GPU.  The
 * reference's RoPE tables are rebuilt on the device by q48_rope_init (the
 * same bits as rope_init, llama_int.c:960-986). */
static int q48_attach(const llama_model_t *m, int device)
{
    const llama_config_t *c = &m->cfg;
    const size_t dim = (size_t)c->hidden_dim, kv_dim = (size_t)c->num_kv_heads * c->head_dim;
    const size_t inter = (size_t)c->intermediate_dim, vocab = (size_t)c->vocab_size;
    int rc;
    q48_detach();
    if (!m->layers_cached || !m->cached_layers) {
        fprintf(stderr, "libintllm_hip: the layers must be resident (not streamed)\n");
        return Q48_EINVAL;
    }
    if (g_kv_quant.enabled || g_kv_quant.packed) {
        fprintf(stderr, "libintllm_hip: only the exact KV cache is supported\n");
        return Q48_EINVAL;
    }
    if ((rc = q48_check(q48_ctx_create(&g_q48.ctx, device), "q48_ctx_create")))
        return rc;
    rc = q48_check(q48_rope_init(g_q48.ctx, c->head_dim, c->max_seq_len, c->rope_theta),
                   "q48_rope_init");
    g_q48.model = m;
    g_q48.fused = 1;
    g_q48.embed_tokens = q48_upload(m->embed_tokens, vocab * dim, &rc);
    g_q48.final_norm = q48_upload(m->final_norm, dim, &rc);
    g_q48.lm_head = m->lm_head_tied ? g_q48.embed_tokens : q48_upload(m->lm_head, vocab * dim, &rc);
    g_q48.layers = (q48_layer_dev_t *)calloc((size_t)c->num_layers, sizeof(q48_layer_dev_t));
    if (!g_q48.layers && !rc)
        rc = Q48_ENOMEM;
    for (int l = 0; l < c->num_layers && !rc; ++l) {
        const layer_weights_t *w = &m->cached_layers[l];
        q48_layer_dev_t *d = &g_q48.layers[l];
        d->input_layernorm = q48_upload(w->input_layernorm, dim, &rc);
        d->qkv = q48_upload(NULL, (dim + 2 * kv_dim) * dim, &rc);
        if (rc)
            break;
        d->q_proj = d->qkv;
        d->k_proj = d->qkv + dim * dim;
        d->v_proj = d->k_proj + kv_dim * dim;
        q48_put(d->q_proj, w->q_proj, dim * dim, &rc);
        q48_put(d->k_proj, w->k_proj, kv_dim * dim, &rc);
        q48_put(d->v_proj, w->v_proj, kv_dim * dim, &rc);
        d->o_proj = q48_upload(w->o_proj, dim * dim, &rc);
        d->post_attn_norm = q48_upload(w->post_attn_norm, dim, &rc);
        d->gu = q48_upload(NULL, 2 * inter * dim, &rc);
        if (rc)
            break;
        d->gate_proj = d->gu;
        d->up_proj = d->gu + inter * dim;
        q48_put(d->gate_proj, w->gate_proj, inter * dim, &rc);
        q48_put(d->up_proj, w->up_proj, inter * dim, &rc);
        d->down_proj = q48_upload(w->down_proj, dim * inter, &rc);
    }
    const size_t kv_elems = (size_t)c->num_layers * c->max_seq_len * kv_dim;
    g_q48.key_cache = q48_upload(NULL, kv_elems, &rc);
    g_q48.value_cache = q48_upload(NULL, kv_elems, &rc);
    if (!rc)
        rc = q48_check(q48_zero(g_q48.ctx, g_q48.key_cache, kv_elems * 8), "q48_zero");
    if (!rc)
        rc = q48_check(q48_zero(g_q48.ctx, g_q48.value_cache, kv_elems * 8), "q48_zero");
    g_q48.hidden = q48_upload(NULL, dim, &rc);
    g_q48.normed = q48_upload(NULL, dim, &rc);
    g_q48.q = q48_upload(NULL, dim + 2 * kv_dim, &rc);   /* q | k | v */
    if (!rc) {
        g_q48.k = g_q48.q + dim;
        g_q48.v = g_q48.k + kv_dim;
    }
    g_q48.attn_out = q48_upload(NULL, dim, &rc);
    g_q48.o_out = q48_upload(NULL, dim, &rc);
    g_q48.gate = q48_upload(NULL, inter, &rc);
    g_q48.up = q48_upload(NULL, inter, &rc);
    g_q48.mlp_out = q48_upload(NULL, dim, &rc);
    g_q48.logits = q48_upload(NULL, vocab, &rc);
    g_q48.s_attn = q48_upload(NULL, (size_t)Q48_STATS_WORDS(c->hidden_dim), &rc);
    g_q48.s_ffn = q48_upload(NULL, (size_t)Q48_STATS_WORDS(c->hidden_dim), &rc);
    if (!rc)
        rc = q48_check(q48_sync(g_q48.ctx), "q48_sync");
    if (rc) {
        q48_detach();
        return rc;
    }
    g_q48_forward = (q48_any_fn)llama_forward_q48;
    return 0;
}

/* transformer_layer_forward (llama_int.c:1326-1569), exact-cache path, on
 * device buffers: the same op sequence, each op one library call. */
static int layer_forward_q48_ops(int64_t *hidden, const q48_layer_dev_t *w,
                                 const llama_config_t *cfg, int layer, int pos)
{
    q48_ctx *x = g_q48.ctx;
    const int dim = cfg->hidden_dim, hd = cfg->head_dim;
    const int kv_dim = cfg->num_kv_heads * hd, inter = cfg->intermediate_dim;
    int rc;
    /* 1-2. RMSNorm, q/k/v projections (:1384-1389) */
    if ((rc = q48_rmsnorm(x, g_q48.normed, hidden, w->input_layernorm, dim)) ||
        (rc = q48_gemv(x, g_q48.q, w->q_proj, g_q48.normed, dim, dim)) ||
        (rc = q48_gemv(x, g_q48.k, w->k_proj, g_q48.normed, kv_dim, dim)) ||
        (rc = q48_gemv(x, g_q48.v, w->v_proj, g_q48.normed, kv_dim, dim)))
        return rc;
    /* 3. RoPE on every q and k head (:1392-1395) */
    if ((rc = q48_rope(x, g_q48.q, cfg->num_heads, hd, pos)) ||
        (rc = q48_rope(x, g_q48.k, cfg->num_kv_heads, hd, pos)))
        return rc;
    /* 4. KV store at pos, scale, exact attention + softmax (:1414-1416,
     *    :1433, :1502-1529) */
    if ((rc = q48_attn_decode(x, g_q48.attn_out, g_q48.q, g_q48.key_cache, g_q48.value_cache,
                              g_q48.k, g_q48.v, layer, pos, cfg->num_heads, cfg->num_kv_heads,
                              hd, cfg->max_seq_len)))
        return rc;
    /* 5-6. output projection and residual (:1532-1535) */
    if ((rc = q48_gemv(x, g_q48.o_out, w->o_proj, g_q48.attn_out, dim, dim)) ||
        (rc = q48_add(x, hidden, g_q48.o_out, dim)))
        return rc;
    /* 7-9. RMSNorm, SwiGLU MLP, residual (:1544-1556) */
    if ((rc = q48_rmsnorm(x, g_q48.normed, hidden, w->post_attn_norm, dim)) ||
        (rc = q48_gemv(x, g_q48.gate, w->gate_proj, g_q48.normed, inter, dim)) ||
        (rc = q48_gemv(x, g_q48.up, w->up_proj, g_q48.normed, inter, dim)) ||
        (rc = q48_silu_mul(x, g_q48.gate, g_q48.gate, g_q48.up, inter)) ||
        (rc = q48_gemv(x, g_q48.mlp_out, w->down_proj, g_q48.gate, dim, inter)))
        return rc;
    return q48_add(x, hidden, g_q48.mlp_out, dim);
}

/* RoPE and the KV store in the q|k|v launch, attention from the cache:
 * positions below the split position, for the head sizes and cache lengths
 * the single-block attention keeps in LDS. */
static int q48_rope_in_gemv(const llama_config_t *cfg, int pos)
{
    const int hd = cfg->head_dim;
    return (hd == 32 || hd == 64 || hd == 128) && cfg->max_seq_len <= 4096 &&
           cfg->hidden_dim % 2 == 0 && cfg->hidden_dim <= 12288 && pos < q48_attn_split_min();
}

/* The same layer in five fused launches, each with the bits of the steps it
 * covers: rmsnorm + q|k|v (+ RoPE + KV store), attention, o + residual (+
 * the next norm's partial sums), rmsnorm + gate|up + SwiGLU, down +
 * residual (+ partial sums). */
static int layer_forward_q48_fused(int64_t *hidden, const q48_layer_dev_t *w,
                                   const llama_config_t *cfg, int layer, int pos)
{
    q48_ctx *x = g_q48.ctx;
    const int dim = cfg->hidden_dim, hd = cfg->head_dim, nh = cfg->num_heads;
    const int nkv = cfg->num_kv_heads, kv_dim = nkv * hd, inter = cfg->intermediate_dim;
    const int ms = cfg->max_seq_len;
    int rc;
    if (q48_rope_in_gemv(cfg, pos)) {
        if ((rc = q48_norm_gemv_rope_kv(x, g_q48.q, w->qkv, hidden, w->input_layernorm,
                                        g_q48.s_attn, g_q48.key_cache, g_q48.value_cache, layer,
                                        pos, nh, nkv, hd, ms, dim)) ||
            (rc = q48_attn_decode_cached(x, g_q48.attn_out, g_q48.q, g_q48.key_cache,
                                         g_q48.value_cache, layer, pos, nh, nkv, hd, ms, NULL,
                                         0)))
            return rc;
    } else if ((rc = q48_norm_gemv_stats(x, g_q48.q, w->qkv, hidden, w->input_layernorm,
                                         g_q48.s_attn, dim + 2 * kv_dim, dim)) ||
               (rc = q48_attn_decode_rope(x, g_q48.attn_out, g_q48.q, g_q48.key_cache,
                                          g_q48.value_cache, g_q48.k, g_q48.v, layer, pos, nh,
                                          nkv, hd, ms))) {
        return rc;
    }
    if ((rc = q48_gemv_residual_stats(x, hidden, w->o_proj, g_q48.attn_out, dim, dim,
                                      g_q48.s_ffn)) ||
        (rc = q48_norm_gemv_swiglu_stats(x, g_q48.gate, w->gu, hidden, w->post_attn_norm,
                                         g_q48.s_ffn, inter, dim)))
        return rc;
    return q48_gemv_residual_stats(x, hidden, w->down_proj, g_q48.gate, dim, inter, g_q48.s_attn);
}

/* Enqueue llama_forward (llama_int.c:2807-2886) up to the logits. */
static int q48_enqueue_forward(const llama_config_t *cfg, int token, int pos)
{
    q48_ctx *x = g_q48.ctx;
    const int dim = cfg->hidden_dim;
    int rc;
    if (g_q48.fused) {
        rc = q48_embed_stats(x, g_q48.hidden, g_q48.embed_tokens, token, dim, g_q48.s_attn);
        for (int layer = 0; layer < cfg->num_layers && !rc; layer++)
            rc = layer_forward_q48_fused(g_q48.hidden, &g_q48.layers[layer], cfg, layer, pos);
        if (!rc)
            rc = q48_norm_gemv_stats(x, g_q48.logits, g_q48.lm_head, g_q48.hidden,
                                     g_q48.final_norm, g_q48.s_attn, cfg->vocab_size, dim);
        return rc;
    }
    rc = q48_embed(x, g_q48.hidden, g_q48.embed_tokens, token, dim);
    for (int layer = 0; layer < cfg->num_layers && !rc; layer++)
        rc = layer_forward_q48_ops(g_q48.hidden, &g_q48.layers[layer], cfg, layer, pos);
    if (!rc)
        rc = q48_rmsnorm(x, g_q48.normed, g_q48.hidden, g_q48.final_norm, dim);
    if (!rc)
        rc = q48_gemv(x, g_q48.logits, g_q48.lm_head, g_q48.normed, cfg->vocab_size, dim);
    return rc;
}

/* The fused forward as a replayed graph: token and position go to the
 * device step state, and the captured kernels read them there.  One graph
 * per attention kernel class (below / from the split position); the first
 * forward of a class runs eagerly (the workspaces reach their size) and is
 * then captured. */
static int q48_forward_graph(const llama_config_t *cfg, int token, int pos)
{
    q48_ctx *x = g_q48.ctx;
    const int kind = pos >= q48_attn_split_min();
    const uint64_t stamp = q48_graph_stamp(x);
    int rc = q48_step_set(x, token, pos);
    if (rc)
        return rc;
    if (g_q48.graph[kind] && g_q48.graph_stamp[kind] == stamp)
        return q48_graph_replay(x, g_q48.graph[kind], 1);
    if (g_q48.graph[kind]) {   /* a context setting changed since the capture */
        q48_graph_destroy(x, g_q48.graph[kind]);
        g_q48.graph[kind] = NULL;
    }
    if ((rc = q48_step_mode(x, 1)))
        return rc;
    rc = q48_enqueue_forward(cfg, token, pos);
    if (!rc)
        rc = q48_sync(x);
    if (!rc)
        rc = q48_graph_capture(x);
    if (!rc) {
        int rc1 = q48_enqueue_forward(cfg, token, pos);
        q48_graph *g = NULL;
        rc = q48_graph_instantiate(x, &g);
        if (!rc && rc1) {
            q48_graph_destroy(x, g);
            g = NULL;
        }
        if (rc1)
            rc = rc1;
        if (!rc) {
            g_q48.graph[kind] = g;
            g_q48.graph_stamp[kind] = stamp;
        }
    }
    q48_step_mode(x, 0);
    return rc;
}

/* llama_forward (llama_int.c:2807-2886) on the device: the same range
 * checks and NULL on error, the logits returned in a malloc'd buffer that
 * the caller frees.  The device cache needs no reset between prompts
 * (kv_cache_reset, llama_int.c:1170-1183): a forward at pos writes row pos
 * before attention reads rows 0..pos. */
static fixed_t *llama_forward_q48(llama_model_t *m, int token, int pos)
{
    const llama_config_t *cfg = &m->cfg;
    if (g_profile.enabled)
        g_profile.forward_calls++;
    if (token < 0 || token >= cfg->vocab_size) {
        fprintf(stderr, "Token ID %d out of range [0, %d)\n", token, cfg->vocab_size);
        return NULL;
    }
    if (pos < 0 || pos >= cfg->max_seq_len) {
        fprintf(stderr, "Position %d out of range [0, %d)\n", pos, cfg->max_seq_len);
        return NULL;
    }
    if (m != g_q48.model) {
        fprintf(stderr, "libintllm_hip: llama_forward on a model that is not attached\n");
        return NULL;
    }
    int rc = g_q48.fused ? q48_forward_graph(cfg, token, pos)
                         : q48_enqueue_forward(cfg, token, pos);
    fixed_t *logits = NULL;
    if (!rc) {
        logits = (fixed_t *)checked_malloc((size_t)cfg->vocab_size * sizeof(fixed_t), "logits");
        rc = q48_memcpy_d2h(g_q48.ctx, logits, g_q48.logits,
                            (size_t)cfg->vocab_size * sizeof(fixed_t));
    }
    /* a split attention that gave up left wrong logits: a failed forward */
    if (!rc)
        rc = q48_attn_status(g_q48.ctx);
    if (rc) {
        q48_check(rc, "llama_forward_q48");
        free(logits);
        return NULL;
    }
    return logits;
}

static void q48_detach(void)
{
    g_q48_forward = NULL;
    if (!g_q48.ctx)
        return;
    for (int i = 0; i < 2; ++i)
        if (g_q48.graph[i])
            q48_graph_destroy(g_q48.ctx, g_q48.graph[i]);
    if (g_q48.layers) {
        for (int l = 0; l < g_q48.model->cfg.num_layers; ++l) {
            q48_layer_dev_t *d = &g_q48.layers[l];
            int64_t *p[] = {d->input_layernorm, d->qkv, d->o_proj, d->post_attn_norm, d->gu,
                            d->down_proj};
            for (size_t i = 0; i < sizeof p / sizeof p[0]; ++i)
                q48_free(g_q48.ctx, p[i]);
        }
        free(g_q48.layers);
    }
    int64_t *p[] = {g_q48.embed_tokens, g_q48.final_norm, g_q48.key_cache, g_q48.value_cache,
                    g_q48.hidden, g_q48.normed, g_q48.q, g_q48.attn_out, g_q48.o_out,
                    g_q48.gate, g_q48.up, g_q48.mlp_out, g_q48.logits, g_q48.s_attn,
                    g_q48.s_ffn};
    for (size_t i = 0; i < sizeof p / sizeof p[0]; ++i)
        q48_free(g_q48.ctx, p[i]);
    if (g_q48.lm_head != g_q48.embed_tokens)
        q48_free(g_q48.ctx, g_q48.lm_head);
    q48_ctx_destroy(g_q48.ctx);
    memset(&g_q48, 0, sizeof g_q48);
}

/* ======================================================================== */
/*  Exports for the tests (ctypes): the reference's own loaders and loops   */
/* ======================================================================== */

/* Every logits vector that llama_forward returns while recording is hashed
 * (FNV-1a 64 over its bytes, index order), through a wrapper around the
 * attached forward. */
static uint64_t *g_rec_hash;
static int g_rec_cap, g_rec_n;

static fixed_t *llama_forward_recorded(llama_model_t *m, int token, int pos)
{
    fixed_t *l = llama_forward_q48(m, token, pos);
    if (l && g_rec_n < g_rec_cap) {
        uint64_t h = 1469598103934665603ULL;
        for (int i = 0; i < m->cfg.vocab_size; ++i) {
            uint64_t u = (uint64_t)l[i];
            for (int b = 0; b < 8; ++b, u >>= 8)
                h = (h ^ (u & 0xff)) * 1099511628211ULL;
        }
        g_rec_hash[g_rec_n] = h;
    }
    if (l)
        g_rec_n++;
    return l;
}

/* mgw_load (llama_int.c:2344-2560), then rope_init, kv_cache_init and
 * llama_init_scratch as the reference's main does after loading. */
void *lq48_model_load_mgw(const char *path)
{
    llama_model_t *m = (llama_model_t *)calloc(1, sizeof *m);
    if (!m)
        return NULL;
    m->native_stream_fd = -1;
    if (mgw_load(m, path) != 0) {
        free(m);
        return NULL;
    }
    rope_init(&m->rope, &m->cfg);
    if (kv_cache_init(&m->kv, &m->cfg) != 0 || llama_init_scratch(m) != 0)
        return NULL;
    return m;
}

void lq48_model_free(void *mm)
{
    llama_model_t *m = (llama_model_t *)mm;
    if (m == g_q48.model)
        q48_detach();
    munmap(m->native_mmap, m->native_mmap_size);
    free(m->cached_layers);
    rope_free(&m->rope);
    kv_cache_free(&m->kv);
    free(m->scratch_buf);
    free(m);
}

/* The model's config, in llama_config_t's field order. */
void lq48_model_config(const void *mm, int out[9])
{
    const llama_config_t *c = &((const llama_model_t *)mm)->cfg;
    const int v[9] = {c->hidden_dim, c->num_heads, c->num_kv_heads, c->head_dim, c->num_layers,
                      c->intermediate_dim, c->vocab_size, c->max_seq_len, c->rope_theta};
    memcpy(out, v, sizeof v);
}

int lq48_attach(void *mm, int device) { return q48_attach((llama_model_t *)mm, device); }

/* The attached forward's route: fused launches replayed from a graph (1,
 * the default) or one library call per step of transformer_layer_forward
 * (0).  The same logits either way. */
int lq48_set_fused(int on)
{
    if (!g_q48.ctx)
        return Q48_ESTATE;
    g_q48.fused = on != 0;
    return 0;
}

/* The attached context's split-attention wait bound (q48_set_attn_wait):
 * 0 makes the one-launch split attention give up at once, so that the
 * failed-forward path can be tested. */
int lq48_set_attn_wait(int64_t ticks)
{
    return g_q48.ctx ? q48_set_attn_wait(g_q48.ctx, ticks) : Q48_ESTATE;
}

void lq48_detach(void) { q48_detach(); }

/* The reference's own generate() (llama_int.c:3067-3135; sp NULL: greedy)
 * with llama_forward routed to the device; hashes[] receives the FNV of
 * every logits vector in call order (*n_hash of them).  Returns generate's
 * value (prompt + generated tokens, or -1). */
int lq48_generate(void *mm, const int *prompt, int plen, int max_new, int *out,
                  uint64_t *hashes, int cap, int *n_hash)
{
    if (!g_q48_forward)
        return Q48_ESTATE;
    q48_any_fn saved = g_q48_forward;
    g_rec_hash = hashes;
    g_rec_cap = cap;
    g_rec_n = 0;
    g_q48_forward = (q48_any_fn)llama_forward_recorded;
    fflush(stdout);
    int total = generate((llama_model_t *)mm, prompt, plen, max_new, out, NULL);
    fflush(stdout);
    g_q48_forward = saved;
    *n_hash = g_rec_n;
    g_rec_hash = NULL;
    return total;
}

/* One routed llama_forward call: 0 and the logits, or -1 where the
 * reference's llama_forward returns NULL. */
int lq48_forward(void *mm, int token, int pos, int64_t *logits)
{
    llama_model_t *m = (llama_model_t *)mm;
    fixed_t *l = g_q48_forward ? llama_forward_q48(m, token, pos) : llama_forward_cpu(m, token, pos);
    if (!l)
        return -1;
    memcpy(logits, l, (size_t)m->cfg.vocab_size * sizeof(fixed_t));
    free(l);
    return 0;
}
