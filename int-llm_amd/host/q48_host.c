/*
 * q48_host.c — C host of the Q16.48 forward pass over libintllm_hip.
 *
 * Device memory layout (one weight slab, one activation slab):
 *   weights   embed [vocab][dim] | final_norm [dim] | lm_head [vocab][dim]
 *             then per layer: attn_norm | ffn_norm | Wqkv | Wo | Wgu | Wd
 *             where Wqkv = q_proj;k_proj;v_proj stacked ([dim+2kvd][dim])
 *             and Wgu = gate_proj;up_proj stacked ([2 ffn][dim]), so one
 *             GEMV produces q|k|v and one produces gate|up.  Stacking rows
 *             does not change any row's dot product, so the bits are the
 *             reference's (matmul_vec is row-independent).
 *   KV cache  [L][max_seq][n_kv][hd] int64, keys and values separately
 *             (kv_cache_t, llama_int.c:1078-1095).
 * Every region starts on a 256-byte boundary (16-byte vector loads).
 */
#include "q48_host.h"
#include "q48_synth.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#define LLAMA_EOS 2
#define FNV_OFF 1469598103934665603ULL

#define ALIGN_ELEMS 32   /* 256 bytes */
#define GRAPH_SLOTS 8

static size_t align_up(size_t n) { return (n + ALIGN_ELEMS - 1) / ALIGN_ELEMS * ALIGN_ELEMS; }

struct q48h_model {
    q48h_config c;
    q48_ctx *ctx;
    int tied;
    int64_t *w;                 /* device weight slab */
    size_t off_embed, off_norm, off_lm, off_layers, layer_elems;
    size_t lo_an, lo_fn, lo_qkv, lo_wo, lo_gu, lo_wd;
    int64_t *kc, *vc;           /* device KV cache */
    int64_t *act;               /* device activations */
    int64_t *hidden, *normed, *qkv, *attn, *o, *gu, *h_ffn, *mlp, *logits;
    int *d_tokens;              /* device: tokens of graph-replayed decode steps */
    /* sampling (sample_token, llama_int.c:2958-3039); greedy while
     * temperature < ONE / 100 */
    int64_t temperature, top_p;
    int top_k;
    uint64_t *d_rng;            /* device: xoroshiro128+ state */
    int64_t *r_attn, *r_ffn;    /* device: rmsnorm statistics of hidden for the next norm */
    int64_t *s_attn, *s_ffn;    /* device: the same as partial sums (Q48_STATS_WORDS) */
    int fused;                  /* 0: one op per kernel; 1: fused, norm statistics in
                                   every consumer block; 2: fused, statistics computed
                                   once by the producer (last block); 3 (default):
                                   fused, the producer leaves partial sums and every
                                   consumer block finishes them */
    int prefetch;               /* attention warms the cache with W_o (fused modes) */
    int rope_gemv;              /* mode 3 below the split position: RoPE and the KV
                                   store in the q|k|v projection, attention from the
                                   cache (q48_norm_gemv_rope_kv, q48_attn_decode_cached) */
    uint16_t *wb;               /* device: bfloat16 bits of the projection matrices and
                                   lm_head, at the element offsets of w (else NULL) */
    int bf16;                   /* mode 3 reads the matrices from wb */
    int batched_prefill;        /* generate's prompt through q48h_prefill (default) */
    int64_t *pf;                /* device: batched-prefill rows (grown on demand) */
    size_t pf_words;
    void *wp;                   /* device: digit planes of every layer's four projection
                                   matrices (q48_gemm_prepare), for the batched prefill */
    int wp_on;                  /* the prefill may prepare and use them (default) */
    int wp_ok;                  /* wp holds the planes of the current weights */
    int64_t *rec;               /* device: logits of recorded decode steps [rec_cap][vocab] */
    int rec_cap;
    int record;                 /* the decode step records its logits into rec */
    /* Captured decode steps, one per combination of the settings baked into
     * the kernels and their arguments.  A graph lives until the model is
     * freed (or, with every slot taken, until it is the least recently
     * used): switching settings between runs replays another slot rather
     * than destroying and re-capturing. */
    struct graph_slot {
        q48_graph *g;
        unsigned long long used;   /* 0: empty, else the run count at last use */
        struct graph_key {
            int kind, record, rec_cap, bf16, fused, rope_gemv, prefetch, top_k;
            int64_t temperature, top_p;
            const void *rec, *wb;
            uint64_t stamp;
        } k;
    } gslot[GRAPH_SLOTS];
    unsigned long long runs;
    q48_graph *g_run;           /* the graph of the run in progress */
};

/* ---------------------------------------------------------------------- */
/* config.json (load_config_json, llama_int.c:819-903)                     */
/* ---------------------------------------------------------------------- */

static int json_int(const char *json, const char *key, int dflt)
{
    char pat[256];
    snprintf(pat, sizeof pat, "\"%s\"", key);
    const char *p = strstr(json, pat);
    if (!p)
        return dflt;
    p += strlen(pat);
    while (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r' || *p == ':')
        p++;
    if (*p == 'n')
        return dflt;   /* null */
    return (int)strtol(p, NULL, 10);
}

int q48h_config_from_json_text(const char *json, q48h_config *c)
{
    if (!json || !c)
        return -2;
    c->dim = json_int(json, "hidden_size", -1);
    c->n_heads = json_int(json, "num_attention_heads", -1);
    c->n_kv_heads = json_int(json, "num_key_value_heads", c->n_heads);
    c->n_layers = json_int(json, "num_hidden_layers", -1);
    c->ffn = json_int(json, "intermediate_size", -1);
    c->vocab = json_int(json, "vocab_size", -1);
    c->max_seq = json_int(json, "max_position_embeddings", 2048);
    c->rope_theta = json_int(json, "rope_theta", 10000);
    if (c->dim <= 0 || c->n_heads <= 0 || c->n_layers <= 0 || c->ffn <= 0 || c->vocab <= 0)
        return -2;
    if (c->dim % c->n_heads != 0)
        return -2;
    c->head_dim = c->dim / c->n_heads;
    if (c->n_kv_heads <= 0 || c->n_heads % c->n_kv_heads != 0)
        return -2;
    return 0;
}

int q48h_config_from_json(const char *model_dir, q48h_config *c)
{
    char path[512];
    snprintf(path, sizeof path, "%s/config.json", model_dir);
    FILE *f = fopen(path, "r");
    if (!f)
        return -1;
    fseek(f, 0, SEEK_END);
    long len = ftell(f);
    if (len <= 0 || len > 1024 * 1024) {
        fclose(f);
        return -1;
    }
    fseek(f, 0, SEEK_SET);
    char *buf = (char *)malloc((size_t)len + 1);
    if (!buf) {
        fclose(f);
        return -1;
    }
    size_t n = fread(buf, 1, (size_t)len, f);
    fclose(f);
    buf[n] = 0;
    int rc = q48h_config_from_json_text(buf, c);
    free(buf);
    return rc;
}

int q48h_config_check(const q48h_config *c)
{
    if (!c || c->dim <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->n_layers <= 0 ||
        c->ffn <= 0 || c->vocab <= 0 || c->max_seq <= 0 || c->rope_theta <= 0)
        return Q48_EINVAL;
    if (c->n_heads % c->n_kv_heads || c->head_dim * c->n_heads != c->dim)
        return Q48_EINVAL;
    if (c->head_dim % 2 || c->head_dim > 256 || 256 % c->head_dim)
        return Q48_EINVAL;
    if (c->max_seq > 32767 || c->rope_theta > 32767)
        return Q48_EINVAL;
    return Q48_OK;
}

/* ---------------------------------------------------------------------- */
/* model                                                                   */
/* ---------------------------------------------------------------------- */

static void layout(q48h_model *m)
{
    const q48h_config *c = &m->c;
    size_t dim = (size_t)c->dim, kvd = (size_t)c->n_kv_heads * c->head_dim, ffn = (size_t)c->ffn;
    size_t o = 0;
    m->off_embed = o;
    o += align_up((size_t)c->vocab * dim);
    m->off_norm = o;
    o += align_up(dim);
    m->off_lm = m->tied ? m->off_embed : o;
    if (!m->tied)
        o += align_up((size_t)c->vocab * dim);
    m->off_layers = o;
    size_t l = 0;
    m->lo_an = l; l += align_up(dim);
    m->lo_fn = l; l += align_up(dim);
    m->lo_qkv = l; l += align_up((dim + 2 * kvd) * dim);
    m->lo_wo = l; l += align_up(dim * dim);
    m->lo_gu = l; l += align_up(2 * ffn * dim);
    m->lo_wd = l; l += align_up(dim * ffn);
    m->layer_elems = l;
}

static size_t weight_elems(const q48h_model *m)
{
    return m->off_layers + (size_t)m->c.n_layers * m->layer_elems;
}

static int model_alloc(q48h_model **out, q48_ctx *ctx, const q48h_config *cfg, int tied)
{
    int rc = q48h_config_check(cfg);
    if (rc)
        return rc;
    q48h_model *m = (q48h_model *)calloc(1, sizeof *m);
    if (!m)
        return Q48_ENOMEM;
    m->c = *cfg;
    m->ctx = ctx;
    m->tied = tied;
    layout(m);
    const q48h_config *c = &m->c;
    size_t dim = (size_t)c->dim, kvd = (size_t)c->n_kv_heads * c->head_dim, ffn = (size_t)c->ffn;
    size_t kvn = (size_t)c->n_layers * c->max_seq * kvd;
    size_t an = 0;
    size_t a_hidden = an; an += align_up(dim);
    size_t a_normed = an; an += align_up(dim);
    size_t a_qkv = an; an += align_up(dim + 2 * kvd);
    size_t a_attn = an; an += align_up(dim);
    size_t a_o = an; an += align_up(dim);
    size_t a_gu = an; an += align_up(2 * ffn);
    size_t a_ffn = an; an += align_up(ffn);
    size_t a_mlp = an; an += align_up(dim);
    size_t a_log = an; an += align_up((size_t)c->vocab);
    size_t a_r = an; an += ALIGN_ELEMS;
    size_t sw = (size_t)Q48_STATS_WORDS(c->dim);
    size_t a_sa = an; an += align_up(sw);
    size_t a_sf = an; an += align_up(sw);

    m->fused = 3;
    m->prefetch = 1;
    m->rope_gemv = 1;
    m->batched_prefill = 1;
    m->wp_on = 1;
    if ((rc = q48_malloc(ctx, (void **)&m->w, weight_elems(m) * 8)) ||
        (rc = q48_malloc(ctx, (void **)&m->kc, kvn * 8)) ||
        (rc = q48_malloc(ctx, (void **)&m->vc, kvn * 8)) ||
        (rc = q48_malloc(ctx, (void **)&m->act, an * 8)) ||
        (rc = q48_malloc(ctx, (void **)&m->d_tokens, (size_t)c->max_seq * sizeof(int)))) {
        q48h_model_free(m);
        return rc;
    }
    m->hidden = m->act + a_hidden;
    m->normed = m->act + a_normed;
    m->qkv = m->act + a_qkv;
    m->attn = m->act + a_attn;
    m->o = m->act + a_o;
    m->gu = m->act + a_gu;
    m->h_ffn = m->act + a_ffn;
    m->mlp = m->act + a_mlp;
    m->logits = m->act + a_log;
    m->r_attn = m->act + a_r;
    m->r_ffn = m->act + a_r + 1;
    m->s_attn = m->act + a_sa;
    m->s_ffn = m->act + a_sf;
    if ((rc = q48_zero(ctx, m->w, weight_elems(m) * 8)) ||
        (rc = q48_zero(ctx, m->kc, kvn * 8)) || (rc = q48_zero(ctx, m->vc, kvn * 8)) ||
        (rc = q48_zero(ctx, m->act, an * 8)) ||
        (rc = q48_rope_init(ctx, c->head_dim, c->max_seq, c->rope_theta)) ||
        (rc = q48_sync(ctx))) {
        q48h_model_free(m);
        return rc;
    }
    *out = m;
    return Q48_OK;
}

int q48h_model_create(q48h_model **out, q48_ctx *ctx, const q48h_config *cfg)
{
    if (!out || !ctx || !cfg)
        return Q48_EINVAL;
    *out = NULL;
    return model_alloc(out, ctx, cfg, 0);
}

static void graphs_free(q48h_model *m)
{
    for (int i = 0; i < GRAPH_SLOTS; ++i)
        if (m->gslot[i].used) {
            q48_graph_destroy(m->ctx, m->gslot[i].g);
            m->gslot[i].g = NULL;
            m->gslot[i].used = 0;
        }
    m->g_run = NULL;
}

/* Forget the bfloat16 copy of the weights (they are about to change). */
static void drop_bf16(q48h_model *m)
{
    if (m->wb) {
        q48_free(m->ctx, m->wb);
        m->wb = NULL;
    }
    m->bf16 = 0;
}

/* Byte offsets of a layer's prepared q|k|v, o, gate|up and down planes
 * within the layer's stride of m->wp; returns the stride (0 on error). */
static size_t planes_layout(const q48h_model *m, size_t off[4])
{
    const q48h_config *c = &m->c;
    const int dim = c->dim, kvd = c->n_kv_heads * c->head_dim, ffn = c->ffn;
    const int shape[4][2] = {{dim + 2 * kvd, dim}, {dim, dim}, {2 * ffn, dim}, {dim, ffn}};
    size_t s = 0;
    for (int i = 0; i < 4; ++i) {
        size_t b = 0;
        if (q48_gemm_planes_bytes(shape[i][0], shape[i][1], &b) != Q48_OK)
            return 0;
        off[i] = s;
        s += (b + 255) & ~(size_t)255;
    }
    return s;
}

/* The prefill's prepared planes, made once per set of weights.  Without
 * device memory for them the prefill goes on splitting W in each call. */
static int prepare_planes(q48h_model *m)
{
    if (!m->wp_on || m->wp_ok)
        return Q48_OK;
    const q48h_config *c = &m->c;
    const int dim = c->dim, kvd = c->n_kv_heads * c->head_dim, ffn = c->ffn;
    size_t off[4];
    const size_t stride = planes_layout(m, off);
    if (!stride)
        return Q48_EINVAL;
    if (!m->wp) {
        int rc = q48_malloc(m->ctx, &m->wp, stride * (size_t)c->n_layers);
        if (rc == Q48_ENOMEM) {
            m->wp = NULL;
            m->wp_on = 0;
            return Q48_OK;
        }
        if (rc)
            return rc;
    }
    for (int l = 0; l < c->n_layers; ++l) {
        const int64_t *b = m->w + m->off_layers + (size_t)l * m->layer_elems;
        char *p = (char *)m->wp + (size_t)l * stride;
        int rc;
        if ((rc = q48_gemm_prepare(m->ctx, p + off[0], b + m->lo_qkv, dim + 2 * kvd, dim)) ||
            (rc = q48_gemm_prepare(m->ctx, p + off[1], b + m->lo_wo, dim, dim)) ||
            (rc = q48_gemm_prepare(m->ctx, p + off[2], b + m->lo_gu, 2 * ffn, dim)) ||
            (rc = q48_gemm_prepare(m->ctx, p + off[3], b + m->lo_wd, dim, ffn)))
            return rc;
    }
    m->wp_ok = 1;
    return Q48_OK;
}

void q48h_model_set_gemm_planes(q48h_model *m, int on)
{
    if (!m)
        return;
    m->wp_on = on != 0;
    if (!m->wp_on && m->wp) {
        (void)q48_sync(m->ctx);   /* earlier prefill kernels may still read them */
        q48_free(m->ctx, m->wp);
        m->wp = NULL;
        m->wp_ok = 0;
    }
}

/* A GEMM of the prefill: through W's prepared planes when there are some. */
static int prefill_gemm(q48_ctx *x, int64_t *Y, const int64_t *W, const void *Wp,
                        const int64_t *X, int T, int N, int K)
{
    return Wp ? q48_gemm_prepared(x, Y, W, Wp, X, T, N, K) : q48_gemm(x, Y, W, X, T, N, K);
}

int q48h_model_set_bf16(q48h_model *m, int on)
{
    if (!m)
        return Q48_EINVAL;
    on = on != 0;
    if (on && !m->wb) {
        const q48h_config *c = &m->c;
        int kvd = c->n_kv_heads * c->head_dim;
        if (c->dim % 512 || c->ffn % 512)
            return Q48_EINVAL;   /* the bfloat16 GEMVs take K = 512 j */
        int mrc = q48_malloc(m->ctx, (void **)&m->wb, weight_elems(m) * 2);
        if (mrc)
            return mrc;
        /* the four projections of every layer and lm_head; each must be
         * bfloat16 values exactly, else the weights stay int64 only */
        struct { size_t off, n; } t[4];
        int inexact = 0, rc = Q48_OK;
        for (int l = 0; l < c->n_layers && !rc && !inexact; ++l) {
            size_t b = m->off_layers + (size_t)l * m->layer_elems;
            t[0].off = b + m->lo_qkv; t[0].n = (size_t)(c->dim + 2 * kvd) * c->dim;
            t[1].off = b + m->lo_wo;  t[1].n = (size_t)c->dim * c->dim;
            t[2].off = b + m->lo_gu;  t[2].n = (size_t)2 * c->ffn * c->dim;
            t[3].off = b + m->lo_wd;  t[3].n = (size_t)c->dim * c->ffn;
            for (int i = 0; i < 4 && !rc && !inexact; ++i)
                rc = q48_bf16_pack(m->ctx, m->wb + t[i].off, m->w + t[i].off, t[i].n,
                                   &inexact);
        }
        if (!rc && !inexact)
            rc = q48_bf16_pack(m->ctx, m->wb + m->off_lm, m->w + m->off_lm,
                               (size_t)c->vocab * c->dim, &inexact);
        if (rc || inexact) {
            q48_free(m->ctx, m->wb);
            m->wb = NULL;
            return rc ? rc : Q48_EINVAL;
        }
    }
    m->bf16 = on;
    return Q48_OK;
}

void q48h_model_free(q48h_model *m)
{
    if (!m)
        return;
    graphs_free(m);   /* before the buffers their kernels read */
    q48_free(m->ctx, m->wb);
    q48_free(m->ctx, m->w);
    q48_free(m->ctx, m->kc);
    q48_free(m->ctx, m->vc);
    q48_free(m->ctx, m->act);
    q48_free(m->ctx, m->d_tokens);
    q48_free(m->ctx, m->d_rng);
    q48_free(m->ctx, m->pf);
    q48_free(m->ctx, m->wp);
    q48_free(m->ctx, m->rec);
    free(m);
}

int q48h_model_set_sampling(q48h_model *m, int64_t temperature, int top_k, int64_t top_p,
                            uint64_t seed)
{
    if (!m)
        return Q48_EINVAL;
    int rc;
    if (!m->d_rng && (rc = q48_malloc(m->ctx, (void **)&m->d_rng, 2 * sizeof(uint64_t))))
        return rc;
    uint64_t st[2];
    q48_rng_seed(seed, st);
    if ((rc = q48_memcpy_h2d(m->ctx, m->d_rng, st, sizeof st)))
        return rc;
    if ((rc = q48_sync(m->ctx)))
        return rc;
    m->temperature = temperature;
    m->top_k = top_k;
    m->top_p = top_p;
    return Q48_OK;
}

/* The next token from the logits on the device: sample_token with the
 * model's parameters (argmax below a temperature of 0.01). */
static int select_token(q48h_model *m, int *next)
{
    if (m->temperature >= Q48_ONE / 100)
        return q48_sample(m->ctx, m->logits, m->c.vocab, m->temperature, m->top_k, m->top_p,
                          m->d_rng, next);
    return q48_argmax(m->ctx, m->logits, m->c.vocab, next);
}

static int select_token_step(q48h_model *m)
{
    if (m->temperature >= Q48_ONE / 100)
        return q48_sample_step(m->ctx, m->logits, m->c.vocab, m->temperature, m->top_k,
                               m->top_p, m->d_rng, m->d_tokens, m->c.max_seq);
    return q48_argmax_step(m->ctx, m->logits, m->c.vocab, m->d_tokens, m->c.max_seq);
}

/* The step's logits recorded (when the model records) and its token chosen,
 * on the device; greedy steps do both in one launch. */
static int record_and_select_step(q48h_model *m)
{
    if (m->record && m->temperature < Q48_ONE / 100)
        return q48_argmax_record_step(m->ctx, m->logits, m->c.vocab, m->d_tokens, m->c.max_seq,
                                      m->rec, m->rec_cap);
    if (m->record) {
        int rc = q48_record_step(m->ctx, m->logits, m->c.vocab, m->rec, m->rec_cap);
        if (rc)
            return rc;
    }
    return select_token_step(m);
}

void q48h_model_set_fused(q48h_model *m, int fused)
{
    if (fused < 0 || fused > 3)
        fused = 3;
    if (m)
        m->fused = fused;
}

/* How a graph-replayed decode step at pos runs: 0 the fused launches with
 * single-block attention, 1 the same with split attention (from
 * q48_attn_split_min). */
static int step_kind(q48h_model *m, int pos)
{
    (void)m;
    return pos >= q48_attn_split_min() ? 1 : 0;
}

void q48h_model_set_rope_gemv(q48h_model *m, int on)
{
    if (m)
        m->rope_gemv = on != 0;
}

void q48h_model_set_prefetch(q48h_model *m, int on)
{
    if (m)
        m->prefetch = on != 0;
}

const q48h_config *q48h_model_config(const q48h_model *m) { return &m->c; }
q48_ctx *q48h_model_ctx(q48h_model *m) { return m->ctx; }
int64_t *q48h_kv_keys(q48h_model *m) { return m->kc; }
int64_t *q48h_kv_values(q48h_model *m) { return m->vc; }

/* Device address and element count of the tensor `name`. */
static int tensor_slot(q48h_model *m, const char *name, int64_t **dst, int64_t *n)
{
    const q48h_config *c = &m->c;
    int64_t dim = c->dim, kvd = (int64_t)c->n_kv_heads * c->head_dim, ffn = c->ffn;
    if (!strcmp(name, "model.embed_tokens.weight")) {
        *dst = m->w + m->off_embed;
        *n = (int64_t)c->vocab * dim;
        return 0;
    }
    if (!strcmp(name, "model.norm.weight")) {
        *dst = m->w + m->off_norm;
        *n = dim;
        return 0;
    }
    if (!strcmp(name, "lm_head.weight")) {
        if (m->tied)
            return -1;
        *dst = m->w + m->off_lm;
        *n = (int64_t)c->vocab * dim;
        return 0;
    }
    int l = -1;
    char rest[128];
    if (sscanf(name, "model.layers.%d.%127s", &l, rest) != 2 || l < 0 || l >= c->n_layers)
        return -1;
    int64_t *b = m->w + m->off_layers + (size_t)l * m->layer_elems;
    struct { const char *s; size_t off; int64_t n; } t[] = {
        {"input_layernorm.weight", m->lo_an, dim},
        {"post_attention_layernorm.weight", m->lo_fn, dim},
        {"self_attn.q_proj.weight", m->lo_qkv, dim * dim},
        {"self_attn.k_proj.weight", m->lo_qkv + (size_t)(dim * dim), kvd * dim},
        {"self_attn.v_proj.weight", m->lo_qkv + (size_t)(dim * dim + kvd * dim), kvd * dim},
        {"self_attn.o_proj.weight", m->lo_wo, dim * dim},
        {"mlp.gate_proj.weight", m->lo_gu, ffn * dim},
        {"mlp.up_proj.weight", m->lo_gu + (size_t)(ffn * dim), ffn * dim},
        {"mlp.down_proj.weight", m->lo_wd, dim * ffn},
    };
    for (size_t i = 0; i < sizeof t / sizeof t[0]; ++i)
        if (!strcmp(rest, t[i].s)) {
            *dst = b + t[i].off;
            *n = t[i].n;
            return 0;
        }
    return -1;
}

int q48h_upload(q48h_model *m, const char *name, const int64_t *host, int64_t n)
{
    if (!m || !name || !host)
        return Q48_EINVAL;
    int64_t *dst;
    int64_t want;
    if (tensor_slot(m, name, &dst, &want) || n != want)
        return Q48_EINVAL;
    drop_bf16(m);   /* the bfloat16 copy would be stale */
    m->wp_ok = 0;   /* and so would the prefill's planes */
    return q48_memcpy_h2d(m->ctx, dst, host, (size_t)n * 8);
}

/* Names and shapes of every tensor, in mgw_export's order
 * (llama_int.c:1736-1760). */
typedef struct {
    char name[64];
    int ndims;
    int64_t rows, cols;
} tdesc;

static int tensor_list(const q48h_config *c, int tied, tdesc *t)
{
    int n = 0, kvd = c->n_kv_heads * c->head_dim;
#define ADD(nm, nd, r, k) do { snprintf(t[n].name, 64, "%s", nm); t[n].ndims = nd; \
        t[n].rows = r; t[n].cols = k; n++; } while (0)
    ADD("model.embed_tokens.weight", 2, c->vocab, c->dim);
    ADD("model.norm.weight", 1, 1, c->dim);
    if (!tied)
        ADD("lm_head.weight", 2, c->vocab, c->dim);
    for (int l = 0; l < c->n_layers; ++l) {
        char b[64];
#define ADDL(sfx, nd, r, k) do { snprintf(b, sizeof b, "model.layers.%d." sfx, l); ADD(b, nd, r, k); } while (0)
        ADDL("input_layernorm.weight", 1, 1, c->dim);
        ADDL("self_attn.q_proj.weight", 2, c->dim, c->dim);
        ADDL("self_attn.k_proj.weight", 2, kvd, c->dim);
        ADDL("self_attn.v_proj.weight", 2, kvd, c->dim);
        ADDL("self_attn.o_proj.weight", 2, c->dim, c->dim);
        ADDL("post_attention_layernorm.weight", 1, 1, c->dim);
        ADDL("mlp.gate_proj.weight", 2, c->ffn, c->dim);
        ADDL("mlp.up_proj.weight", 2, c->ffn, c->dim);
        ADDL("mlp.down_proj.weight", 2, c->dim, c->ffn);
#undef ADDL
    }
#undef ADD
    return n;
}

int q48h_model_synth(q48h_model *m, uint64_t seed, int threads)
{
    if (!m)
        return Q48_EINVAL;
    const q48h_config *c = &m->c;
    int nt = 3 + 9 * c->n_layers;
    tdesc *t = (tdesc *)malloc(sizeof(tdesc) * (size_t)nt);
    if (!t)
        return Q48_ENOMEM;
    nt = tensor_list(c, m->tied, t);
    int64_t maxn = 0;
    for (int i = 0; i < nt; ++i)
        if (t[i].rows * t[i].cols > maxn)
            maxn = t[i].rows * t[i].cols;
    int64_t *buf = (int64_t *)malloc((size_t)maxn * 8);
    int rc = buf ? Q48_OK : Q48_ENOMEM;
    for (int i = 0; i < nt && rc == Q48_OK; ++i) {
        q48s_fill_named(buf, t[i].rows, t[i].cols, seed, t[i].name, Q48_SIGMA_W, 1, threads);
        rc = q48h_upload(m, t[i].name, buf, t[i].rows * t[i].cols);
    }
    free(buf);
    free(t);
    return rc;
}

/* ---------------------------------------------------------------------- */
/* .mgw (llama_int.c:385-454, 1718-1904, 2344-2560)                        */
/* ---------------------------------------------------------------------- */

#define MGW_HEADER_SIZE 64
#define MGW_CONFIG_SIZE 64
#define MGW_ENTRY_SIZE 96
#define MGW_VERSION 1
#define MGW_ENDIAN 0x01020304u

static void put32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }
static void put64(uint8_t *p, uint64_t v) { memcpy(p, &v, 8); }
static uint32_t get32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t get64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }

int q48h_mgw_write_synth(const char *path, const q48h_config *c, uint64_t seed, int threads)
{
    if (!path || !c)
        return Q48_EINVAL;
    int nt = 3 + 9 * c->n_layers;
    tdesc *t = (tdesc *)malloc(sizeof(tdesc) * (size_t)nt);
    if (!t)
        return Q48_ENOMEM;
    nt = tensor_list(c, 0, t);
    uint64_t index_off = MGW_HEADER_SIZE + MGW_CONFIG_SIZE;
    uint64_t data_off = (index_off + (uint64_t)nt * MGW_ENTRY_SIZE + 7) & ~7ull;
    size_t head_n = (size_t)data_off;
    uint8_t *head = (uint8_t *)calloc(1, head_n);
    if (!head) {
        free(t);
        return Q48_ENOMEM;
    }
    memcpy(head, "MGW\0", 4);
    put32(head + 4, MGW_VERSION);
    put32(head + 8, MGW_ENDIAN);
    put32(head + 12, (uint32_t)nt);
    put64(head + 16, index_off);
    put64(head + 24, data_off);
    int32_t cfgv[10] = {c->dim, c->n_heads, c->n_kv_heads, c->head_dim, c->n_layers,
                        c->ffn, c->vocab, c->max_seq, c->rope_theta, 0};
    memcpy(head + MGW_HEADER_SIZE, cfgv, sizeof cfgv);
    uint64_t cur = data_off;
    for (int i = 0; i < nt; ++i) {
        uint8_t *e = head + index_off + (size_t)i * MGW_ENTRY_SIZE;
        uint64_t ne = (uint64_t)(t[i].rows * t[i].cols);
        strncpy((char *)e, t[i].name, 63);
        put64(e + 64, ne);
        put64(e + 72, cur);
        put32(e + 80, (uint32_t)t[i].ndims);
        put32(e + 84, (uint32_t)(t[i].ndims == 2 ? t[i].rows : t[i].cols));
        put32(e + 88, (uint32_t)(t[i].ndims == 2 ? t[i].cols : 0));
        cur += ne * 8;
    }
    FILE *f = fopen(path, "wb");
    int rc = f ? Q48_OK : Q48_EINVAL;
    if (f && fwrite(head, 1, head_n, f) != head_n)
        rc = Q48_EINVAL;
    int64_t maxn = 0;
    for (int i = 0; i < nt; ++i)
        if (t[i].rows * t[i].cols > maxn)
            maxn = t[i].rows * t[i].cols;
    int64_t *buf = rc == Q48_OK ? (int64_t *)malloc((size_t)maxn * 8) : NULL;
    if (rc == Q48_OK && !buf)
        rc = Q48_ENOMEM;
    for (int i = 0; i < nt && rc == Q48_OK; ++i) {
        size_t ne = (size_t)(t[i].rows * t[i].cols);
        q48s_fill_named(buf, t[i].rows, t[i].cols, seed, t[i].name, Q48_SIGMA_W, 1, threads);
        if (fwrite(buf, 8, ne, f) != ne)
            rc = Q48_EINVAL;
    }
    free(buf);
    if (f && fclose(f) != 0)
        rc = Q48_EINVAL;
    free(head);
    free(t);
    return rc;
}

int q48h_model_load_mgw(q48h_model **out, q48_ctx *ctx, const char *path, int max_seq)
{
    if (!out || !ctx || !path)
        return Q48_EINVAL;
    *out = NULL;
    int fd = open(path, O_RDONLY);
    if (fd < 0)
        return Q48_EINVAL;
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < MGW_HEADER_SIZE + MGW_CONFIG_SIZE) {
        close(fd);
        return Q48_EINVAL;
    }
    size_t fsz = (size_t)sb.st_size;
    const uint8_t *base = (const uint8_t *)mmap(NULL, fsz, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == (const uint8_t *)MAP_FAILED)
        return Q48_EINVAL;
    int rc = Q48_EINVAL;
    q48h_model *m = NULL;
    if (memcmp(base, "MGW\0", 4) || get32(base + 4) != MGW_VERSION || get32(base + 8) != MGW_ENDIAN)
        goto done;
    uint32_t nt = get32(base + 12);
    uint64_t ioff = get64(base + 16);
    if (ioff > fsz || (uint64_t)nt * MGW_ENTRY_SIZE > fsz - ioff)
        goto done;
    int32_t cv[10];
    memcpy(cv, base + MGW_HEADER_SIZE, sizeof cv);
    q48h_config c = {cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7], cv[8]};
    int tied = cv[9] != 0;
    if (c.dim <= 0 || c.n_heads <= 0 || c.n_layers <= 0 || c.vocab <= 0)
        goto done;
    if (max_seq > 0)
        c.max_seq = max_seq;
    if ((rc = model_alloc(&m, ctx, &c, tied)) != Q48_OK)
        goto done;
    rc = Q48_EINVAL;
    int got_embed = 0, got_norm = 0, got_lm = 0;
    int *got_layer = (int *)calloc((size_t)c.n_layers, sizeof(int));
    if (!got_layer) {
        rc = Q48_ENOMEM;
        goto done;
    }
    for (uint32_t i = 0; i < nt; ++i) {
        const uint8_t *e = base + ioff + (uint64_t)i * MGW_ENTRY_SIZE;
        char name[64];
        memcpy(name, e, 63);
        name[63] = 0;
        uint64_t ne = get64(e + 64), doff = get64(e + 72);
        if (ne > UINT64_MAX / 8 || doff > fsz || ne * 8 > fsz - doff || doff % 8) {
            free(got_layer);
            goto done;
        }
        int64_t *dst;
        int64_t want;
        if (tensor_slot(m, name, &dst, &want) != 0)
            continue;   /* the reference warns and skips unknown tensors */
        if ((int64_t)ne != want) {
            free(got_layer);
            goto done;
        }
        if (q48_memcpy_h2d(ctx, dst, base + doff, ne * 8) != Q48_OK) {
            rc = Q48_EHIP;
            free(got_layer);
            goto done;
        }
        int l;
        char rest[128];
        if (!strcmp(name, "model.embed_tokens.weight"))
            got_embed = 1;
        else if (!strcmp(name, "model.norm.weight"))
            got_norm = 1;
        else if (!strcmp(name, "lm_head.weight"))
            got_lm = 1;
        else if (sscanf(name, "model.layers.%d.%127s", &l, rest) == 2)
            got_layer[l]++;
    }
    int complete = got_embed && got_norm && (tied || got_lm);
    for (int l = 0; l < c.n_layers; ++l)
        complete = complete && got_layer[l] == 9;
    free(got_layer);
    if (!complete)
        goto done;
    rc = Q48_OK;
done:
    munmap((void *)base, fsz);
    if (rc != Q48_OK) {
        q48h_model_free(m);
        return rc;
    }
    *out = m;
    return Q48_OK;
}

/* ---------------------------------------------------------------------- */
/* KV cache                                                                */
/* ---------------------------------------------------------------------- */

int q48h_kv_reset(q48h_model *m)
{
    if (!m)
        return Q48_EINVAL;
    size_t n = (size_t)m->c.n_layers * m->c.max_seq * m->c.n_kv_heads * m->c.head_dim * 8;
    int rc = q48_zero(m->ctx, m->kc, n);
    return rc ? rc : q48_zero(m->ctx, m->vc, n);
}

int q48h_kv_fill_synth(q48h_model *m, uint64_t seed, int npos, int threads)
{
    if (!m || npos < 0 || npos > m->c.max_seq)
        return Q48_EINVAL;
    if (npos == 0)
        return Q48_OK;
    int kvd = m->c.n_kv_heads * m->c.head_dim;
    int64_t *buf = (int64_t *)malloc((size_t)npos * kvd * 8);
    if (!buf)
        return Q48_ENOMEM;
    int rc = Q48_OK;
    char nm[64];
    for (int l = 0; l < m->c.n_layers && rc == Q48_OK; ++l) {
        size_t off = (size_t)l * m->c.max_seq * kvd;
        snprintf(nm, sizeof nm, "kv.key.%d", l);
        q48s_fill_named(buf, npos, kvd, seed, nm, Q48_SIGMA_ACT, 1, threads);
        rc = q48_memcpy_h2d(m->ctx, m->kc + off, buf, (size_t)npos * kvd * 8);
        if (rc)
            break;
        snprintf(nm, sizeof nm, "kv.value.%d", l);
        q48s_fill_named(buf, npos, kvd, seed, nm, Q48_SIGMA_ACT, 1, threads);
        rc = q48_memcpy_h2d(m->ctx, m->vc + off, buf, (size_t)npos * kvd * 8);
    }
    free(buf);
    return rc;
}

/* ---------------------------------------------------------------------- */
/* forward / generate                                                      */
/* ---------------------------------------------------------------------- */

#define TRY(x) do { int rc_ = (x); if (rc_) return rc_; } while (0)

/* Whether mode 3 runs RoPE and the KV store in the q|k|v projection and
 * attention from the cache (single-block attention: below the split
 * position, head_dim 32, 64 or 128, at most 4096 cached positions). */
static int rope_in_gemv(const q48h_model *m)
{
    const q48h_config *c = &m->c;
    return m->rope_gemv && m->fused == 3 &&
           (c->head_dim == 32 || c->head_dim == 64 || c->head_dim == 128) &&
           c->max_seq <= 4096 && c->dim % 2 == 0 && c->dim <= 12288;
}

/* transformer_layer_forward, llama_int.c:1326-1569 (exact-cache path),
 * fused: 5 launches.  rmsnorm+q|k|v, RoPE+KV store+attention, o+residual,
 * rmsnorm+gate|up+SwiGLU, down+residual; below the split position (mode 3)
 * rmsnorm+q|k|v+RoPE+KV store, attention from the cache, and the rest. */
static int layer_forward_fused(q48h_model *m, int l, int pos)
{
    const q48h_config *c = &m->c;
    q48_ctx *x = m->ctx;
    int dim = c->dim, hd = c->head_dim, kvd = c->n_kv_heads * hd, ffn = c->ffn;
    const int64_t *b = m->w + m->off_layers + (size_t)l * m->layer_elems;
    int64_t *q = m->qkv, *k = m->qkv + dim, *v = m->qkv + dim + kvd;

    const uint16_t *bb = m->bf16 ? m->wb + m->off_layers + (size_t)l * m->layer_elems : NULL;
    const int cached = rope_in_gemv(m) && pos < q48_attn_split_min();
    if (cached) {
        if (bb)
            TRY(q48_norm_gemv_rope_kv_bf16(x, m->qkv, bb + m->lo_qkv, m->hidden, b + m->lo_an,
                                           m->s_attn, m->kc, m->vc, l, pos, c->n_heads,
                                           c->n_kv_heads, hd, c->max_seq, dim));
        else
            TRY(q48_norm_gemv_rope_kv(x, m->qkv, b + m->lo_qkv, m->hidden, b + m->lo_an,
                                      m->s_attn, m->kc, m->vc, l, pos, c->n_heads,
                                      c->n_kv_heads, hd, c->max_seq, dim));
    } else if (m->fused == 3 && bb) {
        TRY(q48_norm_gemv_stats_bf16(x, m->qkv, bb + m->lo_qkv, m->hidden, b + m->lo_an,
                                     m->s_attn, dim + 2 * kvd, dim));
    } else if (m->fused == 3) {
        /* s_attn holds the partial sums of squares of hidden (from the
         * embedding or the previous layer's down projection) */
        TRY(q48_norm_gemv_stats(x, m->qkv, b + m->lo_qkv, m->hidden, b + m->lo_an, m->s_attn,
                                dim + 2 * kvd, dim));
    } else if (m->fused == 2) {
        /* r_attn holds the statistics of hidden (from the embedding or the
         * previous layer's down projection) */
        TRY(q48_norm_gemv(x, m->qkv, b + m->lo_qkv, m->hidden, b + m->lo_an, m->r_attn,
                          dim + 2 * kvd, dim));
    } else {
        TRY(q48_rmsnorm_gemv(x, m->qkv, b + m->lo_qkv, m->hidden, b + m->lo_an,
                             dim + 2 * kvd, dim));
    }
    /* with bfloat16-resident weights the attention's spare blocks warm the
     * cache with W_o, read next (1.4751 against 1.4779 ms per TinyLlama-shape
     * token).  int64 weights are read with non-temporal loads, and warming
     * them measured slower (1.8436 against 1.8234). */
    if (cached)
        TRY(q48_attn_decode_cached(x, m->attn, q, m->kc, m->vc, l, pos, c->n_heads,
                                   c->n_kv_heads, hd, c->max_seq,
                                   m->prefetch && bb ? bb + m->lo_wo : NULL,
                                   m->prefetch && bb ? (size_t)dim * dim * 2 : 0));
    else if (m->prefetch && bb)
        TRY(q48_attn_decode_rope_prefetch(x, m->attn, q, m->kc, m->vc, k, v, l, pos, c->n_heads,
                                          c->n_kv_heads, hd, c->max_seq, bb + m->lo_wo,
                                          (size_t)dim * dim * 2));
    else
        TRY(q48_attn_decode_rope(x, m->attn, q, m->kc, m->vc, k, v, l, pos, c->n_heads,
                                 c->n_kv_heads, hd, c->max_seq));
    if (m->fused == 3 && bb) {
        TRY(q48_gemv_residual_stats_bf16(x, m->hidden, bb + m->lo_wo, m->attn, dim, dim,
                                         m->s_ffn));
        TRY(q48_norm_gemv_swiglu_stats_bf16(x, m->h_ffn, bb + m->lo_gu, m->hidden, b + m->lo_fn,
                                            m->s_ffn, ffn, dim));
        TRY(q48_gemv_residual_stats_bf16(x, m->hidden, bb + m->lo_wd, m->h_ffn, dim, ffn,
                                         m->s_attn));
    } else if (m->fused == 3) {
        TRY(q48_gemv_residual_stats(x, m->hidden, b + m->lo_wo, m->attn, dim, dim, m->s_ffn));
        TRY(q48_norm_gemv_swiglu_stats(x, m->h_ffn, b + m->lo_gu, m->hidden, b + m->lo_fn,
                                       m->s_ffn, ffn, dim));
        TRY(q48_gemv_residual_stats(x, m->hidden, b + m->lo_wd, m->h_ffn, dim, ffn, m->s_attn));
    } else if (m->fused == 2) {
        TRY(q48_gemv_residual_rms(x, m->hidden, b + m->lo_wo, m->attn, dim, dim, m->r_ffn));
        TRY(q48_norm_gemv_swiglu(x, m->h_ffn, b + m->lo_gu, m->hidden, b + m->lo_fn, m->r_ffn,
                                 ffn, dim));
        TRY(q48_gemv_residual_rms(x, m->hidden, b + m->lo_wd, m->h_ffn, dim, ffn, m->r_attn));
    } else {
        TRY(q48_gemv_residual(x, m->hidden, b + m->lo_wo, m->attn, dim, dim));
        TRY(q48_rmsnorm_gemv_swiglu(x, m->h_ffn, b + m->lo_gu, m->hidden, b + m->lo_fn, ffn,
                                    dim));
        TRY(q48_gemv_residual(x, m->hidden, b + m->lo_wd, m->h_ffn, dim, ffn));
    }
    return Q48_OK;
}

/* The same layer as one library op per reference step (testing path). */
static int layer_forward(q48h_model *m, int l, int pos)
{
    const q48h_config *c = &m->c;
    q48_ctx *x = m->ctx;
    int dim = c->dim, hd = c->head_dim, kvd = c->n_kv_heads * hd, ffn = c->ffn;
    const int64_t *b = m->w + m->off_layers + (size_t)l * m->layer_elems;
    int64_t *q = m->qkv, *k = m->qkv + dim, *v = m->qkv + dim + kvd;

    TRY(q48_rmsnorm(x, m->normed, m->hidden, b + m->lo_an, dim));
    TRY(q48_gemv(x, m->qkv, b + m->lo_qkv, m->normed, dim + 2 * kvd, dim));
    TRY(q48_rope(x, q, c->n_heads, hd, pos));
    TRY(q48_rope(x, k, c->n_kv_heads, hd, pos));
    TRY(q48_attn_decode(x, m->attn, q, m->kc, m->vc, k, v, l, pos, c->n_heads,
                        c->n_kv_heads, hd, c->max_seq));
    TRY(q48_gemv(x, m->o, b + m->lo_wo, m->attn, dim, dim));
    TRY(q48_add(x, m->hidden, m->o, dim));
    TRY(q48_rmsnorm(x, m->normed, m->hidden, b + m->lo_fn, dim));
    TRY(q48_gemv(x, m->gu, b + m->lo_gu, m->normed, 2 * ffn, dim));
    TRY(q48_silu_mul(x, m->h_ffn, m->gu, m->gu + ffn, ffn));
    TRY(q48_gemv(x, m->mlp, b + m->lo_wd, m->h_ffn, dim, ffn));
    TRY(q48_add(x, m->hidden, m->mlp, dim));
    return Q48_OK;
}

/* Enqueue one llama_forward (llama_int.c:2807-2886) up to the logits. */
static int enqueue_forward(q48h_model *m, int token, int pos)
{
    const q48h_config *c = &m->c;
    if (m->fused == 3) {
        TRY(q48_embed_stats(m->ctx, m->hidden, m->w + m->off_embed, token, c->dim, m->s_attn));
        for (int l = 0; l < c->n_layers; ++l)
            TRY(layer_forward_fused(m, l, pos));
        if (m->bf16)
            TRY(q48_norm_gemv_stats_bf16(m->ctx, m->logits, m->wb + m->off_lm, m->hidden,
                                         m->w + m->off_norm, m->s_attn, c->vocab, c->dim));
        else
            TRY(q48_norm_gemv_stats(m->ctx, m->logits, m->w + m->off_lm, m->hidden,
                                    m->w + m->off_norm, m->s_attn, c->vocab, c->dim));
    } else if (m->fused == 2) {
        TRY(q48_embed_rms(m->ctx, m->hidden, m->w + m->off_embed, token, c->dim, m->r_attn));
        for (int l = 0; l < c->n_layers; ++l)
            TRY(layer_forward_fused(m, l, pos));
        TRY(q48_norm_gemv(m->ctx, m->logits, m->w + m->off_lm, m->hidden, m->w + m->off_norm,
                          m->r_attn, c->vocab, c->dim));
    } else if (m->fused == 1) {
        TRY(q48_embed(m->ctx, m->hidden, m->w + m->off_embed, token, c->dim));
        for (int l = 0; l < c->n_layers; ++l)
            TRY(layer_forward_fused(m, l, pos));
        TRY(q48_rmsnorm_gemv(m->ctx, m->logits, m->w + m->off_lm, m->hidden,
                             m->w + m->off_norm, c->vocab, c->dim));
    } else {
        TRY(q48_embed(m->ctx, m->hidden, m->w + m->off_embed, token, c->dim));
        for (int l = 0; l < c->n_layers; ++l)
            TRY(layer_forward(m, l, pos));
        TRY(q48_rmsnorm(m->ctx, m->normed, m->hidden, m->w + m->off_norm, c->dim));
        TRY(q48_gemv(m->ctx, m->logits, m->w + m->off_lm, m->normed, c->vocab, c->dim));
    }
    return Q48_OK;
}

int q48h_read_logits(q48h_model *m, int64_t *logits)
{
    if (!m || !logits)
        return Q48_EINVAL;
    return q48_memcpy_d2h(m->ctx, logits, m->logits, (size_t)m->c.vocab * 8);
}

int q48h_forward(q48h_model *m, int token, int pos, int64_t *logits, int *next)
{
    if (!m)
        return Q48_EINVAL;
    const q48h_config *c = &m->c;
    if (token < 0 || token >= c->vocab || pos < 0 || pos >= c->max_seq)
        return Q48_ERANGE;
    TRY(enqueue_forward(m, token, pos));
    if (next)
        TRY(select_token(m, next));
    if (logits)
        TRY(q48_memcpy_d2h(m->ctx, logits, m->logits, (size_t)c->vocab * 8));
    /* a split attention that gave up left wrong logits: the forward fails,
     * as the reference's llama_forward returning NULL (llama_int.c:3083-3086,
     * 3106); synchronises (nothing is read back unless one-launch split
     * attention ran) */
    return q48_attn_status(m->ctx);
}

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

void q48h_model_set_batched_prefill(q48h_model *m, int on)
{
    if (m)
        m->batched_prefill = on != 0;
}

int q48h_prefill(q48h_model *m, const int *tokens, int T, int p0, int64_t *logits_all,
                 int *next)
{
    if (!m || !tokens || T <= 0)
        return Q48_EINVAL;
    const q48h_config *c = &m->c;
    const int dim = c->dim, hd = c->head_dim, kvd = c->n_kv_heads * hd, ffn = c->ffn;
    const int V = c->vocab, nq = dim + 2 * kvd;
    if (p0 < 0 || p0 + T > c->max_seq)
        return Q48_ERANGE;
    for (int t = 0; t < T; ++t)
        if (tokens[t] < 0 || tokens[t] >= V)
            return Q48_ERANGE;
    q48_ctx *x = m->ctx;
    /* one row per token at a time past what a single-block attention keeps
     * in LDS, or for one or two tokens (two forward calls take about 3.8 ms
     * on the TinyLlama shape, one batched pass of 2-8 tokens about 4.3) */
    if (T < 3 || p0 + T > 4096 || !(hd == 32 || hd == 64 || hd == 128)) {
        for (int t = 0; t < T; ++t) {
            TRY(enqueue_forward(m, tokens[t], p0 + t));
            if (logits_all)
                TRY(q48_memcpy_d2h(x, logits_all + (size_t)t * V, m->logits, (size_t)V * 8));
        }
        if (next)
            TRY(select_token(m, next));
        return q48_attn_status(x);
    }
    /* rows: H, XN, QKV, ATT, D, GU, HF, logits (all T, or the last), ids */
    const size_t nlog = logits_all ? (size_t)T * V : (size_t)V;
    const size_t need = (size_t)T * (4 * (size_t)dim + nq + 3 * (size_t)ffn) + nlog +
                        ((size_t)T + 1) / 2;
    if (need > m->pf_words) {
        TRY(q48_sync(x));
        q48_free(x, m->pf);
        m->pf = NULL;
        m->pf_words = 0;
        TRY(q48_malloc(x, (void **)&m->pf, need * 8));
        m->pf_words = need;
    }
    int64_t *H = m->pf, *XN = H + (size_t)T * dim, *QKV = XN + (size_t)T * dim;
    int64_t *ATT = QKV + (size_t)T * nq, *D = ATT + (size_t)T * dim;
    int64_t *GU = D + (size_t)T * dim, *HF = GU + (size_t)T * 2 * ffn;
    int64_t *LG = HF + (size_t)T * ffn;
    int *ids = (int *)(LG + nlog);
    /* prepared weight planes pay off from 2 tokens (q48_gemm_prepared) */
    size_t poff[4] = {0, 0, 0, 0}, pstride = 0;
    if (T >= 2) {
        TRY(prepare_planes(m));
        if (m->wp_ok)
            pstride = planes_layout(m, poff);
    }
    TRY(q48_memcpy_h2d(x, ids, tokens, (size_t)T * sizeof(int)));
    TRY(q48_embed_rows(x, H, m->w + m->off_embed, ids, T, dim));
    for (int l = 0; l < c->n_layers; ++l) {
        const int64_t *b = m->w + m->off_layers + (size_t)l * m->layer_elems;
        const char *wp = pstride ? (const char *)m->wp + (size_t)l * pstride : NULL;
#define WP(i) (wp ? wp + poff[i] : NULL)
        TRY(q48_rmsnorm_rows(x, XN, H, b + m->lo_an, T, dim));
        TRY(prefill_gemm(x, QKV, b + m->lo_qkv, WP(0), XN, T, nq, dim));
        TRY(q48_rope_store_rows(x, QKV, m->kc, m->vc, l, p0, T, c->n_heads, c->n_kv_heads, hd,
                                c->max_seq));
        TRY(q48_attn_prefill(x, ATT, QKV, m->kc, m->vc, l, p0, T, c->n_heads, c->n_kv_heads, hd,
                             c->max_seq));
        TRY(prefill_gemm(x, D, b + m->lo_wo, WP(1), ATT, T, dim, dim));
        TRY(q48_add(x, H, D, T * dim));
        TRY(q48_rmsnorm_rows(x, XN, H, b + m->lo_fn, T, dim));
        TRY(prefill_gemm(x, GU, b + m->lo_gu, WP(2), XN, T, 2 * ffn, dim));
        TRY(q48_silu_mul_rows(x, HF, GU, T, ffn));
        TRY(prefill_gemm(x, D, b + m->lo_wd, WP(3), HF, T, dim, ffn));
#undef WP
        TRY(q48_add(x, H, D, T * dim));
    }
    TRY(q48_rmsnorm_rows(x, XN, H, m->w + m->off_norm, T, dim));
    if (logits_all) {
        TRY(q48_gemm(x, LG, m->w + m->off_lm, XN, T, V, dim));
        TRY(q48_memcpy_d2d(x, m->logits, LG + (size_t)(T - 1) * V, (size_t)V * 8));
        TRY(q48_memcpy_d2h(x, logits_all, LG, (size_t)T * V * 8));
    } else {
        TRY(q48_gemv(x, m->logits, m->w + m->off_lm, XN + (size_t)(T - 1) * dim, V, dim));
    }
    if (next)
        TRY(select_token(m, next));
    return q48_sync(x);
}

int q48h_generate(q48h_model *m, const int *prompt, int prompt_len, int max_new,
                  int *out_tokens, uint64_t *step_hash, int *n_steps, q48h_stats *st)
{
    if (!m || !prompt || !out_tokens || prompt_len <= 0)
        return Q48_EINVAL;
    int vocab = m->c.vocab, steps = 0;
    int64_t *logits = step_hash ? (int64_t *)malloc((size_t)vocab * 8) : NULL;
    if (step_hash && !logits)
        return Q48_ENOMEM;
    int rc = q48h_kv_reset(m);
    memcpy(out_tokens, prompt, (size_t)prompt_len * sizeof(int));
    int total = prompt_len;
    double t0 = now_s();
    if (rc == Q48_OK && m->batched_prefill && prompt_len > 1) {
        /* the prompt in one batched pass: the same cache and logits */
        int64_t *all = step_hash ? (int64_t *)malloc((size_t)prompt_len * vocab * 8) : NULL;
        int next;
        if (step_hash && !all)
            rc = Q48_ENOMEM;
        if (rc == Q48_OK)
            rc = q48h_prefill(m, out_tokens, prompt_len, 0, all, &next);
        if (rc == Q48_OK) {
            for (int pos = 0; pos < prompt_len; ++pos, ++steps)
                if (step_hash)
                    step_hash[steps] = q48s_fnv_i64(FNV_OFF, all + (size_t)pos * vocab,
                                                    (size_t)vocab);
            out_tokens[total++] = next;
        }
        free(all);
    } else {
        for (int pos = 0; pos < prompt_len && rc == Q48_OK; ++pos) {
            int next;
            /* the token is chosen (and a sample drawn) at the last prompt
             * position only (llama_int.c:3087-3090) */
            rc = q48h_forward(m, out_tokens[pos], pos, logits,
                              pos == prompt_len - 1 ? &next : NULL);
            if (rc)
                break;
            if (step_hash)
                step_hash[steps] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
            steps++;
            if (pos == prompt_len - 1)
                out_tokens[total++] = next;
        }
    }
    double t1 = now_s();
    int dec0 = total;
    for (int i = 1; i < max_new && rc == Q48_OK; ++i) {
        int pos = prompt_len + i - 1, next;
        int frc = q48h_forward(m, out_tokens[pos], pos, logits, &next);
        if (frc == Q48_ERANGE)
            break;   /* llama_forward's NULL: generate stops (llama_int.c:3106) */
        if (frc) {
            rc = frc;
            break;
        }
        if (step_hash)
            step_hash[steps] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        if (next == LLAMA_EOS)
            break;
        out_tokens[total++] = next;
    }
    double t2 = now_s();
    free(logits);
    if (st) {
        st->prefill_s += t1 - t0;
        st->prefill_tokens += prompt_len;
        st->decode_s += t2 - t1;
        st->decode_tokens += total - dec0;
    }
    if (n_steps)
        *n_steps = steps;
    return rc ? rc : total;
}

int q48h_decode_from(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                     uint64_t *step_hash, q48h_stats *st)
{
    if (!m || n < 0)
        return Q48_EINVAL;
    int vocab = m->c.vocab, steps = 0, tok = token, rc = Q48_OK;
    int64_t *logits = step_hash ? (int64_t *)malloc((size_t)vocab * 8) : NULL;
    if (step_hash && !logits)
        return Q48_ENOMEM;
    double t0 = now_s();
    for (int i = 0; i < n; ++i) {
        int next;
        rc = q48h_forward(m, tok, start_pos + i, logits, &next);
        if (rc == Q48_ERANGE) {
            rc = Q48_OK;
            break;
        }
        if (rc)
            break;
        if (step_hash)
            step_hash[i] = q48s_fnv_i64(FNV_OFF, logits, (size_t)vocab);
        steps++;
        tok = next;
        if (out_tokens)
            out_tokens[i] = tok;
        if (tok == LLAMA_EOS)
            break;
    }
    if (st) {
        st->decode_s += now_s() - t0;
        st->decode_tokens += steps;
    }
    free(logits);
    return rc ? rc : steps;
}

/* ---------------------------------------------------------------------- */
/* graph-replayed greedy decode                                            */
/* ---------------------------------------------------------------------- */

/* Run decode step 0 eagerly in step mode (forward(token, pos), the device
 * token choice -- argmax or sample_token -- recorded as tokens[0]) -- workspaces reach their size outside any
 * capture -- then capture the same step into the context graph.  Kernels
 * read token / pos from the device step state, so the graph serves every
 * later position. */
static int first_step_and_capture(q48h_model *m, int token, int pos)
{
    q48_ctx *x = m->ctx;
    TRY(q48_step_mode(x, 1));
    int rc = q48_step_set(x, token, pos);
    if (rc == Q48_OK) {
        rc = enqueue_forward(m, token, pos);
        if (rc == Q48_OK)
            rc = record_and_select_step(m);
        if (rc == Q48_OK)
            rc = q48_sync(x);
    }
    /* the graph of this step's settings: cached, or captured now */
    struct graph_key k;
    memset(&k, 0, sizeof k);   /* the key is compared byte for byte */
    k.kind = step_kind(m, pos);
    k.record = m->record;
    k.rec = m->record ? (const void *)m->rec : NULL;
    k.rec_cap = m->record ? m->rec_cap : 0;
    k.bf16 = m->bf16;
    k.wb = m->bf16 ? (const void *)m->wb : NULL;
    k.fused = m->fused;
    k.rope_gemv = m->rope_gemv;
    k.prefetch = m->prefetch;
    if (m->temperature >= Q48_ONE / 100) {   /* sampling: its parameters are kernel arguments */
        k.temperature = m->temperature;
        k.top_k = m->top_k;
        k.top_p = m->top_p;
    }
    k.stamp = q48_graph_stamp(x);
    m->g_run = NULL;
    int slot = -1;
    for (int i = 0; i < GRAPH_SLOTS && slot < 0; ++i)
        if (m->gslot[i].used && !memcmp(&m->gslot[i].k, &k, sizeof k))
            slot = i;
    if (rc == Q48_OK && slot < 0) {
        /* an empty slot, else the least recently used one */
        slot = 0;
        for (int i = 0; i < GRAPH_SLOTS; ++i) {
            if (!m->gslot[i].used) {
                slot = i;
                break;
            }
            if (m->gslot[i].used < m->gslot[slot].used)
                slot = i;
        }
        if (m->gslot[slot].used) {
            q48_graph_destroy(x, m->gslot[slot].g);
            m->gslot[slot].g = NULL;
            m->gslot[slot].used = 0;
        }
        rc = q48_graph_capture(x);
        if (rc == Q48_OK) {
            int rc1 = enqueue_forward(m, token, pos);
            if (rc1 == Q48_OK)
                rc1 = record_and_select_step(m);
            q48_graph *g = NULL;
            rc = q48_graph_instantiate(x, &g);
            if (rc == Q48_OK && rc1) {
                q48_graph_destroy(x, g);
                g = NULL;
            }
            if (rc1)
                rc = rc1;
            if (rc == Q48_OK) {
                m->gslot[slot].g = g;
                m->gslot[slot].k = k;
                m->gslot[slot].used = 1;
            }
        }
    }
    if (rc == Q48_OK) {
        m->gslot[slot].used = ++m->runs;
        m->g_run = m->gslot[slot].g;
    }
    q48_step_mode(x, 0);
    return rc;
}

/* FNV-1a 64 of the recorded logits of steps [0, k), into hash[0..k). */
static int hash_recorded(q48h_model *m, int k, uint64_t *hash)
{
    const size_t V = (size_t)m->c.vocab;
    int64_t *buf = (int64_t *)malloc(V * 8);
    if (!buf)
        return Q48_ENOMEM;
    int rc = Q48_OK;
    for (int i = 0; i < k && rc == Q48_OK; ++i) {
        rc = q48_memcpy_d2h(m->ctx, buf, m->rec + (size_t)i * V, V * 8);
        if (rc == Q48_OK)
            hash[i] = q48s_fnv_i64(FNV_OFF, buf, V);
    }
    free(buf);
    return rc;
}

static int decode_graph_run(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                            uint64_t *step_hash, q48h_stats *st)
{
    if (!m || !out_tokens || n < 0)
        return Q48_EINVAL;
    const q48h_config *c = &m->c;
    if (token < 0 || token >= c->vocab || start_pos < 0)
        return Q48_ERANGE;
    if (start_pos + n > c->max_seq)
        n = c->max_seq - start_pos;   /* llama_forward's NULL past max_seq */
    if (n <= 0)
        return 0;
    /* recording: one logits row per step of the longest part below */
    m->record = step_hash != NULL;
    if (m->record && m->rec_cap < n) {
        /* graphs that record into the old buffer are keyed on its address
         * and capacity: they are never replayed against the new one */
        int cap = n > 512 ? n : (c->max_seq < 512 ? c->max_seq : 512);
        q48_free(m->ctx, m->rec);
        m->rec = NULL;
        m->rec_cap = 0;
        TRY(q48_malloc(m->ctx, (void **)&m->rec, (size_t)cap * c->vocab * 8));
        m->rec_cap = cap;
    }
    /* dt: the steps on the device, from the first step's launch to the
     * tokens back on the host (the hashing of recorded logits is not in it) */
    double t0 = now_s();
    TRY(first_step_and_capture(m, token, start_pos));
    /* a graph serves one attention kernel class: a run that crosses the
     * position where attention changes kernels is replayed in two parts,
     * the second from a graph captured at that position */
    const int B = q48_attn_split_min();
    int k = n;
    if (start_pos < B && start_pos + n > B)
        k = B - start_pos;
    TRY(q48_graph_replay(m->ctx, m->g_run, k - 1));
    TRY(q48_memcpy_d2h(m->ctx, out_tokens, m->d_tokens, (size_t)k * sizeof(int)));
    double dt = now_s() - t0;
    if (step_hash)
        TRY(hash_recorded(m, k, step_hash));
    if (k < n) {
        t0 = now_s();
        TRY(first_step_and_capture(m, out_tokens[k - 1], B));
        TRY(q48_graph_replay(m->ctx, m->g_run, n - k - 1));
        TRY(q48_memcpy_d2h(m->ctx, out_tokens + k, m->d_tokens, (size_t)(n - k) * sizeof(int)));
        dt += now_s() - t0;
        if (step_hash)
            TRY(hash_recorded(m, n - k, step_hash + k));
    }
    /* a split attention that gave up: the run's outputs are wrong (the
     * reference's generate stops on a failed forward, llama_int.c:3106) */
    TRY(q48_attn_status(m->ctx));
    /* generate stops at EOS (llama_int.c:3111): the steps up to and
     * including the one that chose it count; the device replayed the rest */
    int ran = n;
    for (int i = 0; i < n; ++i)
        if (out_tokens[i] == LLAMA_EOS) {
            ran = i + 1;
            break;
        }
    if (st) {
        st->decode_s += dt;
        st->decode_tokens += ran;
    }
    return ran;
}

int q48h_decode_graph(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                      q48h_stats *st)
{
    return decode_graph_run(m, token, start_pos, n, out_tokens, NULL, st);
}

int q48h_decode_graph_hashed(q48h_model *m, int token, int start_pos, int n, int *out_tokens,
                             uint64_t *step_hash, q48h_stats *st)
{
    if (!step_hash)
        return Q48_EINVAL;
    return decode_graph_run(m, token, start_pos, n, out_tokens, step_hash, st);
}

/* ---------------------------------------------------------------------- */
/* measurement helper                                                      */
/* ---------------------------------------------------------------------- */

int q48h_gemv_sweep(q48h_model *m, int reps, int *launches, double *bytes)
{
    if (!m || reps < 0)
        return Q48_EINVAL;
    const q48h_config *c = &m->c;
    q48_ctx *x = m->ctx;
    int dim = c->dim, kvd = c->n_kv_heads * c->head_dim, ffn = c->ffn;
    int n = 0;
    double b = 0;
    const int wb16 = m->fused == 3 && m->bf16;
    const int rq = rope_in_gemv(m);
    const double wbytes = wb16 ? 2.0 : 8.0;
#define GB(M, K, out) (b += wbytes * (double)(M) * (K) + 8.0 * ((double)(K) + (out)), ++n)
    for (int r = 0; r < reps; ++r) {
        for (int l = 0; l < c->n_layers; ++l) {
            const int64_t *w = m->w + m->off_layers + (size_t)l * m->layer_elems;
            const uint16_t *bw = wb16 ? m->wb + m->off_layers + (size_t)l * m->layer_elems : NULL;
            /* the q|k|v form short-context decode runs; its k and v go to
             * the last cache row, which a decode step writes before it
             * reads it */
            if (wb16 && rq)
                TRY(q48_norm_gemv_rope_kv_bf16(x, m->qkv, bw + m->lo_qkv, m->hidden,
                                               w + m->lo_an, m->s_attn, m->kc, m->vc, l,
                                               c->max_seq - 1, c->n_heads, c->n_kv_heads,
                                               c->head_dim, c->max_seq, dim));
            else if (m->fused == 3 && rq)
                TRY(q48_norm_gemv_rope_kv(x, m->qkv, w + m->lo_qkv, m->hidden, w + m->lo_an,
                                          m->s_attn, m->kc, m->vc, l, c->max_seq - 1,
                                          c->n_heads, c->n_kv_heads, c->head_dim, c->max_seq,
                                          dim));
            if (wb16) {
                if (!rq)
                    TRY(q48_norm_gemv_stats_bf16(x, m->qkv, bw + m->lo_qkv, m->hidden,
                                                 w + m->lo_an, m->s_attn, dim + 2 * kvd, dim));
                TRY(q48_gemv_residual_stats_bf16(x, m->hidden, bw + m->lo_wo, m->attn, dim, dim,
                                                 m->s_ffn));
                TRY(q48_norm_gemv_swiglu_stats_bf16(x, m->h_ffn, bw + m->lo_gu, m->hidden,
                                                    w + m->lo_fn, m->s_ffn, ffn, dim));
                TRY(q48_gemv_residual_stats_bf16(x, m->hidden, bw + m->lo_wd, m->h_ffn, dim, ffn,
                                                 m->s_attn));
            } else if (m->fused == 3) {
                if (!rq)
                    TRY(q48_norm_gemv_stats(x, m->qkv, w + m->lo_qkv, m->hidden, w + m->lo_an,
                                            m->s_attn, dim + 2 * kvd, dim));
                TRY(q48_gemv_residual_stats(x, m->hidden, w + m->lo_wo, m->attn, dim, dim,
                                            m->s_ffn));
                TRY(q48_norm_gemv_swiglu_stats(x, m->h_ffn, w + m->lo_gu, m->hidden,
                                               w + m->lo_fn, m->s_ffn, ffn, dim));
                TRY(q48_gemv_residual_stats(x, m->hidden, w + m->lo_wd, m->h_ffn, dim, ffn,
                                            m->s_attn));
            } else {
                TRY(q48_norm_gemv(x, m->qkv, w + m->lo_qkv, m->hidden, w + m->lo_an,
                                  m->r_attn, dim + 2 * kvd, dim));
                TRY(q48_gemv_residual_rms(x, m->hidden, w + m->lo_wo, m->attn, dim, dim,
                                          m->r_ffn));
                TRY(q48_norm_gemv_swiglu(x, m->h_ffn, w + m->lo_gu, m->hidden, w + m->lo_fn,
                                         m->r_ffn, ffn, dim));
                TRY(q48_gemv_residual_rms(x, m->hidden, w + m->lo_wd, m->h_ffn, dim, ffn,
                                          m->r_attn));
            }
            GB(dim + 2 * kvd, dim, dim + 2 * kvd);
            GB(dim, dim, dim);
            GB(2 * ffn, dim, ffn);
            GB(dim, ffn, dim);
        }
        if (wb16)
            TRY(q48_norm_gemv_stats_bf16(x, m->logits, m->wb + m->off_lm, m->hidden,
                                         m->w + m->off_norm, m->s_attn, c->vocab, dim));
        else if (m->fused == 3)
            TRY(q48_norm_gemv_stats(x, m->logits, m->w + m->off_lm, m->hidden,
                                    m->w + m->off_norm, m->s_attn, c->vocab, dim));
        else
            TRY(q48_norm_gemv(x, m->logits, m->w + m->off_lm, m->hidden, m->w + m->off_norm,
                              m->r_attn, c->vocab, dim));
        GB(c->vocab, dim, c->vocab);
    }
#undef GB
    if (launches)
        *launches = n;
    if (bytes)
        *bytes = b;
    return Q48_OK;
}
