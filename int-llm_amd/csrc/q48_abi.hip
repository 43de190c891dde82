// q48_abi.hip — extern "C" entry points of libintllm_hip (include/intllm_hip.h).
//
// Validates every argument on the host before anything is launched (a
// kernel never sees a shape it does not support), then enqueues the
// kernels on the context's stream.
#include "../../include/intllm_hip.h"
#include "q48_internal.h"

#include <new>
#include <stdlib.h>

namespace {

int hip_rc(hipError_t e) { return e == hipSuccess ? Q48_OK : Q48_EHIP; }
int launch_rc(int e) { return e == (int)hipSuccess ? Q48_OK : Q48_EHIP; }

// Largest sizes the kernels are written for.
constexpr int kMaxDim = 1 << 28;
constexpr int kMaxHeadDim = 256;

} // namespace

int q48_release(q48_ctx *c, void *p)
{
    if (!p)
        return Q48_OK;
    // earlier kernels may still read it
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    if (c->n_graphs <= 0)
        return hip_rc(hipFree(p));
    // an instantiated graph may hold this address: keep the buffer until the
    // last graph is destroyed (the graph keeps working on it)
    if (c->n_retired == c->cap_retired) {
        const int cap = c->cap_retired ? 2 * c->cap_retired : 8;
        void **r = (void **)realloc(c->retired, (size_t)cap * sizeof(void *));
        if (!r)
            return Q48_ENOMEM;
        c->retired = r;
        c->cap_retired = cap;
    }
    c->retired[c->n_retired++] = p;
    return Q48_OK;
}

namespace {
void graph_destroy(q48_ctx *c, q48_graph *g);

void free_retired(q48_ctx *c)
{
    for (int i = 0; i < c->n_retired; ++i)
        (void)hipFree(c->retired[i]);
    c->n_retired = 0;
}
} // namespace

int q48_ws_reserve(q48_ctx *c, size_t bytes)
{
    if (bytes <= c->ws_bytes)
        return Q48_OK;
    if (c->capturing)
        return Q48_ESTATE;   // workspaces reach their size outside a capture
    if (c->ws) {
        int rc = q48_release(c, c->ws);
        if (rc)
            return rc;
        c->ws = nullptr;
        c->ws_bytes = 0;
    }
    size_t sz = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    if (hipMalloc(&c->ws, sz) != hipSuccess) {
        c->ws = nullptr;
        (void)hipGetLastError();   // not left for the next launch's error check
        return Q48_ENOMEM;
    }
    c->ws_bytes = sz;
    return Q48_OK;
}

int q48_rms_reserve(q48_ctx *c, int blocks)
{
    if (blocks <= c->rms_blocks)
        return Q48_OK;
    if (c->capturing)
        return Q48_ESTATE;
    if (c->rms_part) {
        int rc = q48_release(c, c->rms_part);
        if (rc)
            return rc;
        c->rms_part = nullptr;
        c->rms_blocks = 0;
    }
    int n = blocks < 1024 ? 1024 : blocks;
    if (hipMalloc(&c->rms_part, (size_t)n * 2 * sizeof(uint64_t)) != hipSuccess) {
        c->rms_part = nullptr;
        (void)hipGetLastError();
        return Q48_ENOMEM;
    }
    c->rms_blocks = n;
    return Q48_OK;
}

extern "C" {

const char *q48_strerror(int code)
{
    switch (code) {
    case Q48_OK: return "ok";
    case Q48_EINVAL: return "invalid argument";
    case Q48_ENOMEM: return "device out of memory";
    case Q48_EHIP: return "HIP runtime error";
    case Q48_ERANGE: return "token or position out of range";
    case Q48_ESTATE: return "context state not initialised (call q48_rope_init)";
    case Q48_ETIMEOUT: return "one-launch decode step or attention timed out (blocks not resident)";
    case Q48_ETOOBIG: return "size exceeds the allocation-free scratch";
    default: return "unknown error";
    }
}

int q48_ctx_create(q48_ctx **out, int device)
{
    if (!out)
        return Q48_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return Q48_EINVAL;
    if (hipSetDevice(device) != hipSuccess)
        return Q48_EHIP;
    q48_ctx *c = new (std::nothrow) q48_ctx();
    if (!c)
        return Q48_ENOMEM;
    c->device = device;
    c->gemv_persistent = 1;
    if (hipDeviceGetAttribute(&c->cu_count, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        c->cu_count <= 0)
        c->cu_count = 1;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return Q48_EHIP;
    }
    c->attn_one_launch = 1;
    c->pf_attn_mfma = 1;
    c->attx_per_cu[0] = c->attx_per_cu[1] = c->attx_per_cu[2] = c->attx_per_cu[3] = -1;
    c->attn_g_mfma = 1;
    c->attg_wait = q48_attg_default_wait();
    if (hipMalloc(&c->consts, sizeof(q48_consts)) != hipSuccess ||
        hipMalloc(&c->d_scalar, 64 * sizeof(int)) != hipSuccess ||
        hipMalloc(&c->d_step, 4 * sizeof(int)) != hipSuccess ||
        hipMalloc(&c->amax_part, q48_amax_part_bytes()) != hipSuccess ||
        hipMalloc(&c->rms_count, 512 * sizeof(int)) != hipSuccess ||
        hipMalloc(&c->attx_sync, q48_attn_sync_bytes()) != hipSuccess) {
        q48_ctx_destroy(c);
        return Q48_ENOMEM;
    }
    int rc = launch_rc(q48_launch_math_init(c));
    if (rc == Q48_OK)
        rc = launch_rc(q48_launch_zero(c, c->attx_sync, q48_attn_sync_bytes()));
    if (rc == Q48_OK)   // the allocation-free entry point's scratch on this device
        rc = q48_scratch_init(c);
    if (rc == Q48_OK)
        rc = launch_rc(q48_launch_step_set(c, 0, 0));
    if (rc == Q48_OK)
        rc = launch_rc(q48_launch_zero(c, c->rms_count, 512 * sizeof(int)));
    if (rc == Q48_OK)
        rc = launch_rc(q48_launch_zero(c, c->amax_part, q48_amax_part_bytes()));
    if (rc == Q48_OK)
        rc = launch_rc(q48_launch_zero(c, c->d_scalar, 64 * sizeof(int)));
    if (rc == Q48_OK)
        rc = hip_rc(hipStreamSynchronize(c->stream));
    if (rc != Q48_OK) {
        q48_ctx_destroy(c);
        return rc;
    }
    *out = c;
    return Q48_OK;
}

int q48_ctx_destroy(q48_ctx *c)
{
    if (!c)
        return Q48_EINVAL;
    if (c->stream)
        (void)hipStreamSynchronize(c->stream);
    (void)hipFree(c->consts);
    (void)hipFree(c->rope_cos);
    (void)hipFree(c->rope_sin);
    (void)hipFree(c->ws);
    (void)hipFree(c->d_scalar);
    (void)hipFree(c->d_step);
    (void)hipFree(c->amax_part);
    (void)hipFree(c->rms_count);
    (void)hipFree(c->rms_part);
    (void)hipFree(c->smp);
    (void)hipFree(c->tmp);
    (void)hipFree(c->attx_sync);
    graph_destroy(c, c->cur);
    c->cur = nullptr;
    free_retired(c);   // handles the caller never destroyed keep nothing alive
    free(c->retired);
    for (int i = 0; i < c->prof_cap; ++i) {
        if (c->prof[i].a)
            (void)hipEventDestroy(c->prof[i].a);
        if (c->prof[i].b)
            (void)hipEventDestroy(c->prof[i].b);
    }
    free(c->prof);
    if (c->span_a)
        (void)hipEventDestroy(c->span_a);
    if (c->span_b)
        (void)hipEventDestroy(c->span_b);
    if (c->stream)
        (void)hipStreamDestroy(c->stream);
    delete c;
    return Q48_OK;
}

int q48_malloc(q48_ctx *c, void **dptr, size_t bytes)
{
    if (!c || !dptr || bytes == 0)
        return Q48_EINVAL;
    if (hipMalloc(dptr, bytes) != hipSuccess) {
        *dptr = nullptr;
        (void)hipGetLastError();   // not left for the next launch's error check
        return Q48_ENOMEM;
    }
    return Q48_OK;
}

int q48_free(q48_ctx *c, void *dptr)
{
    if (c && c->capturing)
        return Q48_ESTATE;
    if (!c)
        return Q48_EINVAL;
    if (!dptr)
        return Q48_OK;
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    return hip_rc(hipFree(dptr));
}

int q48_memcpy_h2d(q48_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (c && c->capturing)
        return Q48_ESTATE;
    if (!c || (bytes && (!dst || !src)))
        return Q48_EINVAL;
    if (!bytes)
        return Q48_OK;
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    return hip_rc(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
}

int q48_memcpy_d2h(q48_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (c && c->capturing)
        return Q48_ESTATE;
    if (!c || (bytes && (!dst || !src)))
        return Q48_EINVAL;
    if (!bytes)
        return Q48_OK;
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    return hip_rc(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
}

int q48_memcpy_d2d(q48_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (!c || (bytes && (!dst || !src)))
        return Q48_EINVAL;
    if (!bytes)
        return Q48_OK;
    return hip_rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream));
}

int q48_zero(q48_ctx *c, void *dptr, size_t bytes)
{
    if (!c || (bytes && !dptr))
        return Q48_EINVAL;
    if (!bytes)
        return Q48_OK;
    if (((uintptr_t)dptr & 7) != 0)
        return Q48_EINVAL;
    return launch_rc(q48_launch_zero(c, dptr, bytes));
}

int q48_sync(q48_ctx *c)
{
    if (!c)
        return Q48_EINVAL;
    if (c->capturing)
        return Q48_ESTATE;
    return hip_rc(hipStreamSynchronize(c->stream));
}

namespace {
// HIP-event bracket of one GEMV launch while timing is enabled.
q48_ctx::ProfRec *prof_begin(q48_ctx *c, double bytes, int *rc)
{
    *rc = Q48_OK;
    if (!c->prof_on || c->capturing)
        return nullptr;
    if (c->prof_n == c->prof_cap) {
        int cap = c->prof_cap ? 2 * c->prof_cap : 1024;
        auto *p = (q48_ctx::ProfRec *)realloc(c->prof, sizeof(q48_ctx::ProfRec) * cap);
        if (!p) {
            *rc = Q48_ENOMEM;
            return nullptr;
        }
        for (int i = c->prof_cap; i < cap; ++i)
            p[i].a = p[i].b = nullptr;
        c->prof = p;
        c->prof_cap = cap;
    }
    q48_ctx::ProfRec *r = &c->prof[c->prof_n];
    if ((!r->a && hipEventCreate(&r->a) != hipSuccess) ||
        (!r->b && hipEventCreate(&r->b) != hipSuccess) ||
        hipEventRecord(r->a, c->stream) != hipSuccess) {
        *rc = Q48_EHIP;
        return nullptr;
    }
    r->bytes = bytes;
    return r;
}

int prof_end(q48_ctx *c, q48_ctx::ProfRec *r, int rc)
{
    if (r && rc == Q48_OK) {
        if (hipEventRecord(r->b, c->stream) != hipSuccess)
            return Q48_EHIP;
        c->prof_n++;
    }
    return rc;
}

double gemv_bytes(int M, int K, int out) { return 8.0 * ((double)M * K + K + out); }
} // namespace

int q48_gemv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x, int M, int K)
{
    if (!c || !y || !W || !x || M <= 0 || K <= 0 || M > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    if ((((uintptr_t)W | (uintptr_t)x | (uintptr_t)y) & 7) != 0)
        return Q48_EINVAL;
    int rc;
    q48_ctx::ProfRec *r = prof_begin(c, gemv_bytes(M, K, M), &rc);
    if (rc)
        return rc;
    return prof_end(c, r, launch_rc(q48_launch_gemv(c, y, W, x, M, K)));
}

int q48_timer_start(q48_ctx *c)
{
    if (!c || c->capturing)
        return Q48_EINVAL;
    if ((!c->span_a && hipEventCreate(&c->span_a) != hipSuccess) ||
        (!c->span_b && hipEventCreate(&c->span_b) != hipSuccess))
        return Q48_EHIP;
    return hip_rc(hipEventRecord(c->span_a, c->stream));
}

int q48_timer_stop(q48_ctx *c, double *ms)
{
    if (!c || !ms || !c->span_a || c->capturing)
        return Q48_EINVAL;
    float f = 0;
    if (hipEventRecord(c->span_b, c->stream) != hipSuccess ||
        hipEventSynchronize(c->span_b) != hipSuccess ||
        hipEventElapsedTime(&f, c->span_a, c->span_b) != hipSuccess)
        return Q48_EHIP;
    *ms = f;
    return Q48_OK;
}

int q48_prof_enable(q48_ctx *c, int on)
{
    if (!c)
        return Q48_EINVAL;
    c->prof_on = on != 0;
    return Q48_OK;
}

int q48_prof_read(q48_ctx *c, q48_prof *out, int reset)
{
    if (!c || !out)
        return Q48_EINVAL;
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    out->launches = c->prof_n;
    out->ms = 0;
    out->bytes = 0;
    for (int i = 0; i < c->prof_n; ++i) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, c->prof[i].a, c->prof[i].b) != hipSuccess)
            return Q48_EHIP;
        out->ms += ms;
        out->bytes += c->prof[i].bytes;
    }
    if (reset)
        c->prof_n = 0;
    return Q48_OK;
}

int q48_gemm_ex(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X, int T, int N,
                int K, int kernel)
{
    if (!c || !Y || !W || !X || T <= 0 || N <= 0 || K <= 0 || T > 65535 * 64 ||
        N > kMaxDim || K > kMaxDim || kernel < Q48_GEMM_AUTO || kernel > Q48_GEMM_I8_PLANES)
        return Q48_EINVAL;
    if ((((uintptr_t)W | (uintptr_t)X | (uintptr_t)Y) & 7) != 0)
        return Q48_EINVAL;
    int rc;
    if (kernel == Q48_GEMM_AUTO && T == 1)
        rc = q48_launch_gemv(c, Y, W, X, N, K);   // one token: the decode GEMV
    else if (kernel == Q48_GEMM_VALU ||
             (kernel == Q48_GEMM_AUTO && q48_gemm_auto_kernel(T, N, K) == Q48_GEMM_VALU))
        rc = q48_launch_gemm(c, Y, W, X, T, N, K);
    else
        rc = q48_launch_gemm_i8(c, Y, W, X, T, N, K, kernel, nullptr);
    if (rc < 0)
        return rc;   // a Q48_E* code from the launcher (ENOMEM, EINVAL)
    return launch_rc(rc);
}

int q48_gemm(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X, int T, int N, int K)
{
    return q48_gemm_ex(c, Y, W, X, T, N, K, Q48_GEMM_AUTO);
}

int q48_gemm_planes_bytes(int N, int K, size_t *bytes)
{
    if (!bytes || N <= 0 || K <= 0 || N > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    *bytes = q48_gemm_planes_size(N, K);
    return Q48_OK;
}

int q48_gemm_prepare(q48_ctx *c, void *Wp, const int64_t *W, int N, int K)
{
    if (!c || !Wp || !W || N <= 0 || K <= 0 || N > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    if ((((uintptr_t)W) & 7) != 0 || (((uintptr_t)Wp) & 15) != 0)
        return Q48_EINVAL;
    const int rc = q48_launch_gemm_prepare(c, Wp, W, N, K);
    return rc < 0 ? rc : launch_rc(rc);
}

int q48_gemm_prepared(q48_ctx *c, int64_t *Y, const int64_t *W, const void *Wp,
                      const int64_t *X, int T, int N, int K)
{
    if (!c || !Y || !W || !Wp || !X || T <= 0 || N <= 0 || K <= 0 || T > 65535 * 64 ||
        N > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    if ((((uintptr_t)W | (uintptr_t)X | (uintptr_t)Y) & 7) != 0 || (((uintptr_t)Wp) & 15) != 0)
        return Q48_EINVAL;
    int rc = T == 1 ? q48_launch_gemv(c, Y, W, X, N, K)
                    : q48_launch_gemm_i8(c, Y, W, X, T, N, K, Q48_GEMM_I8, Wp);
    if (rc < 0)
        return rc;   // a Q48_E* code from the launcher (ENOMEM, EINVAL)
    return launch_rc(rc);
}

int q48_rmsnorm(q48_ctx *c, int64_t *out, const int64_t *x, const int64_t *w, int dim)
{
    if (!c || !out || !x || !w || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_rmsnorm(c, out, x, w, dim));
}

int q48_rope_init(q48_ctx *c, int head_dim, int max_seq, int theta)
{
    if (!c || head_dim <= 0 || head_dim % 2 || head_dim > kMaxHeadDim || max_seq <= 0 ||
        max_seq > 32767 || theta <= 0 || theta > 32767)
        return Q48_EINVAL;
    if (c->rope_cos && c->rope_head_dim == head_dim && c->rope_max_seq == max_seq &&
        c->rope_theta == theta)
        return Q48_OK;
    if (c->capturing)
        return Q48_ESTATE;
    int rrc = q48_release(c, c->rope_cos);
    if (rrc == Q48_OK)
        rrc = q48_release(c, c->rope_sin);
    if (rrc)
        return rrc;
    c->rope_cos = c->rope_sin = nullptr;
    c->rope_head_dim = c->rope_max_seq = c->rope_theta = 0;
    ++c->stamp;   // captured kernels hold the old tables' addresses
    size_t n = (size_t)max_seq * (head_dim / 2) * sizeof(int64_t);
    // the sine table carries one more value: the attention score scale
    if (hipMalloc(&c->rope_cos, n) != hipSuccess ||
        hipMalloc(&c->rope_sin, n + sizeof(int64_t)) != hipSuccess) {
        (void)hipFree(c->rope_cos);
        c->rope_cos = c->rope_sin = nullptr;
        (void)hipGetLastError();
        return Q48_ENOMEM;
    }
    c->rope_head_dim = head_dim;
    c->rope_max_seq = max_seq;
    c->rope_theta = theta;
    return launch_rc(q48_launch_rope_init(c));
}

int q48_rope(q48_ctx *c, int64_t *vec, int n_heads, int head_dim, int pos)
{
    if (!c || !vec || n_heads <= 0 || head_dim <= 0)
        return Q48_EINVAL;
    if (!c->rope_cos || head_dim != c->rope_head_dim)
        return Q48_ESTATE;
    if (pos < 0 || pos >= c->rope_max_seq)
        return Q48_ERANGE;
    return launch_rc(q48_launch_rope(c, vec, n_heads, head_dim,
                                     c->step_mode ? c->d_step + 1 : nullptr, pos));
}

int q48_attn_decode(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                    int64_t *vcache, const int64_t *k_new, const int64_t *v_new, int layer,
                    int pos, int n_heads, int n_kv, int head_dim, int max_seq)
{
    if (!c || !out || !q || !kcache || !vcache || !k_new || !v_new)
        return Q48_EINVAL;
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || head_dim <= 0 ||
        head_dim > kMaxHeadDim || 256 % head_dim || layer < 0 || max_seq <= 0)
        return Q48_EINVAL;
    if (pos < 0 || pos >= max_seq)
        return Q48_ERANGE;
    const int *dp = c->step_mode ? c->d_step + 1 : nullptr;
    int rc = head_dim % 8 == 0
                 ? q48_launch_attn_v2(c, out, q, kcache, vcache, k_new, v_new, layer, dp, pos,
                                      n_heads, n_kv, head_dim, max_seq, 0, nullptr, 0)
                 : q48_launch_attn(c, out, q, kcache, vcache, k_new, v_new, layer, dp, pos,
                                   n_heads, n_kv, head_dim, max_seq);
    if (rc < 0)
        return rc;   // a Q48_E* code from the launcher (ENOMEM, EINVAL)
    return launch_rc(rc);
}

int q48_silu_mul(q48_ctx *c, int64_t *out, const int64_t *gate, const int64_t *up, int n)
{
    if (!c || !out || !gate || !up || n <= 0 || n > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_silu_mul(c, out, gate, up, n));
}

int q48_add(q48_ctx *c, int64_t *acc, const int64_t *d, int n)
{
    if (!c || !acc || !d || n <= 0 || n > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_add(c, acc, d, n));
}

int q48_embed(q48_ctx *c, int64_t *out, const int64_t *table, int token, int dim)
{
    if (!c || !out || !table || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    if (token < 0)
        return Q48_ERANGE;
    return launch_rc(q48_launch_embed(c, out, table, c->step_mode ? c->d_step : nullptr,
                                      token, dim));
}

int q48_argmax(q48_ctx *c, const int64_t *v, int n, int *host_out)
{
    if (!c || !v || !host_out || n <= 0)
        return Q48_EINVAL;
    int rc = launch_rc(q48_launch_argmax(c, c->d_scalar, v, n));
    if (rc)
        return rc;
    if (hipMemcpyAsync(host_out, c->d_scalar, sizeof(int), hipMemcpyDeviceToHost,
                       c->stream) != hipSuccess)
        return Q48_EHIP;
    return hip_rc(hipStreamSynchronize(c->stream));
}

int q48_rope_tables(q48_ctx *c, const int64_t **cos_t, const int64_t **sin_t)
{
    if (!c || !cos_t || !sin_t)
        return Q48_EINVAL;
    if (!c->rope_cos)
        return Q48_ESTATE;
    *cos_t = c->rope_cos;
    *sin_t = c->rope_sin;
    return Q48_OK;
}

int q48_fp_eval(q48_ctx *c, int func, const int64_t *x, const int64_t *y, int64_t *out0,
                int64_t *out1, int n)
{
    if (!c || !x || !out0 || n <= 0 || func < 0 || func > 12)
        return Q48_EINVAL;
    if ((func == 0 || func == 1 || func == 11 || func == 12) && !y)
        return Q48_EINVAL;
    if (func == 7 && !out1)
        return Q48_EINVAL;
    return launch_rc(q48_launch_fp_eval(c, func, x, y, out0, out1, n));
}


// ---- fused decode ops ------------------------------------------------------

namespace {
int tmp_reserve(q48_ctx *c, size_t bytes)
{
    if (bytes <= c->tmp_bytes)
        return Q48_OK;
    if (c->capturing)
        return Q48_ESTATE;
    if (c->tmp) {
        int rc = q48_release(c, c->tmp);
        if (rc)
            return rc;
        c->tmp = nullptr;
        c->tmp_bytes = 0;
    }
    if (hipMalloc(&c->tmp, bytes) != hipSuccess)
        return Q48_ENOMEM;
    c->tmp_bytes = bytes;
    return Q48_OK;
}

bool bad_ptrs(const void *a, const void *b, const void *d)
{
    return !a || !b || !d || ((((uintptr_t)a) | ((uintptr_t)b) | ((uintptr_t)d)) & 7);
}
} // namespace

int q48_rmsnorm_gemv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                     const int64_t *norm_w, int M, int K)
{
    if (!c || bad_ptrs(y, W, x) || !norm_w || M <= 0 || K <= 0 || M > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(W, K)) {
        int prc;
        q48_ctx::ProfRec *r = prof_begin(c, gemv_bytes(M, K, M), &prc);
        if (prc)
            return prc;
        return prof_end(c, r, launch_rc(q48_launch_gemv_fused(c, y, W, x, norm_w, nullptr, nullptr, M, K, 1, 0)));
    }
    int rc = tmp_reserve(c, (size_t)K * 8);
    if (rc)
        return rc;
    int64_t *t = (int64_t *)c->tmp;
    rc = launch_rc(q48_launch_rmsnorm(c, t, x, norm_w, K));
    return rc ? rc : launch_rc(q48_launch_gemv(c, y, W, t, M, K));
}

int q48_gemv_residual(q48_ctx *c, int64_t *acc, const int64_t *W, const int64_t *x, int M,
                      int K)
{
    if (!c || bad_ptrs(acc, W, x) || M <= 0 || K <= 0 || M > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(W, K)) {
        int prc;
        q48_ctx::ProfRec *r = prof_begin(c, gemv_bytes(M, K, M), &prc);
        if (prc)
            return prc;
        return prof_end(c, r, launch_rc(q48_launch_gemv_fused(c, acc, W, x, nullptr, nullptr, nullptr, M, K, 0, 1)));
    }
    int rc = tmp_reserve(c, (size_t)M * 8);
    if (rc)
        return rc;
    int64_t *t = (int64_t *)c->tmp;
    rc = launch_rc(q48_launch_gemv(c, t, W, x, M, K));
    return rc ? rc : launch_rc(q48_launch_add(c, acc, t, M));
}

int q48_rmsnorm_gemv_swiglu(q48_ctx *c, int64_t *out, const int64_t *Wgu, const int64_t *x,
                            const int64_t *norm_w, int ffn, int K)
{
    if (!c || bad_ptrs(out, Wgu, x) || !norm_w || ffn <= 0 || K <= 0 || ffn > kMaxDim / 2 ||
        K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(Wgu, K)) {
        int prc;
        q48_ctx::ProfRec *r = prof_begin(c, gemv_bytes(2 * ffn, K, ffn), &prc);
        if (prc)
            return prc;
        return prof_end(c, r,
                        launch_rc(q48_launch_gemv_fused(c, out, Wgu, x, norm_w, nullptr, nullptr, 2 * ffn, K, 1, 2)));
    }
    int rc = tmp_reserve(c, ((size_t)K + 2 * (size_t)ffn) * 8);
    if (rc)
        return rc;
    int64_t *xn = (int64_t *)c->tmp, *t = xn + K;
    if ((rc = launch_rc(q48_launch_rmsnorm(c, xn, x, norm_w, K))) ||
        (rc = launch_rc(q48_launch_gemv(c, t, Wgu, xn, 2 * ffn, K))))
        return rc;
    return launch_rc(q48_launch_silu_mul(c, out, t, t + ffn, ffn));
}

int q48_attn_decode_rope(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                         int64_t *vcache, const int64_t *k_new, const int64_t *v_new, int layer,
                         int pos, int n_heads, int n_kv, int head_dim, int max_seq)
{
    return q48_attn_decode_rope_prefetch(c, out, q, kcache, vcache, k_new, v_new, layer, pos,
                                         n_heads, n_kv, head_dim, max_seq, nullptr, 0);
}

int q48_attn_split_min(void) { return q48_att_split_min(); }


int q48_attn_status(q48_ctx *c)
{
    if (!c)
        return Q48_EINVAL;
    if (c->capturing)
        return Q48_ESTATE;
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    if (!c->attg_unchecked)
        return Q48_OK;   // no k_attn_g launch since the words were last read
    const size_t off = q48_attn_sync_bytes() - 16 * sizeof(unsigned);   // the error word
    int e[2] = {0, 0};
    if (hipMemcpy(&e[0], (char *)c->attx_sync + off, sizeof(int), hipMemcpyDeviceToHost) !=
            hipSuccess ||
        (c->scratch_sync &&
         hipMemcpy(&e[1], (char *)c->scratch_sync + off, sizeof(int), hipMemcpyDeviceToHost) !=
             hipSuccess))
        return Q48_EHIP;
    c->attg_unchecked = 0;
    if (!e[0] && !e[1])
        return Q48_OK;
    // a timed-out launch left its exchange words behind: clear both regions
    int rc = launch_rc(q48_launch_zero(c, c->attx_sync, q48_attn_sync_bytes()));
    if (rc == Q48_OK && c->scratch_sync)
        rc = launch_rc(q48_launch_zero(c, c->scratch_sync, q48_attn_sync_bytes()));
    if (rc == Q48_OK)
        rc = hip_rc(hipStreamSynchronize(c->stream));
    if (rc == Q48_OK) {
        c->attg_count = 0;
        if (c->scratch_sync)
            *q48_scratch_attg_count(c->device) = 0;
    }
    return rc ? rc : Q48_ETIMEOUT;
}

int q48_set_attn_wait(q48_ctx *c, int64_t ticks)
{
    if (!c)
        return Q48_EINVAL;
    const uint64_t w = ticks < 0 ? q48_attg_default_wait() : (uint64_t)ticks;
    if (w != c->attg_wait) {
        c->attg_wait = w;
        ++c->stamp;   // a kernel argument of captured launches
    }
    return Q48_OK;
}

int q48_set_attn_one_launch(q48_ctx *c, int on)
{
    if (!c)
        return Q48_EINVAL;
    if (c->attn_one_launch != (on != 0))
        ++c->stamp;
    c->attn_one_launch = on != 0;
    return Q48_OK;
}

int q48_set_attn_g_mfma(q48_ctx *c, int on)
{
    if (!c)
        return Q48_EINVAL;
    if (c->attn_g_mfma != (on != 0))
        ++c->stamp;
    c->attn_g_mfma = on != 0;
    return Q48_OK;
}

int q48_set_pf_attn_mfma(q48_ctx *c, int on)
{
    if (!c)
        return Q48_EINVAL;
    c->pf_attn_mfma = on != 0;
    return Q48_OK;
}

int q48_set_gemv_persistent(q48_ctx *c, int on)
{
    if (!c)
        return Q48_EINVAL;
    if (c->gemv_persistent != (on != 0))
        ++c->stamp;
    c->gemv_persistent = on != 0;
    return Q48_OK;
}

int q48_attn_decode_rope_prefetch(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                                  int64_t *vcache, const int64_t *k_new, const int64_t *v_new,
                                  int layer, int pos, int n_heads, int n_kv, int head_dim,
                                  int max_seq, const void *prefetch, size_t prefetch_bytes)
{
    if (prefetch && ((uintptr_t)prefetch & 15))
        return Q48_EINVAL;
    if (!c || !out || !q || !kcache || !vcache || !k_new || !v_new)
        return Q48_EINVAL;
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || head_dim <= 0 ||
        head_dim > kMaxHeadDim || 256 % head_dim || head_dim % 8 || layer < 0 || max_seq <= 0)
        return Q48_EINVAL;
    if (!c->rope_cos || head_dim != c->rope_head_dim || max_seq > c->rope_max_seq)
        return Q48_ESTATE;
    if (pos < 0 || pos >= max_seq)
        return Q48_ERANGE;
    const int *dp = c->step_mode ? c->d_step + 1 : nullptr;
    int rc = q48_launch_attn_v2(c, out, q, kcache, vcache, k_new, v_new, layer, dp, pos, n_heads,
                                n_kv, head_dim, max_seq, 1, prefetch,
                                prefetch ? prefetch_bytes : 0);
    if (rc < 0)
        return rc;   // a Q48_E* code from the launcher (ENOMEM, EINVAL)
    return launch_rc(rc);
}


// ---- batched prefill rows -------------------------------------------------------

static bool heads_ok(int n_heads, int n_kv, int head_dim)
{
    return n_heads > 0 && n_kv > 0 && n_heads % n_kv == 0 &&
           (head_dim == 32 || head_dim == 64 || head_dim == 128);
}

int q48_embed_rows(q48_ctx *c, int64_t *H, const int64_t *table, const int *d_tokens, int T,
                   int dim)
{
    if (!c || !H || !table || !d_tokens || T <= 0 || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_pf_embed(c, H, table, d_tokens, T, dim));
}

int q48_rmsnorm_rows(q48_ctx *c, int64_t *out, const int64_t *X, const int64_t *w, int T,
                     int dim)
{
    if (!c || !out || !X || !w || T <= 0 || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_pf_rmsnorm(c, out, X, w, T, dim));
}

int q48_rope_store_rows(q48_ctx *c, int64_t *QKV, int64_t *kcache, int64_t *vcache, int layer,
                        int p0, int T, int n_heads, int n_kv, int head_dim, int max_seq)
{
    if (!c || !QKV || !kcache || !vcache || T <= 0 || layer < 0 || max_seq <= 0 ||
        !heads_ok(n_heads, n_kv, head_dim))
        return Q48_EINVAL;
    if (!c->rope_cos || head_dim != c->rope_head_dim || max_seq > c->rope_max_seq)
        return Q48_ESTATE;
    if (p0 < 0 || p0 + T > max_seq)
        return Q48_ERANGE;
    return launch_rc(q48_launch_pf_rope_store(c, QKV, kcache, vcache, layer, p0, T, n_heads,
                                              n_kv, head_dim, max_seq));
}

int q48_attn_prefill(q48_ctx *c, int64_t *out, const int64_t *QKV, int64_t *kcache,
                     int64_t *vcache, int layer, int p0, int T, int n_heads, int n_kv,
                     int head_dim, int max_seq)
{
    if (!c || !out || !QKV || !kcache || !vcache || T <= 0 || layer < 0 || max_seq <= 0 ||
        !heads_ok(n_heads, n_kv, head_dim))
        return Q48_EINVAL;
    if (!c->rope_cos || head_dim != c->rope_head_dim || max_seq > c->rope_max_seq)
        return Q48_ESTATE;
    if (p0 < 0 || p0 + T > max_seq)
        return Q48_ERANGE;
    if (c->pf_attn_mfma && q48_pf_attn_mfma_ok(p0, T, head_dim))
        return launch_rc(q48_launch_pf_attn_mfma(c, out, QKV, kcache, vcache, layer, p0, T,
                                                 n_heads, n_kv, head_dim, max_seq));
    if (p0 + T > q48_att_lds_max())
        return Q48_ERANGE;
    return launch_rc(q48_launch_pf_attn(c, out, QKV, kcache, vcache, layer, p0, T, n_heads, n_kv,
                                        head_dim, max_seq));
}

int q48_silu_mul_rows(q48_ctx *c, int64_t *out, const int64_t *GU, int T, int ffn)
{
    if (!c || !out || !GU || T <= 0 || ffn <= 0 || ffn > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_pf_silu(c, out, GU, T, ffn));
}

// ---- norm statistics computed once per vector ---------------------------------

int q48_rms_inv(q48_ctx *c, int64_t *r_out, const int64_t *x, int dim)
{
    if (!c || !r_out || !x || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_rms_inv(c, r_out, nullptr, x, nullptr, nullptr, 0, dim));
}

int q48_embed_rms(q48_ctx *c, int64_t *out, const int64_t *table, int token, int dim,
                  int64_t *r_out)
{
    if (!c || !out || !table || !r_out || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    if (token < 0)
        return Q48_ERANGE;
    return launch_rc(q48_launch_rms_inv(c, r_out, out, nullptr, table,
                                        c->step_mode ? c->d_step : nullptr, token, dim));
}

int q48_norm_gemv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                  const int64_t *norm_w, const int64_t *r, int M, int K)
{
    if (!c || bad_ptrs(y, W, x) || !norm_w || !r || M <= 0 || K <= 0 || M > kMaxDim ||
        K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(W, K)) {
        int prc;
        q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(M, K, M), &prc);
        if (prc)
            return prc;
        return prof_end(c, pr, launch_rc(q48_launch_gemv_fused(c, y, W, x, norm_w, r, nullptr,
                                                               M, K, 2, 0)));
    }
    int rc = tmp_reserve(c, (size_t)K * 8);
    if (rc)
        return rc;
    int64_t *t = (int64_t *)c->tmp;
    rc = launch_rc(q48_launch_rms_apply(c, t, x, norm_w, r, K));
    return rc ? rc : launch_rc(q48_launch_gemv(c, y, W, t, M, K));
}

int q48_norm_gemv_swiglu(q48_ctx *c, int64_t *out, const int64_t *Wgu, const int64_t *x,
                         const int64_t *norm_w, const int64_t *r, int ffn, int K)
{
    if (!c || bad_ptrs(out, Wgu, x) || !norm_w || !r || ffn <= 0 || K <= 0 ||
        ffn > kMaxDim / 2 || K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(Wgu, K)) {
        int prc;
        q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(2 * ffn, K, ffn), &prc);
        if (prc)
            return prc;
        return prof_end(c, pr, launch_rc(q48_launch_gemv_fused(c, out, Wgu, x, norm_w, r,
                                                               nullptr, 2 * ffn, K, 2, 2)));
    }
    int rc = tmp_reserve(c, ((size_t)K + 2 * (size_t)ffn) * 8);
    if (rc)
        return rc;
    int64_t *xn = (int64_t *)c->tmp, *t = xn + K;
    if ((rc = launch_rc(q48_launch_rms_apply(c, xn, x, norm_w, r, K))) ||
        (rc = launch_rc(q48_launch_gemv(c, t, Wgu, xn, 2 * ffn, K))))
        return rc;
    return launch_rc(q48_launch_silu_mul(c, out, t, t + ffn, ffn));
}

int q48_gemv_residual_rms(q48_ctx *c, int64_t *acc, const int64_t *W, const int64_t *x, int M,
                          int K, int64_t *r_out)
{
    if (!c || bad_ptrs(acc, W, x) || !r_out || M <= 0 || K <= 0 || M > kMaxDim ||
        K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(W, K)) {
        int prc;
        q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(M, K, M), &prc);
        if (prc)
            return prc;
        int rc = q48_launch_gemv_fused(c, acc, W, x, nullptr, nullptr, r_out, M, K, 0, 3);
        if (rc == Q48_ENOMEM || rc == Q48_ESTATE || rc == Q48_EHIP)
            return rc;
        return prof_end(c, pr, launch_rc(rc));
    }
    int rc = tmp_reserve(c, (size_t)M * 8);
    if (rc)
        return rc;
    int64_t *t = (int64_t *)c->tmp;
    if ((rc = launch_rc(q48_launch_gemv(c, t, W, x, M, K))) ||
        (rc = launch_rc(q48_launch_add(c, acc, t, M))))
        return rc;
    return launch_rc(q48_launch_rms_inv(c, r_out, nullptr, acc, nullptr, nullptr, 0, M));
}

int q48_rms_stats(q48_ctx *c, int64_t *stats, const int64_t *x, int dim)
{
    if (!c || !stats || !x || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    return launch_rc(q48_launch_rms_stats(c, stats, nullptr, x, nullptr, nullptr, 0, dim));
}

int q48_embed_stats(q48_ctx *c, int64_t *out, const int64_t *table, int token, int dim,
                    int64_t *stats)
{
    if (!c || !out || !table || !stats || dim <= 0 || dim > kMaxDim)
        return Q48_EINVAL;
    if (token < 0)
        return Q48_ERANGE;
    return launch_rc(q48_launch_rms_stats(c, stats, out, nullptr, table,
                                          c->step_mode ? c->d_step : nullptr, token, dim));
}

// r from the partial sums into the context's scratch word (the fallbacks)
static int stats_to_r(q48_ctx *c, const int64_t *stats, int dim, int64_t **r)
{
    *r = (int64_t *)(c->d_scalar + 16);   // bytes 64..71: clear of the argmax slot
    return launch_rc(q48_launch_stats_r(c, *r, stats, dim));
}

int q48_norm_gemv_stats(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                        const int64_t *norm_w, const int64_t *stats, int M, int K)
{
    if (!c || bad_ptrs(y, W, x) || !norm_w || !stats || M <= 0 || K <= 0 || M > kMaxDim ||
        K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(W, K)) {
        int prc;
        q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(M, K, M), &prc);
        if (prc)
            return prc;
        return prof_end(c, pr, launch_rc(q48_launch_gemv_fused(c, y, W, x, norm_w, stats,
                                                               nullptr, M, K, 3, 0)));
    }
    int64_t *r;
    int rc = stats_to_r(c, stats, K, &r);
    return rc ? rc : q48_norm_gemv(c, y, W, x, norm_w, r, M, K);
}

int q48_norm_gemv_swiglu_stats(q48_ctx *c, int64_t *out, const int64_t *Wgu, const int64_t *x,
                               const int64_t *norm_w, const int64_t *stats, int ffn, int K)
{
    if (!c || bad_ptrs(out, Wgu, x) || !norm_w || !stats || ffn <= 0 || K <= 0 ||
        ffn > kMaxDim / 2 || K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(Wgu, K)) {
        int prc;
        q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(2 * ffn, K, ffn), &prc);
        if (prc)
            return prc;
        return prof_end(c, pr, launch_rc(q48_launch_gemv_fused(c, out, Wgu, x, norm_w, stats,
                                                               nullptr, 2 * ffn, K, 3, 2)));
    }
    int64_t *r;
    int rc = stats_to_r(c, stats, K, &r);
    return rc ? rc : q48_norm_gemv_swiglu(c, out, Wgu, x, norm_w, r, ffn, K);
}

int q48_gemv_residual_stats(q48_ctx *c, int64_t *acc, const int64_t *W, const int64_t *x,
                            int M, int K, int64_t *stats)
{
    if (!c || bad_ptrs(acc, W, x) || !stats || M <= 0 || K <= 0 || M > kMaxDim || K > kMaxDim)
        return Q48_EINVAL;
    if (q48_gemv_v2_ok(W, K)) {
        int prc;
        q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(M, K, M), &prc);
        if (prc)
            return prc;
        return prof_end(c, pr, launch_rc(q48_launch_gemv_fused(c, acc, W, x, nullptr, nullptr,
                                                               stats, M, K, 0, 4)));
    }
    int rc = q48_gemv_residual(c, acc, W, x, M, K);
    return rc ? rc : launch_rc(q48_launch_rms_stats(c, stats, nullptr, acc, nullptr, nullptr, 0, M));
}

// ---- decode-step state and graphs --------------------------------------------

int q48_step_mode(q48_ctx *c, int on)
{
    if (!c)
        return Q48_EINVAL;
    c->step_mode = on != 0;
    return Q48_OK;
}

int q48_step_set(q48_ctx *c, int token, int pos)
{
    if (!c || token < 0 || pos < 0)
        return Q48_EINVAL;
    return launch_rc(q48_launch_step_set(c, token, pos));
}

int q48_step_get(q48_ctx *c, int *token, int *pos, int *count)
{
    if (!c)
        return Q48_EINVAL;
    if (c->capturing)
        return Q48_ESTATE;
    int st[4];
    if (hipMemcpyAsync(st, c->d_step, 4 * sizeof(int), hipMemcpyDeviceToHost, c->stream) !=
            hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    if (token)
        *token = st[0];
    if (pos)
        *pos = st[1];
    if (count)
        *count = st[2];
    return Q48_OK;
}

int q48_argmax_step(q48_ctx *c, const int64_t *v, int n, int *d_tokens, int cap)
{
    if (!c || !v || n <= 0 || cap < 0 || (cap > 0 && !d_tokens))
        return Q48_EINVAL;
    return launch_rc(q48_launch_step_argmax(c, d_tokens, cap, v, n, nullptr, 0));
}

int q48_argmax_record_step(q48_ctx *c, const int64_t *v, int n, int *d_tokens, int cap,
                           int64_t *rec, int rec_cap)
{
    if (!c || !v || n <= 0 || cap < 0 || (cap > 0 && !d_tokens) || !rec || rec_cap <= 0)
        return Q48_EINVAL;
    return launch_rc(q48_launch_step_argmax(c, d_tokens, cap, v, n, rec, rec_cap));
}

int q48_record_step(q48_ctx *c, const int64_t *v, int n, int64_t *rec, int cap)
{
    if (!c || !v || !rec || n <= 0 || cap <= 0)
        return Q48_EINVAL;
    return launch_rc(q48_launch_step_record(c, rec, cap, v, n));
}

void q48_rng_seed(uint64_t seed, uint64_t state[2])
{
    // rng_seed, llama_int.c:2909-2920: SplitMix64 of seed and of
    // seed + 0x9E3779B97F4A7C15; an all-zero state becomes (1, 0)
    auto mix = [](uint64_t z) {
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    if (!state)
        return;
    state[0] = mix(seed);
    state[1] = mix(seed + 0x9E3779B97F4A7C15ull);
    if (state[0] == 0 && state[1] == 0)
        state[0] = 1;
}

int q48_sample_reserve(q48_ctx *c, int vocab)
{
    if (!c || vocab <= 0)
        return Q48_EINVAL;
    const size_t words = q48_sample_ws_words(vocab);
    if (words <= c->smp_words)
        return Q48_OK;
    if (c->capturing)
        return Q48_ESTATE;
    if (c->smp) {
        int rc = q48_release(c, c->smp);
        if (rc)
            return rc;
        c->smp = nullptr;
        c->smp_words = 0;
    }
    if (hipMalloc(&c->smp, words * sizeof(int64_t)) != hipSuccess)
        return Q48_ENOMEM;
    c->smp_words = words;
    return Q48_OK;
}

// greedy below a temperature of 0.01 (llama_int.c:2962-2964)
static bool sample_greedy(int64_t temperature)
{
    return temperature <= 0 || temperature < ((int64_t)1 << 48) / 100;
}

int q48_sample(q48_ctx *c, const int64_t *logits, int vocab, int64_t temperature, int top_k,
               int64_t top_p, uint64_t *rng, int *token)
{
    if (!c || !logits || vocab <= 0 || !token || (!rng && !sample_greedy(temperature)))
        return Q48_EINVAL;
    if (c->capturing)
        return Q48_ESTATE;
    if (sample_greedy(temperature))
        return q48_argmax(c, logits, vocab, token);
    int rc = q48_sample_reserve(c, vocab);
    if (rc)
        return rc;
    rc = launch_rc(q48_launch_sample(c, c->smp, logits, vocab, temperature, top_k, top_p, rng,
                                     c->d_scalar, nullptr, 0));
    if (rc)
        return rc;
    if (hipMemcpyAsync(token, c->d_scalar, sizeof(int), hipMemcpyDeviceToHost, c->stream) !=
        hipSuccess)
        return Q48_EHIP;
    return hip_rc(hipStreamSynchronize(c->stream));
}

int q48_sample_step(q48_ctx *c, const int64_t *logits, int vocab, int64_t temperature,
                    int top_k, int64_t top_p, uint64_t *rng, int *d_tokens, int cap)
{
    if (!c || !logits || vocab <= 0 || cap < 0 || !d_tokens ||
        (!rng && !sample_greedy(temperature)))
        return Q48_EINVAL;
    if (sample_greedy(temperature))
        return q48_argmax_step(c, logits, vocab, d_tokens, cap);
    int rc = q48_sample_reserve(c, vocab);
    if (rc)
        return rc;
    return launch_rc(q48_launch_sample(c, c->smp, logits, vocab, temperature, top_k, top_p, rng,
                                       nullptr, d_tokens, cap));
}

namespace {
void graph_destroy(q48_ctx *c, q48_graph *g)
{
    if (!g)
        return;
    // launches of the graph may still be in flight on the stream
    (void)hipStreamSynchronize(c->stream);
    if (g->x)
        (void)hipGraphExecDestroy(g->x);
    if (g->g)
        (void)hipGraphDestroy(g->g);
    delete g;
    if (--c->n_graphs == 0)
        free_retired(c);
}

// End the capture in progress into a new executable graph.
int graph_finish(q48_ctx *c, q48_graph **out)
{
    c->capturing = 0;
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(c->stream, &g) != hipSuccess || !g)
        return Q48_EHIP;
    q48_graph *h = new (std::nothrow) q48_graph();
    if (!h) {
        (void)hipGraphDestroy(g);
        return Q48_ENOMEM;
    }
    h->g = g;
    h->attg[0] = c->capture_attg[0];
    h->attg[1] = c->capture_attg[1];
    if (hipGraphInstantiate(&h->x, g, nullptr, nullptr, 0) != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete h;
        return Q48_EHIP;
    }
    // the executable graph's device-side setup now, not inside the first launch
    if (hipGraphUpload(h->x, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess) {
        (void)hipGraphExecDestroy(h->x);
        (void)hipGraphDestroy(g);
        delete h;
        return Q48_EHIP;
    }
    ++c->n_graphs;
    *out = h;
    return Q48_OK;
}

int graph_replay(q48_ctx *c, q48_graph *g, int times)
{
    // one replay at a time, each counted on the exchange regions its
    // k_attn_g launches use
    for (int i = 0; i < times; ++i) {
        if (g->attg[0]) {
            int rc = q48_attg_account(c, c->attx_sync, g->attg[0]);
            if (rc)
                return rc;
        }
        if (g->attg[1]) {
            int rc = q48_attg_account(c, c->scratch_sync, g->attg[1]);
            if (rc)
                return rc;
        }
        if (hipGraphLaunch(g->x, c->stream) != hipSuccess)
            return Q48_EHIP;
    }
    return Q48_OK;
}
} // namespace

int q48_graph_begin(q48_ctx *c)
{
    if (!c || c->capturing)
        return Q48_EINVAL;
    graph_destroy(c, c->cur);
    c->cur = nullptr;
    return q48_graph_capture(c);
}

int q48_graph_capture(q48_ctx *c)
{
    if (!c || c->capturing)
        return Q48_EINVAL;
    if (hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
        return Q48_EHIP;
    c->capturing = 1;
    c->capture_attg[0] = c->capture_attg[1] = 0;
    return Q48_OK;
}

int q48_graph_end(q48_ctx *c)
{
    if (!c || !c->capturing)
        return Q48_EINVAL;
    graph_destroy(c, c->cur);
    c->cur = nullptr;
    return graph_finish(c, &c->cur);
}

int q48_graph_instantiate(q48_ctx *c, q48_graph **out)
{
    if (!c || !c->capturing || !out)
        return Q48_EINVAL;
    *out = nullptr;
    return graph_finish(c, out);
}

int q48_graph_launch(q48_ctx *c, int times)
{
    if (!c || times < 0 || c->capturing)
        return Q48_EINVAL;
    if (!c->cur)
        return Q48_ESTATE;
    return graph_replay(c, c->cur, times);
}

int q48_graph_replay(q48_ctx *c, q48_graph *g, int times)
{
    if (!c || !g || times < 0 || c->capturing)
        return Q48_EINVAL;
    return graph_replay(c, g, times);
}

int q48_graph_drop(q48_ctx *c)
{
    if (!c || c->capturing)
        return Q48_EINVAL;
    graph_destroy(c, c->cur);
    c->cur = nullptr;
    return Q48_OK;
}

int q48_graph_destroy(q48_ctx *c, q48_graph *g)
{
    if (!c || c->capturing)
        return Q48_EINVAL;
    if (g == c->cur)
        c->cur = nullptr;
    graph_destroy(c, g);
    return Q48_OK;
}

uint64_t q48_graph_stamp(const q48_ctx *c) { return c ? c->stamp : 0; }

} // extern "C"

/* ---- bfloat16-resident weights ------------------------------------------ */

namespace {
double gemv_bytes_bf16(int M, int K, int out)
{
    return 2.0 * (double)M * K + 8.0 * ((double)K + out);
}
// x, norm_w, stats 16-byte aligned, W 16-byte aligned, K a multiple of 512
bool bad_bf16(const void *y, const void *W, const void *x, const void *nw, const void *st, int K)
{
    return !y || !W || !x || ((uintptr_t)y & 7) || ((uintptr_t)W & 15) || ((uintptr_t)x & 15) ||
           (nw && ((uintptr_t)nw & 15)) || (st && ((uintptr_t)st & 15)) || !q48_gemv_bf16_ok(K);
}
int bf16_fused(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
               const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M, int K, int pro,
               int epi, double bytes)
{
    int prc;
    q48_ctx::ProfRec *pr = prof_begin(c, bytes, &prc);
    if (prc)
        return prc;
    const int rc = q48_launch_gemv_fused_bf16(c, y, W, x, norm_w, r_in, r_out, M, K, pro, epi);
    return prof_end(c, pr, rc < 0 ? Q48_EINVAL : launch_rc(rc));
}
} // namespace

int q48_bf16_pack(q48_ctx *c, uint16_t *out, const int64_t *in, size_t n, int *inexact)
{
    if (!c || !out || !in || !inexact || ((uintptr_t)in & 7) || ((uintptr_t)out & 1))
        return Q48_EINVAL;
    int *flag = c->d_scalar + 40;
    int rc = launch_rc(q48_launch_zero(c, flag, sizeof(int)));
    if (rc)
        return rc;
    if (n) {
        rc = launch_rc(q48_launch_bf16_pack(c, out, in, n, flag));
        if (rc)
            return rc;
    }
    int f = 0;
    if (hipMemcpyAsync(&f, flag, sizeof(int), hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return Q48_EHIP;
    *inexact = f != 0;
    return Q48_OK;
}

int q48_gemv_bf16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x, int M, int K)
{
    if (!c || bad_bf16(y, W, x, nullptr, nullptr, K) || M <= 0 || M > kMaxDim)
        return Q48_EINVAL;
    return bf16_fused(c, y, W, x, nullptr, nullptr, nullptr, M, K, 0, 0, gemv_bytes_bf16(M, K, M));
}

int q48_norm_gemv_stats_bf16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                             const int64_t *norm_w, const int64_t *stats, int M, int K)
{
    if (!c || !norm_w || !stats || bad_bf16(y, W, x, norm_w, stats, K) || M <= 0 ||
        M > kMaxDim)
        return Q48_EINVAL;
    return bf16_fused(c, y, W, x, norm_w, stats, nullptr, M, K, 3, 0, gemv_bytes_bf16(M, K, M));
}

int q48_norm_gemv_swiglu_stats_bf16(q48_ctx *c, int64_t *out, const uint16_t *Wgu,
                                    const int64_t *x, const int64_t *norm_w,
                                    const int64_t *stats, int ffn, int K)
{
    if (!c || !norm_w || !stats || bad_bf16(out, Wgu, x, norm_w, stats, K) || ffn <= 0 ||
        ffn > kMaxDim / 2)
        return Q48_EINVAL;
    return bf16_fused(c, out, Wgu, x, norm_w, stats, nullptr, 2 * ffn, K, 3, 2,
                      gemv_bytes_bf16(2 * ffn, K, ffn));
}

int q48_gemv_residual_stats_bf16(q48_ctx *c, int64_t *acc, const uint16_t *W, const int64_t *x,
                                 int M, int K, int64_t *stats)
{
    if (!c || !stats || bad_bf16(acc, W, x, nullptr, stats, K) || M <= 0 || M > kMaxDim)
        return Q48_EINVAL;
    return bf16_fused(c, acc, W, x, nullptr, nullptr, stats, M, K, 0, 4,
                      gemv_bytes_bf16(M, K, M));
}


// ---- projection with RoPE + KV store, attention over the cache ---------------

namespace {
// Shape and state checks shared by the two q48_norm_gemv_rope_kv forms.
int rope_kv_args(q48_ctx *c, int64_t *kcache, int64_t *vcache, int layer, int pos, int n_heads,
                 int n_kv, int head_dim, int max_seq, int K, q48_ropekv *rk, int *M)
{
    if (!kcache || !vcache || !heads_ok(n_heads, n_kv, head_dim) || layer < 0 ||
        max_seq <= 0 || K <= 0 || K > kMaxDim ||
        (long long)(n_heads + 2LL * n_kv) * head_dim > kMaxDim)
        return Q48_EINVAL;
    if (!c->rope_cos || head_dim != c->rope_head_dim || max_seq > c->rope_max_seq)
        return Q48_ESTATE;
    if (pos < 0 || pos >= max_seq)
        return Q48_ERANGE;
    *rk = q48_ropekv{kcache, vcache, c->rope_cos, c->rope_sin,
                     c->step_mode ? c->d_step + 1 : nullptr, pos, layer, max_seq, n_heads,
                     n_kv, head_dim};
    *M = (n_heads + 2 * n_kv) * head_dim;
    return Q48_OK;
}
} // namespace

int q48_norm_gemv_rope_kv(q48_ctx *c, int64_t *qkv, const int64_t *W, const int64_t *x,
                          const int64_t *norm_w, const int64_t *stats, int64_t *kcache,
                          int64_t *vcache, int layer, int pos, int n_heads, int n_kv,
                          int head_dim, int max_seq, int K)
{
    if (!c || bad_ptrs(qkv, W, x) || !norm_w || !stats || !q48_gemv_v2_ok(W, K))
        return Q48_EINVAL;
    q48_ropekv rk;
    int M;
    int rc = rope_kv_args(c, kcache, vcache, layer, pos, n_heads, n_kv, head_dim, max_seq, K,
                          &rk, &M);
    if (rc)
        return rc;
    int prc;
    q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes(M, K, M), &prc);
    if (prc)
        return prc;
    return prof_end(c, pr,
                    launch_rc(q48_launch_gemv_rope_kv(c, qkv, W, x, norm_w, stats, &rk, M, K)));
}

int q48_norm_gemv_rope_kv_bf16(q48_ctx *c, int64_t *qkv, const uint16_t *W, const int64_t *x,
                               const int64_t *norm_w, const int64_t *stats, int64_t *kcache,
                               int64_t *vcache, int layer, int pos, int n_heads, int n_kv,
                               int head_dim, int max_seq, int K)
{
    if (!c || !norm_w || !stats || bad_bf16(qkv, W, x, norm_w, stats, K))
        return Q48_EINVAL;
    q48_ropekv rk;
    int M;
    int rc = rope_kv_args(c, kcache, vcache, layer, pos, n_heads, n_kv, head_dim, max_seq, K,
                          &rk, &M);
    if (rc)
        return rc;
    int prc;
    q48_ctx::ProfRec *pr = prof_begin(c, gemv_bytes_bf16(M, K, M), &prc);
    if (prc)
        return prc;
    const int lrc = q48_launch_gemv_rope_kv_bf16(c, qkv, W, x, norm_w, stats, &rk, M, K);
    return prof_end(c, pr, lrc < 0 ? Q48_EINVAL : launch_rc(lrc));
}

int q48_attn_decode_cached(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                           int64_t *vcache, int layer, int pos, int n_heads, int n_kv,
                           int head_dim, int max_seq, const void *prefetch,
                           size_t prefetch_bytes)
{
    if (!c || !out || !q || !kcache || !vcache || !heads_ok(n_heads, n_kv, head_dim) ||
        layer < 0 || max_seq <= 0 || max_seq > q48_att_lds_max() ||
        (prefetch && ((uintptr_t)prefetch & 15)))
        return Q48_EINVAL;
    // the score scale lives after the sine table
    if (!c->rope_cos || head_dim != c->rope_head_dim || max_seq > c->rope_max_seq)
        return Q48_ESTATE;
    if (pos < 0 || pos >= max_seq)
        return Q48_ERANGE;
    const int *dp = c->step_mode ? c->d_step + 1 : nullptr;
    return launch_rc(q48_launch_attn_cached(c, out, q, kcache, vcache, layer, dp, pos, n_heads,
                                            n_kv, head_dim, max_seq, prefetch,
                                            prefetch ? prefetch_bytes : 0));
}
