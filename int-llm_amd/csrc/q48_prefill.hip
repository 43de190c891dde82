// q48_prefill.hip — the per-token ops of the layer (llama_int.c:1326-1569)
// over T tokens at once, for a batched prefill whose projections are
// q48_gemm: embedding rows, RoPE + KV store rows, causal attention of T
// queries, SwiGLU rows (rmsnorm rows are q48_ops.hip's kernel, one block per
// row).  Each token's arithmetic is the
// reference's for that token at its position; the attention of token t
// reads the cache rows 0 .. p0 + t, all stored before it runs, so the
// results and the cache equal T sequential forward calls bit for bit.
#include "q48_internal.h"
#include "q48_attn.hpp"

namespace {

// hidden[t] = embed_tokens[tokens[t]] (llama_int.c:2822-2824)
__global__ __launch_bounds__(256) void k_pf_embed(int64_t *__restrict__ H,
                                                 const int64_t *__restrict__ table,
                                                 const int *__restrict__ tokens, int dim)
{
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i < dim)
        H[(size_t)t * dim + i] = table[(size_t)tokens[t] * dim + i];
}

// rope_apply (llama_int.c:997-1008) of the q heads and k heads of row t at
// position p0 + t, in place, then the KV store (1414-1416) of the rotated k
// and of v.  Row layout [q (nh hd) | k (nkv hd) | v (nkv hd)].
__global__ __launch_bounds__(256) void k_pf_rope_store(
    int64_t *__restrict__ QKV, int64_t *__restrict__ kcache, int64_t *__restrict__ vcache,
    const int64_t *__restrict__ cos_t, const int64_t *__restrict__ sin_t, int layer, int p0,
    int n_heads, int n_kv, int hd, int max_seq)
{
    const int t = blockIdx.x, pos = p0 + t, half = hd / 2;
    const size_t kvd = (size_t)n_kv * hd, row = (size_t)(n_heads + 2 * n_kv) * hd;
    int64_t *q = QKV + (size_t)t * row, *k = q + (size_t)n_heads * hd, *v = k + kvd;
    const size_t cr = ((size_t)layer * max_seq + pos) * kvd;
    for (int idx = threadIdx.x; idx < (n_heads + n_kv) * half; idx += 256) {
        const int h = idx / half, i = idx % half;
        int64_t *vec = q + (size_t)h * hd;   // k heads follow the q heads
        const int64_t c = cos_t[(size_t)pos * half + i];
        const int64_t s = sin_t[(size_t)pos * half + i];
        const int64_t x0 = vec[i], x1 = vec[i + half];
        const int64_t y0 = (int64_t)((uint64_t)q48_mul(x0, c) - (uint64_t)q48_mul(x1, s));
        const int64_t y1 = (int64_t)((uint64_t)q48_mul(x1, c) + (uint64_t)q48_mul(x0, s));
        vec[i] = y0;
        vec[i + half] = y1;
        if (h >= n_heads) {
            const size_t o = (size_t)(h - n_heads) * hd;
            kcache[cr + o + i] = y0;
            kcache[cr + o + i + half] = y1;
        }
    }
    for (int j = threadIdx.x; j < (int)kvd; j += 256)
        vcache[cr + j] = v[j];
}

// causal attention of query row t (position p0 + t), head blockIdx.x
template <int HD>
__global__ __launch_bounds__(256) void k_pf_attn(int64_t *__restrict__ out,
                                                const int64_t *__restrict__ QKV,
                                                int64_t *__restrict__ kcache,
                                                int64_t *__restrict__ vcache,
                                                const int64_t *__restrict__ scale_p, int layer,
                                                int p0, int n_heads, int n_kv, int max_seq)
{
    const int t = blockIdx.y;
    const size_t row = (size_t)(n_heads + 2 * n_kv) * HD;
    attn_v3_head<HD, ATT_LDS_MAX, false, true>(
        out + (size_t)t * n_heads * HD, QKV + (size_t)t * row, kcache, vcache, nullptr, nullptr,
        nullptr, nullptr, scale_p, layer, nullptr, p0 + t, n_heads, n_kv, max_seq,
        (int)blockIdx.x);
}

// SwiGLU (llama_int.c:1549-1552) of row t: out = fp_mul(fp_silu(gate), up)
// with the row [gate (ffn) | up (ffn)]
__global__ __launch_bounds__(256) void k_pf_silu(int64_t *__restrict__ out,
                                                const int64_t *__restrict__ GU, int ffn)
{
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i < ffn) {
        const int64_t *g = GU + (size_t)t * 2 * ffn;
        out[(size_t)t * ffn + i] = q48_mul(q48_silu(g[i]), g[ffn + i]);
    }
}

} // namespace

int q48_launch_pf_embed(q48_ctx *c, int64_t *H, const int64_t *table, const int *tokens, int T,
                        int dim)
{
    hipLaunchKernelGGL(k_pf_embed, dim3((dim + 255) / 256, T), dim3(256), 0, c->stream, H, table,
                       tokens, dim);
    return (int)hipGetLastError();
}

int q48_launch_pf_rope_store(q48_ctx *c, int64_t *QKV, int64_t *kcache, int64_t *vcache,
                             int layer, int p0, int T, int n_heads, int n_kv, int hd,
                             int max_seq)
{
    hipLaunchKernelGGL(k_pf_rope_store, dim3(T), dim3(256), 0, c->stream, QKV, kcache, vcache,
                       c->rope_cos, c->rope_sin, layer, p0, n_heads, n_kv, hd, max_seq);
    return (int)hipGetLastError();
}

int q48_launch_pf_attn(q48_ctx *c, int64_t *out, const int64_t *QKV, int64_t *kcache,
                       int64_t *vcache, int layer, int p0, int T, int n_heads, int n_kv, int hd,
                       int max_seq)
{
    const int64_t *scale_p = c->rope_sin + (size_t)c->rope_max_seq * (c->rope_head_dim / 2);
    const dim3 grid(n_heads, T);
    if (hd == 64)
        hipLaunchKernelGGL(k_pf_attn<64>, grid, dim3(256), 0, c->stream, out, QKV, kcache, vcache,
                           scale_p, layer, p0, n_heads, n_kv, max_seq);
    else if (hd == 32)
        hipLaunchKernelGGL(k_pf_attn<32>, grid, dim3(256), 0, c->stream, out, QKV, kcache, vcache,
                           scale_p, layer, p0, n_heads, n_kv, max_seq);
    else
        hipLaunchKernelGGL(k_pf_attn<128>, grid, dim3(256), 0, c->stream, out, QKV, kcache,
                           vcache, scale_p, layer, p0, n_heads, n_kv, max_seq);
    return (int)hipGetLastError();
}

int q48_launch_pf_silu(q48_ctx *c, int64_t *out, const int64_t *GU, int T, int ffn)
{
    hipLaunchKernelGGL(k_pf_silu, dim3((ffn + 255) / 256, T), dim3(256), 0, c->stream, out, GU,
                       ffn);
    return (int)hipGetLastError();
}
