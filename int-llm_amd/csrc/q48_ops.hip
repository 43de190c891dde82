// q48_ops.hip — the non-GEMV ops of the Q16.48 layer on gfx950:
// RMSNorm, RoPE (tables + rotation), exact GQA decode attention with its
// fixed-point softmax, SwiGLU, residual add, embedding row, argmax, the
// fp_math constant init and an element-wise fp_math evaluator.
//
// Every output is bit-identical to llama_int.c (cited per kernel): all
// arithmetic is integer, and every reduction is an integer sum (mod 2^64
// or 2^128) or a max, so the parallel order cannot change a bit.
#include "q48_internal.h"

#include "q48_attn.hpp"
#include "q48_digits.hpp"

namespace {

// ---------------------------------------------------------------------------
// fp_math_init on the device (fp_math.h:833-858)
// ---------------------------------------------------------------------------
__global__ void k_math_init(q48_consts *k)
{
    if (threadIdx.x == 0 && blockIdx.x == 0)
        q48_math_init(k);
}

// ---------------------------------------------------------------------------
// rmsnorm, llama_int.c:1048-1058.  One block of 256 threads.
//   ss = sum (int128) x^2;  ms = (int64)((ss >> 48) / dim) + 2814749767
//   r = fp_inv_sqrt(ms);    out[i] = fp_mul(fp_mul(x[i], r), w[i])
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(int64_t *__restrict__ out,
                                                const int64_t *__restrict__ x,
                                                const int64_t *__restrict__ w,
                                                int dim)
{
    __shared__ uint64_t red_lo[4], red_hi[4];
    __shared__ int64_t r_sh;
    const int tid = threadIdx.x;
    x += (size_t)blockIdx.x * dim;   // one row per block
    out += (size_t)blockIdx.x * dim;
    q48_u128 ss = 0;
    for (int i = tid; i < dim; i += 256) {
        int64_t v = x[i];
        ss += (q48_u128)q48_smul128(v, v);
    }
    ss = q48_wave_sum128(ss);
    if ((tid & 63) == 0) {
        red_lo[tid >> 6] = (uint64_t)ss;
        red_hi[tid >> 6] = (uint64_t)(ss >> 64);
    }
    __syncthreads();
    if (tid == 0) {
        q48_u128 t = 0;
        for (int i = 0; i < 4; ++i)
            t += ((q48_u128)red_hi[i] << 64) | red_lo[i];
        int64_t ms = (int64_t)q48_divs_128_64((q48_i128)t >> 48, (int64_t)dim);
        ms = (int64_t)((uint64_t)ms + 2814749767ull);
        r_sh = q48_inv_sqrt(ms);
    }
    __syncthreads();
    const int64_t r = r_sh;
    for (int i = tid; i < dim; i += 256)
        out[i] = q48_mul(q48_mul(x[i], r), w[i]);
}

// ---------------------------------------------------------------------------
// rope_init, llama_int.c:960-986.  One thread per (pos, i < half).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope_init(int64_t *__restrict__ cos_t,
                                                  int64_t *__restrict__ sin_t,
                                                  const q48_consts *__restrict__ k,
                                                  int head_dim, int max_seq, int theta)
{
    const int half = head_dim / 2;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)half * max_seq)
        return;
    const int pos = (int)(idx / half), i = (int)(idx % half);
    const int64_t lt = q48_log(q48_from_int(theta));
    const int64_t nf = (int64_t)(0 - (uint64_t)q48_div(q48_from_int(2 * i), q48_from_int(head_dim)));
    const int64_t th = q48_exp(q48_mul(nf, lt));
    int64_t c, s;
    q48_sincos(k, q48_mul(q48_from_int(pos), th), &c, &s);
    cos_t[idx] = c;
    sin_t[idx] = s;
    if (idx == 0)   // the attention score scale, stored after the sine table
        sin_t[(size_t)half * max_seq] = q48_inv_sqrt(q48_from_int(head_dim));
}

// ---------------------------------------------------------------------------
// rope_apply, llama_int.c:997-1008, over n_heads heads of one vector.
// pos comes from device memory when d_pos != nullptr (graph replay).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope(int64_t *__restrict__ vec,
                                             const int64_t *__restrict__ cos_t,
                                             const int64_t *__restrict__ sin_t,
                                             int n_heads, int head_dim,
                                             const int *__restrict__ d_pos, int pos,
                                             int max_seq)
{
    const int half = head_dim / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_heads * half)
        return;
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;
    const int h = idx / half, i = idx % half;
    int64_t *v = vec + (size_t)h * head_dim;
    const int64_t c = cos_t[(size_t)pos * half + i];
    const int64_t s = sin_t[(size_t)pos * half + i];
    const int64_t x0 = v[i], x1 = v[i + half];
    v[i] = (int64_t)((uint64_t)q48_mul(x0, c) - (uint64_t)q48_mul(x1, s));
    v[i + half] = (int64_t)((uint64_t)q48_mul(x1, c) + (uint64_t)q48_mul(x0, s));
}

// ---------------------------------------------------------------------------
// Exact GQA decode attention: KV store (llama_int.c:1414-1416), scale
// (:1433) and the exact branch (:1502-1529) with softmax (:1060-1072).
// One block (256 threads) per query head; sc = per-head score row in the
// workspace.  Position pos reads k_new / v_new directly, so the cache write
// done by the first head of each KV group cannot race with the reads.
// ---------------------------------------------------------------------------
constexpr int ATT_NT = 256;

__global__ __launch_bounds__(ATT_NT) void k_attn_decode(
    int64_t *__restrict__ out, const int64_t *__restrict__ q,
    int64_t *__restrict__ kcache, int64_t *__restrict__ vcache,
    const int64_t *__restrict__ k_new, const int64_t *__restrict__ v_new,
    int64_t *__restrict__ scores, int layer, const int *__restrict__ d_pos, int pos,
    int n_heads, int n_kv, int hd, int max_seq)
{
    __shared__ int64_t qs[256];
    __shared__ int64_t red[ATT_NT / 64];
    __shared__ int64_t part[ATT_NT];
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;   // uniform over the block
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int group = n_heads / n_kv;
    const int kh = h / group;
    const size_t kvd = (size_t)n_kv * hd;
    const size_t base = (size_t)layer * max_seq;
    const int64_t *kn = k_new + (size_t)kh * hd;
    const int64_t *vn = v_new + (size_t)kh * hd;

    if (h % group == 0)
        for (int d = tid; d < hd; d += ATT_NT) {
            kcache[(base + pos) * kvd + (size_t)kh * hd + d] = kn[d];
            vcache[(base + pos) * kvd + (size_t)kh * hd + d] = vn[d];
        }
    for (int d = tid; d < hd; d += ATT_NT)
        qs[d] = q[(size_t)h * hd + d];
    __syncthreads();

    const int64_t scale = q48_inv_sqrt(q48_from_int(hd));
    const int S = pos + 1;
    int64_t *sc = scores + (size_t)h * max_seq;

    // scores s_t = fp_mul((int64)(q . k_t >> 48), scale)
    int64_t mx = INT64_MIN;
    for (int t = tid; t < S; t += ATT_NT) {
        const int64_t *kt = t == pos ? kn : kcache + (base + t) * kvd + (size_t)kh * hd;
        q48_u128 dot = 0;
        for (int d = 0; d < hd; ++d)
            dot += (q48_u128)q48_smul128(qs[d], kt[d]);
        const int64_t s = q48_mul((int64_t)((q48_i128)dot >> 48), scale);
        sc[t] = s;
        mx = s > mx ? s : mx;
    }
    mx = block_max64<ATT_NT>(mx, red);

    // e_t = fp_safe_exp(s_t - max); sum (int64, wrapping)
    int64_t sum = 0;
    for (int t = tid; t < S; t += ATT_NT) {
        const int64_t e = q48_safe_exp((int64_t)((uint64_t)sc[t] - (uint64_t)mx));
        sc[t] = e;
        sum = (int64_t)((uint64_t)sum + (uint64_t)e);
    }
    sum = block_sum64<ATT_NT>(sum, red);
    if (sum > 0) {
        const q48_divisor dv = q48_divisor_of(sum);
        for (int t = tid; t < S; t += ATT_NT)
            sc[t] = q48_div_by(sc[t], dv);
    }
    __syncthreads();

    // o[d] = sum_t fp_mul(p_t, v_t[d])  (int64, wrapping)
    const int slices = ATT_NT / hd;   // hd divides ATT_NT (checked on host)
    const int d = tid % hd, sl = tid / hd;
    int64_t acc = 0;
    for (int t = sl; t < S; t += slices) {
        const int64_t *vt = t == pos ? vn : vcache + (base + t) * kvd + (size_t)kh * hd;
        acc = (int64_t)((uint64_t)acc + (uint64_t)q48_mul(sc[t], vt[d]));
    }
    part[tid] = acc;
    __syncthreads();
    if (sl == 0) {
        uint64_t o = 0;
        for (int s2 = 0; s2 < slices; ++s2)
            o += (uint64_t)part[s2 * hd + d];
        out[(size_t)h * hd + d] = (int64_t)o;
    }
}

// ---------------------------------------------------------------------------
// Attention v2: the same exact computation as k_attn_decode with
//  - RoPE fused (ROPE = 1): q_h and k_new are rotated in the block
//    (rope_apply, llama_int.c:997-1008, 1392-1395); the first head of each
//    KV group writes the rotated k and v_new into the cache;
//  - 8 lanes per score: each lane multiplies hd/8 dimensions, a 3-step
//    128-bit butterfly sums them, so a score costs hd/8 MACs of latency;
//  - scores / probabilities in LDS when the cache fits (LDS = 1), else in
//    the global workspace row of the head;
//  - the V pass keeps 8 independent loads in flight per thread.
// pos is read from *d_pos when given (graph replay of a decode step).
// hd must be a multiple of 8 and divide 256 (checked on the host).
// ---------------------------------------------------------------------------

template <int ROPE, int LDS>
__global__ __launch_bounds__(ATT_NT) void k_attn_v2(
    int64_t *__restrict__ out, const int64_t *__restrict__ q,
    int64_t *__restrict__ kcache, int64_t *__restrict__ vcache,
    const int64_t *__restrict__ k_new, const int64_t *__restrict__ v_new,
    int64_t *__restrict__ scores, const int64_t *__restrict__ cos_t,
    const int64_t *__restrict__ sin_t, int layer, const int *__restrict__ d_pos, int pos,
    int n_heads, int n_kv, int hd, int max_seq, const ulonglong2 *__restrict__ pf,
    size_t pf_n16)
{
    __shared__ int64_t qs[256], ks[256], vs[256];
    __shared__ int64_t red[ATT_NT / 64];
    __shared__ int64_t part[ATT_NT];
    __shared__ int64_t sc_lds[LDS ? ATT_LDS_MAX : 1];
    if ((int)blockIdx.x >= n_heads) {
        // Blocks past the heads run on otherwise idle compute units while
        // the heads' latency-bound chain runs: they read the next op's
        // weights so that op finds them in the device-side cache (MALL).
        // The values are only consumed by an empty asm statement.
        const size_t stride = (size_t)(gridDim.x - n_heads) * ATT_NT;
        size_t i = (size_t)(blockIdx.x - n_heads) * ATT_NT + threadIdx.x;
        uint64_t acc = 0;
        for (; i + 7 * stride < pf_n16; i += 8 * stride) {
            ulonglong2 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = pf[i + u * stride];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                acc ^= v[u].x ^ v[u].y;
        }
        for (; i < pf_n16; i += stride)
            acc ^= pf[i].x ^ pf[i].y;
        asm volatile("" ::"v"(acc));
        return;
    }
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;   // uniform over the block: no barrier is skipped by part of it
    const int h = blockIdx.x, tid = threadIdx.x;
    const int group = n_heads / n_kv, kh = h / group;
    const size_t kvd = (size_t)n_kv * hd;
    const size_t base = (size_t)layer * max_seq;
    const int64_t *qh = q + (size_t)h * hd;
    const int64_t *kn = k_new + (size_t)kh * hd;
    const int64_t *vn = v_new + (size_t)kh * hd;
    const int half = hd / 2;
    int64_t *sc = LDS ? sc_lds : scores + (size_t)h * max_seq;

    if (ROPE) {
        if (tid < half) {
            const int64_t c = cos_t[(size_t)pos * half + tid];
            const int64_t sn = sin_t[(size_t)pos * half + tid];
            const int64_t q0 = qh[tid], q1 = qh[tid + half];
            qs[tid] = (int64_t)((uint64_t)q48_mul(q0, c) - (uint64_t)q48_mul(q1, sn));
            qs[tid + half] = (int64_t)((uint64_t)q48_mul(q1, c) + (uint64_t)q48_mul(q0, sn));
            const int64_t k0 = kn[tid], k1 = kn[tid + half];
            ks[tid] = (int64_t)((uint64_t)q48_mul(k0, c) - (uint64_t)q48_mul(k1, sn));
            ks[tid + half] = (int64_t)((uint64_t)q48_mul(k1, c) + (uint64_t)q48_mul(k0, sn));
        }
    } else {
        for (int d = tid; d < hd; d += ATT_NT) {
            qs[d] = qh[d];
            ks[d] = kn[d];
        }
    }
    for (int d = tid; d < hd; d += ATT_NT)
        vs[d] = vn[d];
    __syncthreads();
    if (h % group == 0)
        for (int d = tid; d < hd; d += ATT_NT) {
            kcache[(base + pos) * kvd + (size_t)kh * hd + d] = ks[d];
            vcache[(base + pos) * kvd + (size_t)kh * hd + d] = vs[d];
        }

    const int64_t scale = q48_inv_sqrt(q48_from_int(hd));
    const int S = pos + 1;

    // scores: group g of 8 lanes takes position t; lane l8 dims [l8*dpl, +dpl)
    const int g = tid >> 3, l8 = tid & 7, dpl = hd >> 3;
    int64_t mx = INT64_MIN;
    for (int t0 = 0; t0 < S; t0 += ATT_NT / 8) {
        const int t = t0 + g;
        q48_u128 dot = 0;
        if (t < S) {
            const int64_t *kt = t == pos ? ks : kcache + (base + t) * kvd + (size_t)kh * hd;
            kt += l8 * dpl;
            const int64_t *qd = qs + l8 * dpl;
            for (int d = 0; d < dpl; d += 2) {
                const int64_t a0 = kt[d], a1 = kt[d + 1];
                dot += (q48_u128)q48_smul128(qd[d], a0);
                dot += (q48_u128)q48_smul128(qd[d + 1], a1);
            }
        }
        dot = q48_sum8_u128(dot);
        if (t < S && l8 == 0) {
            const int64_t s = q48_mul((int64_t)((q48_i128)dot >> 48), scale);
            sc[t] = s;
            mx = s > mx ? s : mx;
        }
    }
    mx = block_max64<ATT_NT>(mx, red);

    int64_t sum = 0;
    for (int t = tid; t < S; t += ATT_NT) {
        const int64_t e = q48_safe_exp((int64_t)((uint64_t)sc[t] - (uint64_t)mx));
        sc[t] = e;
        sum = (int64_t)((uint64_t)sum + (uint64_t)e);
    }
    sum = block_sum64<ATT_NT>(sum, red);
    if (sum > 0) {
        const q48_divisor dv = q48_divisor_of(sum);
        for (int t = tid; t < S; t += ATT_NT)
            sc[t] = q48_div_by(sc[t], dv);
    }
    __syncthreads();

    // o[d] = sum_t fp_mul(p_t, v_t[d]): 8 positions per batch, loads first
    const int slices = ATT_NT / hd;
    const int d = tid % hd, sl = tid / hd;
    const int64_t *vcol = vcache + base * kvd + (size_t)kh * hd + d;
    uint64_t acc = 0;
    int t = sl;
    for (; t + 7 * slices < S; t += 8 * slices) {
        int64_t vv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int tu = t + u * slices;
            vv[u] = tu == pos ? vs[d] : vcol[(size_t)tu * kvd];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            acc += (uint64_t)q48_mul(sc[t + u * slices], vv[u]);
    }
    for (; t < S; t += slices)
        acc += (uint64_t)q48_mul(sc[t], t == pos ? vs[d] : vcol[(size_t)t * kvd]);
    part[tid] = (int64_t)acc;
    __syncthreads();
    if (sl == 0) {
        uint64_t o = 0;
        for (int s2 = 0; s2 < slices; ++s2)
            o += (uint64_t)part[s2 * hd + d];
        out[(size_t)h * hd + d] = (int64_t)o;
    }
}

// ---------------------------------------------------------------------------
// Attention v3: k_attn_v2's computation with its memory round trips cut
// (attn_v3_head, q48_attn.hpp).  One block of 256 threads per query head;
// HD = 32, 64 or 128; at most ATT_LDS_MAX positions.  Blocks past n_heads
// prefetch like k_attn_v2's.  ROT: q rotated, k and v at pos already in the
// cache (q48_launch_gemv_rope_kv); k_new, v_new and the RoPE tables unused.
// ---------------------------------------------------------------------------
template <int HD, int NT, bool ROT = false>
__global__ __launch_bounds__(NT) void k_attn_v3(
    int64_t *__restrict__ out, const int64_t *__restrict__ q, int64_t *__restrict__ kcache,
    int64_t *__restrict__ vcache, const int64_t *__restrict__ k_new,
    const int64_t *__restrict__ v_new, const int64_t *__restrict__ cos_t,
    const int64_t *__restrict__ sin_t, const int64_t *__restrict__ scale_p, int layer,
    const int *__restrict__ d_pos, int pos, int n_heads, int n_kv, int max_seq,
    const ulonglong2 *__restrict__ pf, size_t pf_n16)
{
    if ((int)blockIdx.x >= n_heads) {
        const size_t stride = (size_t)(gridDim.x - n_heads) * NT;
        size_t i = (size_t)(blockIdx.x - n_heads) * NT + threadIdx.x;
        uint64_t acc = 0;
        for (; i + 7 * stride < pf_n16; i += 8 * stride) {
            ulonglong2 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = pf[i + u * stride];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                acc ^= v[u].x ^ v[u].y;
        }
        for (; i < pf_n16; i += stride)
            acc ^= pf[i].x ^ pf[i].y;
        asm volatile("" ::"v"(acc));
        return;
    }
    attn_v3_head<HD, ATT_LDS_MAX, false, false, false, NT, ROT>(
        out, q, kcache, vcache, k_new, v_new, cos_t, sin_t, scale_p, layer, d_pos, pos, n_heads,
        n_kv, max_seq, (int)blockIdx.x);
}

// This thread's share of argmax (llama_int.c:2888-2893) over v[0..n) with
// 1024 threads: elements tid + 1024 i, scanned in ascending order with a
// strict > (the first maximum wins).  The loads of a batch of 32 are all
// issued before any comparison: one memory round trip per batch instead of
// one per element.
__device__ __forceinline__ void argmax_scan(const int64_t *__restrict__ v, int n, int tid,
                                            int64_t &best, int &idx)
{
    constexpr int B = 32;
    for (int i0 = 0; i0 < n; i0 += 1024 * B) {
        int64_t x[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int i = i0 + tid + 1024 * b;
            x[b] = v[i < n ? i : n - 1];
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int i = i0 + tid + 1024 * b;
            if (i < n && x[b] > best) {
                best = x[b];
                idx = i;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Split attention for long caches: the same exact computation spread over
// (chunk of ATT_CH positions, head) blocks, so that a head's keys and values
// stream through many compute units instead of one.  The reference's
// softmax needs the global max before any exponential and the global sum
// before any division, so three launches over the same (chunk, head) grid:
//  - k_attn_s1: each block rotates q_h / the new k (RoPE), scores its chunk
//    into sc[h][t] and its chunk maximum into cmax[h][c]
//    (llama_int.c:1502-1512);
//  - k_attn_se: each block takes the global max over the chunk maxima,
//    turns its chunk's scores into e_t = fp_safe_exp(s_t - max) (one per
//    thread) and stores the chunk's int64 (wrapping) sum in csum[h][c]; the
//    chunk-0 block zeroes out[h] (llama_int.c:1060-1068);
//  - k_attn_s2: each block adds the chunk sums (wrapping: the reference's
//    sum in any order), turns its chunk into p_t = fp_div(e_t, sum) when
//    sum > 0 (one per thread, llama_int.c:1069-1071), then adds
//    sum_t fp_mul(p_t, v_t[d]) over its chunk into out[h][d] with 64-bit
//    atomic adds: int64 wrap sums in any order, the bits of
//    llama_int.c:1514-1529.
// Every exponential and division runs on its own thread, spread over all the
// chunk blocks, instead of on one block per head.
// Blocks whose chunk starts past pos exit at once (the grid covers the
// whole cache, so a captured graph stays valid as pos grows).
// ---------------------------------------------------------------------------
constexpr int ATT_CH = 256;        // positions per chunk
// k_attn_v3 block size: 512 threads score 64 positions per pass and hold 8
// value slices, so up to 128 positions have their keys and values loaded
// before the first score (with 256 threads a second round of loads waited)
constexpr int ATT_V3_NT = 512;
// first position served by the split kernels: from 256 positions on the
// one-launch split form (about 13.4 us per launch at TinyLlama's heads,
// whatever the position up to 2048) is faster than one block per head
// (14.9 us at 256, 22.5 us at 511: its fifth key pass and value batch go out
// after the first are consumed)
constexpr int ATT_SPLIT_MIN = 256;
constexpr int ATT_NCMAX = 128;   // chunks per head: max_seq <= 32768

template <int HD>
__global__ __launch_bounds__(256) void k_attn_s1(
    const int64_t *__restrict__ q, int64_t *__restrict__ kcache, int64_t *__restrict__ vcache,
    const int64_t *__restrict__ k_new, const int64_t *__restrict__ v_new,
    const int64_t *__restrict__ cos_t, const int64_t *__restrict__ sin_t,
    const int64_t *__restrict__ scale_p, int64_t *__restrict__ sc, int64_t *__restrict__ cmax,
    int layer, const int *__restrict__ d_pos, int pos, int n_heads, int n_kv, int max_seq)
{
    constexpr int NT = 256, DPL = HD / 8, DP2 = DPL / 2, NG = NT / 8;
    __shared__ int64_t qs[HD], ks[HD], vs[HD];
    __shared__ int64_t red[NT / 64];
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int S = pos + 1, t0 = c * ATT_CH;
    if (t0 >= S)
        return;   // uniform: no barrier is skipped by part of the block
    const int tend = min(t0 + ATT_CH, S);
    const int group = n_heads / n_kv, kh = h / group;
    const size_t kvd = (size_t)n_kv * HD;
    const size_t base = (size_t)layer * max_seq;
    const int half = HD / 2;
    const int g = tid >> 3, l8 = tid & 7;
    const int64_t scale = *scale_p;
    int64_t *sch = sc + (size_t)h * max_seq;

    // RoPE inputs and the new v first, then the first two key passes
    const int64_t *qh = q + (size_t)h * HD, *kn = k_new + (size_t)kh * HD;
    const int i = min(tid, half - 1), j = min(tid, HD - 1);
    int64_t cs = cos_t[(size_t)pos * half + i];
    int64_t sn = sin_t[(size_t)pos * half + i];
    int64_t q0 = qh[i], q1 = qh[i + half];
    int64_t k0 = kn[i], k1 = kn[i + half];
    int64_t vn = v_new[(size_t)kh * HD + j];
    __builtin_amdgcn_sched_barrier(0);
    const int64_t *kb0 = kcache + base * kvd + (size_t)kh * HD + l8 * DPL;
    auto krow = [&](int t) {
        return reinterpret_cast<const ulonglong2 *>(kb0 + (size_t)min(t, tend - 1) * kvd);
    };
    ulonglong2 ka[DP2], kb[DP2];
#pragma unroll
    for (int d = 0; d < DP2; ++d)
        ka[d] = krow(t0 + g)[d];
#pragma unroll
    for (int d = 0; d < DP2; ++d)
        kb[d] = krow(t0 + NG + g)[d];
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(cs), "+v"(sn), "+v"(q0), "+v"(q1), "+v"(k0), "+v"(k1), "+v"(vn));
    qs[i] = (int64_t)((uint64_t)q48_mul(q0, cs) - (uint64_t)q48_mul(q1, sn));
    qs[i + half] = (int64_t)((uint64_t)q48_mul(q1, cs) + (uint64_t)q48_mul(q0, sn));
    ks[i] = (int64_t)((uint64_t)q48_mul(k0, cs) - (uint64_t)q48_mul(k1, sn));
    ks[i + half] = (int64_t)((uint64_t)q48_mul(k1, cs) + (uint64_t)q48_mul(k0, sn));
    vs[j] = vn;
    __syncthreads();
    if (h % group == 0 && c == pos / ATT_CH && tid < HD) {
        kcache[(base + pos) * kvd + (size_t)kh * HD + tid] = ks[tid];
        vcache[(base + pos) * kvd + (size_t)kh * HD + tid] = vs[tid];
    }

    // scores of the chunk (the row at pos is the block's own rotated k)
    const int64_t *qd = qs + l8 * DPL, *kd = ks + l8 * DPL;
    int64_t mx = INT64_MIN;
    auto score = [&](const ulonglong2 (&kr)[DP2], int t) {
        const bool own = t == pos;
        q48_u128 dot = 0;
#pragma unroll
        for (int d = 0; d < DP2; ++d) {
            const int64_t a0 = own ? kd[2 * d] : (int64_t)kr[d].x;
            const int64_t a1 = own ? kd[2 * d + 1] : (int64_t)kr[d].y;
            dot += (q48_u128)q48_smul128(qd[2 * d], a0);
            dot += (q48_u128)q48_smul128(qd[2 * d + 1], a1);
        }
        dot = q48_sum8_u128(dot);
        if (t < tend && l8 == 0) {
            const int64_t sv = q48_mul((int64_t)((q48_i128)dot >> 48), scale);
            sch[t] = sv;
            mx = sv > mx ? sv : mx;
        }
    };
    // the next passes' rows only where there is a next pass (block-uniform)
    for (int tt = t0; tt < tend; tt += 2 * NG) {
        score(ka, tt + g);
        if (tt + 2 * NG < tend) {
#pragma unroll
            for (int d = 0; d < DP2; ++d)
                ka[d] = krow(tt + 2 * NG + g)[d];
        }
        score(kb, tt + NG + g);
        if (tt + 3 * NG < tend) {
#pragma unroll
            for (int d = 0; d < DP2; ++d)
                kb[d] = krow(tt + 3 * NG + g)[d];
        }
    }
    mx = block_max64<NT>(mx, red);
    if (tid == 0)
        cmax[(size_t)h * ATT_NCMAX + c] = mx;
}

// exponentials of one chunk and their sum (see above)
template <int HD>
__global__ __launch_bounds__(256) void k_attn_se(int64_t *__restrict__ out,
                                                int64_t *__restrict__ sc,
                                                const int64_t *__restrict__ cmax,
                                                int64_t *__restrict__ csum,
                                                const int *__restrict__ d_pos, int pos,
                                                int n_heads, int max_seq)
{
    constexpr int NT = 256;
    static_assert(ATT_CH == NT, "one position per thread");
    __shared__ int64_t red[NT / 64];
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int S = pos + 1, t0 = c * ATT_CH;
    if (t0 >= S)
        return;   // uniform
    const int nc = (S + ATT_CH - 1) / ATT_CH, t = t0 + tid;
    int64_t *sch = sc + (size_t)h * max_seq;
    const int64_t s = sch[min(t, S - 1)];
    int64_t gm = tid < nc ? cmax[(size_t)h * ATT_NCMAX + tid] : INT64_MIN;
    gm = block_max64<NT>(gm, red, false);
    int64_t e = 0;
    if (t < S) {
        e = q48_safe_exp((int64_t)((uint64_t)s - (uint64_t)gm));
        sch[t] = e;
    }
    e = block_sum64<NT>(e, red);
    if (tid == 0)
        csum[(size_t)h * ATT_NCMAX + c] = e;
    if (c == 0 && tid < HD)
        out[(size_t)h * HD + tid] = 0;
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_s2(int64_t *__restrict__ out,
                                                const int64_t *__restrict__ vcache,
                                                const int64_t *__restrict__ sc,
                                                const int64_t *__restrict__ csum, int layer,
                                                const int *__restrict__ d_pos, int pos,
                                                int n_heads, int n_kv, int max_seq)
{
    constexpr int NT = 256, SL = NT / HD, VB = 8;
    __shared__ int64_t part[NT], pl[ATT_CH], red[NT / 64];
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int S = pos + 1, t0 = c * ATT_CH;
    if (t0 >= S)
        return;
    const int tend = min(t0 + ATT_CH, S);
    const int group = n_heads / n_kv, kh = h / group;
    const size_t kvd = (size_t)n_kv * HD;
    const int d = tid % HD, sl = tid / HD;
    const int64_t *vcol = vcache + (size_t)layer * max_seq * kvd + (size_t)kh * HD + d;
    const int64_t *ph = sc + (size_t)h * max_seq;
    // positions t0 + sl + SL i of this thread, VB per batch, one batch ahead;
    // the first value batches go out before the division
    auto tpos = [&](int i) { return min(t0 + sl + SL * i, tend - 1); };
    const int nc = (S + ATT_CH - 1) / ATT_CH;
    const int64_t ev = ph[min(t0 + tid, tend - 1)];
    int64_t cs = tid < nc ? csum[(size_t)h * ATT_NCMAX + tid] : 0;
    int64_t va[VB], vb[VB];
#pragma unroll
    for (int u = 0; u < VB; ++u)
        va[u] = vcol[(size_t)tpos(u) * kvd];
#pragma unroll
    for (int u = 0; u < VB; ++u)
        vb[u] = vcol[(size_t)tpos(VB + u) * kvd];
    // p_t = fp_div(e_t, sum) when sum > 0, one position per thread
    const int64_t sum = block_sum64<NT>(cs, red, false);
    pl[tid] = sum > 0 ? q48_div_by(ev, q48_divisor_of(sum)) : ev;
    __syncthreads();
    uint64_t acc = 0;
    auto vmac = [&](const int64_t (&vv)[VB], int i0) {
#pragma unroll
        for (int u = 0; u < VB; ++u)
            if (t0 + sl + SL * (i0 + u) < tend)
                acc += (uint64_t)q48_mul(pl[sl + SL * (i0 + u)], vv[u]);
    };
    // the next batches only where some position of them exists (block-uniform)
    for (int i0 = 0; t0 + sl + SL * i0 < tend; i0 += 2 * VB) {
        vmac(va, i0);
        if (t0 + SL * (i0 + 2 * VB) < tend) {
#pragma unroll
            for (int u = 0; u < VB; ++u)
                va[u] = vcol[(size_t)tpos(i0 + 2 * VB + u) * kvd];
        }
        vmac(vb, i0 + VB);
        if (t0 + SL * (i0 + 3 * VB) < tend) {
#pragma unroll
            for (int u = 0; u < VB; ++u)
                vb[u] = vcol[(size_t)tpos(i0 + 3 * VB + u) * kvd];
        }
    }
    part[tid] = (int64_t)acc;
    __syncthreads();
    if (sl == 0) {
        uint64_t o = 0;
#pragma unroll
        for (int s2 = 0; s2 < SL; ++s2)
            o += (uint64_t)part[s2 * HD + d];
        __hip_atomic_fetch_add(reinterpret_cast<uint64_t *>(out) + (size_t)h * HD + d, o,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------
// One-launch split attention (k_attn_g).  One block per (chunk of ATTG_CH
// positions, KV head) serves every query head of the KV head's group
// (llama_int.c:1506, kv_h = h / gqa_group), so each key and value row is
// read from memory once per launch, not once per query head.  The chunk
// blocks of a KV head hand the softmax's global max and global sum to each
// other at two exchanges inside the kernel (the reference's softmax needs
// the max before any exponential and the sum before any division,
// llama_int.c:1060-1072).  Per block:
//  1. the chunk's key and value rows and the RoPE inputs are loaded at once;
//     RoPE of the group's q heads and of the new k (llama_int.c:1392-1395);
//     the KV store at pos by the chunk that holds it (llama_int.c:1414-1416);
//     keys and values go to LDS (the row at pos replaced by the block's own
//     rotated k and new v); the score of each (query head, position), two
//     threads per score, s_t = fp_mul((sum_d q_d k_t,d) >> 48, scale)
//     (llama_int.c:1502-1512), and the chunk maximum per head;
//  2. exchange 1 of the chunk maxima; e_t = fp_safe_exp(s_t - max), one per
//     thread, and the chunk's int64 (wrapping) sum per head;
//  3. exchange 2 of the chunk sums; p_t = fp_div(e_t, sum) when sum > 0;
//     each thread owns one output (head, d) of the group and adds
//     sum_t fp_mul(p_t, v_t[d]) over the chunk into out with a 64-bit atomic
//     add (int64 wrapping sums in any order: the bits of
//     llama_int.c:1514-1529); the chunk-0 block zeroes the group's output at
//     its start, long before any block adds.
// A cache of one chunk skips the exchanges and stores out directly.
//
// Exchanges (no atomics, no separate flags).  Every published int64 goes out
// as two 64-bit words (low half, epoch) and (high half, epoch): a 64-bit
// store is seen whole or not at all, so a reader that finds the expected
// epoch in a word also finds its half.  Per KV head an epoch word E is read
// at the start; the block's values go out with epoch E + 1 and the readers
// poll the words of all nc chunks until each carries E + 1.  After the second
// exchange the chunk-0 block stores E + 1 into the epoch (the next launch
// then expects E + 2, which no word of this launch carries).  A wait longer
// than the wait bound `tmo` (ATTG_TIMEOUT unless the host sets another; 0
// gives up at once, without polling) ends the block and sets the error word,
// for q48_attn_status; the host sizes the grid so that every active block is
// resident at once.  Blocks whose chunk starts past pos exit at once (the
// grid covers max_seq, so a captured graph stays valid as pos grows).
// ---------------------------------------------------------------------------
constexpr int ATTG_NT = 512;
constexpr int ATTG_CH = 32;                       // positions per chunk
constexpr int ATTG_NCMAX = 256;                   // chunks per KV head: max_seq <= 8192
constexpr int ATTG_GMAX = 8;                      // query heads per KV head
constexpr uint64_t ATTG_TIMEOUT = 1ull << 24;     // wall-clock ticks (0.17 s at 100 MHz)
constexpr int ATTG_KVMAX = 16;                    // KV heads
// words (uint64) of one exchange per KV head and chunk: (half, epoch) x 2 per head
constexpr int ATTG_XW = 2 * ATTG_GMAX;
// the exchange region: uint64 words [2 exchanges][ATTG_KVMAX][ATTG_NCMAX]
// [ATTG_XW], then uint32 epochs [ATTG_KVMAX] 16 apart and the error word;
// zero before the first launch, never cleared after: a word counts only
// when it carries the current launch's epoch
constexpr size_t ATTG_XWORDS = (size_t)2 * ATTG_KVMAX * ATTG_NCMAX * ATTG_XW;
constexpr size_t ATTG_SYNC_BYTES = ATTG_XWORDS * 8 + ((size_t)ATTG_KVMAX * 16 + 16) * 4;

__device__ __forceinline__ uint64_t attg_ld64(const uint64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void attg_st64(uint64_t *p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Maximum and wrapping sum over each 32-lane half of a wave (all lanes
// active; every lane returns its half's result): DPP within rows of 16, then
// the other row of the half.
__device__ __forceinline__ int64_t attg_max32(int64_t v)
{
    int64_t o = (int64_t)q48_dpp64<Q48_DPP_XOR1>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_XOR2>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_HALF_MIRROR>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_MIRROR>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)__shfl_xor((long long)v, 16, 64);
    return o > v ? o : v;
}

__device__ __forceinline__ uint64_t attg_sum32(uint64_t v)
{
    v += q48_dpp64<Q48_DPP_XOR1>(v);
    v += q48_dpp64<Q48_DPP_XOR2>(v);
    v += q48_dpp64<Q48_DPP_HALF_MIRROR>(v);
    v += q48_dpp64<Q48_DPP_MIRROR>(v);
    return v + (uint64_t)__shfl_xor((long long)v, 16, 64);
}

// Publish v[0..G) (thread hh < G publishes v for head hh) as epoch-tagged
// halves into row `mine`, then gather, for every head hh < G, the values of
// all nc chunks (rows xw + ATTG_XW c) into got[hh][c] (LDS).  Block-wide;
// false on every thread after a timeout.
template <int NT>
__device__ bool attg_exchange(uint64_t *xw, int c, int nc, int G, unsigned epoch,
                              const int64_t *v, int64_t (*got)[ATTG_NCMAX], int *err,
                              uint64_t tmo)
{
    const int tid = threadIdx.x;
    if (tid < G) {
        const uint64_t u = (uint64_t)v[tid];
        attg_st64(xw + (size_t)ATTG_XW * c + 2 * tid, (u << 32) | epoch);
        attg_st64(xw + (size_t)ATTG_XW * c + 2 * tid + 1, (u & 0xFFFFFFFF00000000ull) | epoch);
    }
    // every thread reads words (chunk, head, half) = i, i + NT, ... of nc x 2G;
    // each wave polls until all of its words carry the epoch (a wave vote, no
    // block barrier per round: a round is one load latency), then one
    // barrier joins the waves
    const int nw = nc * 2 * G;
    const uint64_t t0 = wall_clock64();
    int ok = tmo != 0;
    while (ok) {
        bool mine = true;
        for (int i = tid; i < nw; i += NT) {
            const int cc = i / (2 * G), r = i % (2 * G);
            const uint64_t w = attg_ld64(xw + (size_t)ATTG_XW * cc + r);
            if ((unsigned)w != epoch) {
                mine = false;
            } else {
                // halves: word 2 hh carries bits 0..31 in its top, 2 hh + 1 bits 32..63
                uint32_t *g32 = reinterpret_cast<uint32_t *>(&got[r >> 1][cc]);
                g32[r & 1] = (uint32_t)(w >> 32);
            }
        }
        if (__all(mine))
            break;
        // the give-up decision: the wave's clock (a scalar read, uniform)
        if (wall_clock64() - t0 > tmo) {
            ok = 0;
            break;
        }
    }
    // got[] complete (or abandoned) for every thread; a wave that gave up
    // fails the block
    if (__syncthreads_or(!ok)) {
        if (tid == 0)
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    return true;
}

// head_dim 32/64: at most 128 VGPRs, so that two blocks (16 waves) fit a
// compute unit and the grid of a 4096-position cache with 4 KV heads (512
// blocks) is resident; head_dim 128: its LDS rows allow one block per unit.
// MF (head_dim 64): the scores on the int8 matrix cores.  The chunk's key
// rows and the group's rotated q heads become digit planes in LDS (the key
// planes share their LDS with the exchange buffer, which is used only after
// the scores); waves 0 and 1 each run the 63 digit-pair
// v_mfma_i32_16x16x64_i8 of one 16-position tile (query heads as rows,
// padded to 16 with zero digits), and the corrections C sum_d q_d and
// C sum_d S(k_d) (a ones row of the same tile) complete the exact int128
// dot (q48_digits.hpp).
template <int HD, bool MF = false>
__global__ __launch_bounds__(ATTG_NT) __attribute__((amdgpu_waves_per_eu(HD == 128 ? 2 : 4))) void k_attn_g(
    int64_t *__restrict__ out, const int64_t *__restrict__ q, int64_t *__restrict__ kcache,
    int64_t *__restrict__ vcache, const int64_t *__restrict__ k_new,
    const int64_t *__restrict__ v_new, const int64_t *__restrict__ cos_t,
    const int64_t *__restrict__ sin_t, const int64_t *__restrict__ scale_p,
    uint64_t *__restrict__ xbuf, int layer, const int *__restrict__ d_pos, int pos,
    int n_heads, int n_kv, int max_seq, uint64_t tmo)
{
    constexpr int NT = ATTG_NT, CH = ATTG_CH, GM = ATTG_GMAX;
    constexpr int HALF = HD / 2, RS = HD + 1;
    constexpr int RP = (GM * HALF + NT - 1) / NT;       // RoPE pairs per thread
    constexpr int LW = CH * HD / NT;                    // row words per thread
    constexpr int NO = (GM * HD + NT - 1) / NT;         // outputs per thread
    constexpr int DH = HD / 2;                          // dims per score thread
    static_assert(LW % 2 == 0 && HD % LW == 0, "16-byte row loads");
    static_assert(GM * CH * 2 == NT, "two threads per score");
    static_assert(CH == 32 && NT == 64 * GM, "32 lanes per head in a chunk, a wave per head");
    static_assert(!MF || (HD == 64 && LW == 4 && CH == 32 && GM == 8), "matrix-core scores");
    constexpr int KDW = HD / 4 + 4;                     // digit-plane row: 16 words + 4 pad
    __shared__ int64_t qs[GM][HD];
    __shared__ int64_t ks[HD], vs[HD];
    __shared__ int64_t kl[CH][RS], vl[CH][RS];           // odd row stride: no bank conflicts
    __shared__ int64_t sc[GM][CH];
    __shared__ q48_u128 dpart[MF ? 1 : GM * CH];
    __shared__ int64_t loc[GM];
    // the exchange buffer, and before it the key digit planes (MF)
    __shared__ union __align__(16) {
        int64_t got[GM][ATTG_NCMAX];
        uint32_t kd[MF ? 8 : 1][CH][KDW];
    } gk;
    int64_t (*got)[ATTG_NCMAX] = gk.got;
    __shared__ __align__(16) uint32_t qd[MF ? 8 : 1][GM][KDW];   // q digit planes (MF)
    __shared__ uint64_t ck[MF ? CH : 1][2], cq[MF ? GM : 1][2];   // correction sums (MF)
    // the digit sums of the matrix-core scores, [14][head][position], in
    // the key rows' LDS (MF)
    int(*accs)[GM][CH] = reinterpret_cast<int(*)[GM][CH]>(&kl[0][0]);
    static_assert(!MF || 14 * GM * CH * 4 <= (int)sizeof(int64_t) * CH * RS, "digit sums fit");
    static_assert(!MF || GM <= 8, "row 8 of the score tile is the ones row");
    if (d_pos)
        pos = *d_pos;
    if (pos < 0 || pos >= max_seq)
        return;
    const int c = blockIdx.y, kh = blockIdx.x, tid = threadIdx.x;
    const int S = pos + 1, t0 = c * CH;
    if (t0 >= S)
        return;   // uniform: no barrier is skipped by part of the block
    const int nc = (S + CH - 1) / CH, tend = min(t0 + CH, S), nt = tend - t0;
    const int G = n_heads / n_kv, h0 = kh * G;
    const size_t kvd = (size_t)n_kv * HD;
    const size_t base = (size_t)layer * max_seq;
    uint64_t *xw1 = xbuf + (size_t)kh * ATTG_NCMAX * ATTG_XW;
    uint64_t *xw2 = xw1 + (size_t)ATTG_KVMAX * ATTG_NCMAX * ATTG_XW;
    unsigned *sync = reinterpret_cast<unsigned *>(xbuf + ATTG_XWORDS);
    unsigned *ep = sync + (size_t)kh * 16;
    int *err = reinterpret_cast<int *>(sync + (size_t)ATTG_KVMAX * 16);

    // loads: the epoch and the RoPE inputs first, then the chunk's rows
    const unsigned E = nc > 1 ? __hip_atomic_load(ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : 0u;
    int64_t cs[RP], sn[RP], q0[RP], q1[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const int idx = min(tid + r * NT, G * HALF - 1);
        const int hh = idx / HALF, i = idx % HALF;
        cs[r] = cos_t[(size_t)pos * HALF + i];
        sn[r] = sin_t[(size_t)pos * HALF + i];
        q0[r] = q[(size_t)(h0 + hh) * HD + i];
        q1[r] = q[(size_t)(h0 + hh) * HD + i + HALF];
    }
    const int ik = min(tid, HALF - 1), jv = min(tid, HD - 1);
    int64_t kc0 = cos_t[(size_t)pos * HALF + ik], ks0 = sin_t[(size_t)pos * HALF + ik];
    int64_t k0 = k_new[(size_t)kh * HD + ik], k1 = k_new[(size_t)kh * HD + ik + HALF];
    int64_t vn = v_new[(size_t)kh * HD + jv];
    __builtin_amdgcn_sched_barrier(0);
    // row words: thread tid holds LW consecutive words of row tid / (HD / LW)
    const int rr = tid / (HD / LW), rw = (tid % (HD / LW)) * LW;
    const int tr = min(t0 + rr, tend - 1);
    const ulonglong2 *krow = reinterpret_cast<const ulonglong2 *>(
        kcache + (base + tr) * kvd + (size_t)kh * HD + rw);
    const ulonglong2 *vrow = reinterpret_cast<const ulonglong2 *>(
        vcache + (base + tr) * kvd + (size_t)kh * HD + rw);
    ulonglong2 kr[LW / 2], vr[LW / 2];
#pragma unroll
    for (int d = 0; d < LW / 2; ++d)
        kr[d] = krow[d];
#pragma unroll
    for (int d = 0; d < LW / 2; ++d)
        vr[d] = vrow[d];
    __builtin_amdgcn_sched_barrier(0);
    if (c == 0 && nc > 1)   // the group's output starts at zero (atomic adds below)
#pragma unroll
        for (int o = 0; o < NO; ++o)
            if (tid + o * NT < G * HD)
                __hip_atomic_store(out + (size_t)h0 * HD + tid + o * NT, (int64_t)0,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // RoPE (rope_apply, llama_int.c:997-1008): the group's q heads, the new k
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const int idx = tid + r * NT;
        if (idx < G * HALF) {
            const int hh = idx / HALF, i = idx % HALF;
            qs[hh][i] = (int64_t)((uint64_t)q48_mul(q0[r], cs[r]) - (uint64_t)q48_mul(q1[r], sn[r]));
            qs[hh][i + HALF] =
                (int64_t)((uint64_t)q48_mul(q1[r], cs[r]) + (uint64_t)q48_mul(q0[r], sn[r]));
        }
    }
    if (tid < HALF) {
        ks[tid] = (int64_t)((uint64_t)q48_mul(k0, kc0) - (uint64_t)q48_mul(k1, ks0));
        ks[tid + HALF] = (int64_t)((uint64_t)q48_mul(k1, kc0) + (uint64_t)q48_mul(k0, ks0));
    }
    if (tid < HD)
        vs[tid] = vn;
#pragma unroll
    for (int d = 0; d < LW / 2; ++d) {
        kl[rr][rw + 2 * d] = (int64_t)kr[d].x;
        kl[rr][rw + 2 * d + 1] = (int64_t)kr[d].y;
        vl[rr][rw + 2 * d] = (int64_t)vr[d].x;
        vl[rr][rw + 2 * d + 1] = (int64_t)vr[d].y;
    }
    __syncthreads();
    if (pos < tend && tid < HD) {   // the row at pos: this block's rotated k, new v
        kl[pos - t0][tid] = ks[tid];
        vl[pos - t0][tid] = vs[tid];
        kcache[(base + pos) * kvd + (size_t)kh * HD + tid] = ks[tid];
        vcache[(base + pos) * kvd + (size_t)kh * HD + tid] = vs[tid];
    }
    __syncthreads();

    // scores: pair p = (head hh, position t) = tid % (GM CH), dims half tid / (GM CH)
    const int pi = tid % (GM * CH), hh = pi / CH, t = pi % CH, dh = tid / (GM * CH);
    const bool live = hh < G && t < nt;
    if constexpr (MF) {
        // digit planes: the key words this thread loaded (row rr, dims rw..rw+3,
        // read back from LDS: the row at pos may have been replaced) and, on
        // threads below 128, four dims of one q head (zero digits past G)
        {
            uint64_t v4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v4[e] = (uint64_t)kl[rr][rw + e];
            uint32_t wd[8];
            digits4(v4, wd);
#pragma unroll
            for (int a = 0; a < 8; ++a)
                gk.kd[a][rr][rw / 4] = wd[a];
        }
        if (tid < GM * 16) {
            const int qh = tid >> 4, dq = 4 * (tid & 15);
            uint64_t v4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v4[e] = qh < G ? (uint64_t)qs[qh][dq + e] : kDig;
            uint32_t wd[8];
            digits4(v4, wd);
#pragma unroll
            for (int a = 0; a < 8; ++a)
                qd[a][qh][dq / 4] = wd[a];
        }
        __syncthreads();
        // waves 0 and 1: tile w = positions 16 w .. 16 w + 15.  Lane l holds
        // A row (q head) l % 16 and B column (position) l % 16, dims 16 (l / 16)
        // .. + 15; the result rows 4 (l / 16) + i at column l % 16.  A row 8
        // (never a head: at most 8 per group) is ones in digit 0, so that its
        // result is sum_d S(k_t,d), and the correction C sum_d q_d + C sum_d
        // k_d - hd C^2 is C sum_d q_d + C sum_d S(k_t,d).  Waves 2 and 3 sum
        // the q heads meanwhile.
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        if (wv < 2) {
            const int ln = tid & 63, col = ln & 15, kq = ln >> 4, tt = 16 * wv + col;
            v4i A[8];
#pragma unroll
            for (int a = 0; a < 8; ++a)
                A[a] = col < GM ? *reinterpret_cast<const v4i *>(&qd[a][col][4 * kq])
                       : col == 8 && a == 0 ? (v4i){0x01010101, 0x01010101, 0x01010101, 0x01010101}
                                            : (v4i){0, 0, 0, 0};
            v4i acc[14];
#pragma unroll
            for (int d = 0; d < 14; ++d)
                acc[d] = (v4i){0, 0, 0, 0};
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const v4i B = *reinterpret_cast<const v4i *>(&gk.kd[b][tt][4 * kq]);
#pragma unroll
                for (int a = 0; a < 8; ++a)
                    if (a + b <= 13)
                        acc[a + b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[a], B, acc[a + b],
                                                                          0, 0, 0);
            }
            // the raw sums to LDS (the key rows' space: kl is read only by the
            // digit split above), [d][head][position]; row 8's lanes the key
            // correction
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int qh = 4 * kq + i;
                if (qh < G)
#pragma unroll
                    for (int d = 0; d < 14; ++d)
                        accs[d][qh][tt] = acc[d][i];
            }
            if (kq == 2) {
                const q48_u128 cc = digits_total(acc, 0) * kDig;
                ck[tt][0] = (uint64_t)cc;
                ck[tt][1] = (uint64_t)(cc >> 64);
            }
        } else if (wv < 4) {
            // C sum_d q_d of head (tid - 128) / 16: 16 threads, 4 dims each
            const int qh = (tid - 128) >> 4, dq = 4 * (tid & 15);
            uint64_t v4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v4[e] = qh < G ? (uint64_t)qs[qh][dq + e] : 0;
            const q48_u128 sm = row16_sum4(v4);
            if ((tid & 15) == 0) {
                const q48_u128 cc = sm * kDig;
                cq[qh][0] = (uint64_t)cc;
                cq[qh][1] = (uint64_t)(cc >> 64);
            }
        }
        __syncthreads();
        // one score per thread: the digit sums, the corrections, the scale
        if (tid < GM * CH) {
            const int qh = tid / CH, tt = tid % CH;
            if (qh < G) {
                int a14[14];
#pragma unroll
                for (int d = 0; d < 14; ++d)
                    a14[d] = accs[d][qh][tt];
                const q48_u128 tot = digits_total14(a14) +
                                     (((q48_u128)ck[tt][1] << 64) | ck[tt][0]) +
                                     (((q48_u128)cq[qh][1] << 64) | cq[qh][0]);
                sc[qh][tt] = tt < nt ? q48_mul((int64_t)(tot >> 48), *scale_p) : INT64_MIN;
            }
        }
        __syncthreads();
    } else {
        q48_u128 dot = 0;
        if (hh < G) {
            const int64_t *qa = qs[hh] + dh * DH, *ka = kl[t] + dh * DH;
#pragma unroll 8
            for (int d = 0; d < DH; ++d)
                dot += (q48_u128)q48_smul128(qa[d], ka[d]);
        }
        if (dh == 1)
            dpart[pi] = dot;
        __syncthreads();
        if (dh == 0 && hh < G) {
            dot += dpart[pi];
            sc[hh][t] = live ? q48_mul((int64_t)((q48_i128)dot >> 48), *scale_p) : INT64_MIN;
        }
        __syncthreads();
    }
    // the chunk's maximum per head: 32 lanes per head (waves 0 .. GM / 2 - 1)
    if (tid < 32 * GM) {
        const int hq = tid >> 5, u = tid & 31;
        const int64_t m = attg_max32(hq < G && u < nt ? sc[hq][u] : INT64_MIN);
        if (u == 0 && hq < G)
            loc[hq] = m;
    }
    __syncthreads();
    if (nc > 1) {
        __builtin_amdgcn_s_waitcnt(0);   // chunk 0: the output zeroes are out
        if (!attg_exchange<NT>(xw1, c, nc, G, E + 1, loc, got, err, tmo)) {
            if (tid == 0)
                __hip_atomic_store(ep, E + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        {
            // the maximum over the chunks: wave hq for head hq
            const int hq = tid >> 6, l = tid & 63;
            int64_t m = INT64_MIN;
            for (int u = l; u < nc; u += 64)
                m = got[hq][u] > m ? got[hq][u] : m;
            m = q48_wave_max64(m);
            if (l == 0 && hq < G)
                loc[hq] = m;
        }
        __syncthreads();
    }

    // e_t = fp_safe_exp(s_t - max), one per thread, and the chunk sums
    if (dh == 0 && hh < G)
        sc[hh][t] = live ? q48_safe_exp((int64_t)((uint64_t)sc[hh][t] - (uint64_t)loc[hh])) : 0;
    __syncthreads();
    if (tid < 32 * GM) {
        const int hq = tid >> 5, u = tid & 31;
        const uint64_t sm = attg_sum32(hq < G && u < nt ? (uint64_t)sc[hq][u] : 0);
        if (u == 0 && hq < G)
            loc[hq] = (int64_t)sm;
    }
    __syncthreads();
    if (nc > 1) {
        if (!attg_exchange<NT>(xw2, c, nc, G, E + 1, loc, got, err, tmo)) {
            if (tid == 0)
                __hip_atomic_store(ep, E + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        {
            const int hq = tid >> 6, l = tid & 63;
            uint64_t sm = 0;
            for (int u = l; u < nc; u += 64)
                sm += (uint64_t)got[hq][u];
            sm = (uint64_t)q48_wave_sum64((int64_t)sm);
            if (l == 0 && hq < G)
                loc[hq] = (int64_t)sm;
        }
        if (c == 0 && tid == 0)   // every block of the head is past exchange 2
            __hip_atomic_store(ep, E + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
    }
    // p_t = fp_div(e_t, sum) when sum > 0 (llama_int.c:1069-1071).  The
    // weights are never negative (exponentials over a positive sum, or the
    // exponentials themselves); the block checks it, and the values take
    // the product for non-negative weights (q48_pv_mac) unless one is
    int neg = 0;
    if (dh == 0 && live) {
        const int64_t sum = loc[hh];
        if (sum > 0)
            sc[hh][t] = q48_div_by(sc[hh][t], q48_divisor_of(sum));
        neg = sc[hh][t] < 0;
    }
    neg = __syncthreads_or(neg);

    // o[h][d] += sum_t fp_mul(p_t, v_t[d]) over the chunk: thread owns the
    // outputs tid + NT o of the group's [G][HD]
#pragma unroll
    for (int o = 0; o < NO; ++o) {
        const int oi = tid + o * NT;
        if (oi < G * HD) {
            const int oh = oi / HD, d = oi % HD;
            uint64_t acc = 0;
            if (!neg) {
                q48_pv_acc pa = {0, 0};
                for (int u = 0; u < nt; ++u)
                    q48_pv_mac(pa, sc[oh][u], vl[u][d]);
                acc = (uint64_t)q48_pv_total(pa);
            } else {
                for (int u = 0; u < nt; ++u)
                    acc += (uint64_t)q48_mul(sc[oh][u], vl[u][d]);
            }
            int64_t *dst = out + (size_t)h0 * HD + oi;
            if (nc > 1)
                __hip_atomic_fetch_add(reinterpret_cast<uint64_t *>(dst), acc, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            else
                *dst = (int64_t)acc;
        }
    }
}

// ---------------------------------------------------------------------------
// Decode-step state (graph replay): st[0] = token, st[1] = pos, st[2] =
// number of tokens recorded.  k_step_argmax is argmax (llama_int.c:
// 2888-2893) feeding the next step: token <- argmax, pos += 1, and the
// token is appended to tokens[] while st[2] < cap.
// ---------------------------------------------------------------------------
__global__ void k_step_set(int *__restrict__ st, int token, int pos)
{
    if (threadIdx.x == 0) {
        st[0] = token;
        st[1] = pos;
        st[2] = 0;
    }
}

// argmax of v[0..n) into the state on AMAX_BLOCKS blocks of 256: each block
// scans a chunk (and with rec copies it to rec[count][..] while count <
// rec_cap, count read before any block's ticket), its (maximum, first index)
// goes out with agent-coherent stores ahead of a ticket, and the last block
// combines the partials (the largest value, the lowest index among equal
// ones: the reference's first maximum), updates the state and resets the
// ticket.  The same token as k_step_argmax; no block waits on another.
constexpr int AMAX_BLOCKS = 32;
__global__ __launch_bounds__(256) void k_step_argmax_mb(int *__restrict__ st,
                                                       int *__restrict__ tokens, int cap,
                                                       const int64_t *__restrict__ v, int n,
                                                       int64_t *__restrict__ rec, int rec_cap,
                                                       uint64_t *__restrict__ part)
{
    __shared__ int64_t bv[4];
    __shared__ int bi[4];
    __shared__ int last_sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int k = st[2];
    int64_t *dst = rec && k >= 0 && k < rec_cap ? rec + (size_t)k * n : nullptr;
    const int chunk = (n + (int)gridDim.x - 1) / (int)gridDim.x;
    const int i0 = (int)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
    int64_t best = INT64_MIN;
    int idx = n;
    for (int i = i0 + tid; i < i1; i += 256) {
        const int64_t x = v[i];
        if (dst)
            dst[i] = x;
        if (x > best) {   // ascending i: the first maximum of this thread
            best = x;
            idx = i;
        }
    }
    auto wave_best = [&]() {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const int64_t ov = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (ov > best || (ov == best && oi < idx)) {
                best = ov;
                idx = oi;
            }
        }
    };
    wave_best();
    if (lane == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    uint64_t *ticket = part + 2 * AMAX_BLOCKS;
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        __hip_atomic_store(&part[2 * blockIdx.x], (uint64_t)best, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&part[2 * blockIdx.x + 1], (uint64_t)(uint32_t)idx, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const uint64_t t = __hip_atomic_fetch_add(ticket, (uint64_t)1, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        last_sh = t == (uint64_t)gridDim.x - 1;
    }
    __syncthreads();
    if (!last_sh || tid >= 64)
        return;
    best = INT64_MIN;
    idx = n;
    if (tid < (int)gridDim.x) {
        best = (int64_t)__hip_atomic_load(&part[2 * tid], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        idx = (int)__hip_atomic_load(&part[2 * tid + 1], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    }
    wave_best();
    if (tid == 0) {
        const int tok = idx < n ? idx : 0;
        st[0] = tok;
        st[1] = st[1] + 1;
        if (k < cap)
            tokens[k] = tok;
        st[2] = k + 1;
        __hip_atomic_store(ticket, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ __launch_bounds__(1024) void k_step_argmax(int *__restrict__ st,
                                                     int *__restrict__ tokens, int cap,
                                                     const int64_t *__restrict__ v, int n)
{
    __shared__ int64_t bv[16];
    __shared__ int bi[16];
    const int tid = threadIdx.x;
    int64_t best = INT64_MIN;
    int idx = n;
    argmax_scan(v, n, tid, best, idx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int64_t ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((tid & 63) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        const int tok = idx < n ? idx : 0;
        st[0] = tok;
        st[1] = st[1] + 1;
        const int k = st[2];
        if (k < cap)
            tokens[k] = tok;
        st[2] = k + 1;
    }
}

// Step-mode parity hook: rec[count][0..n) = v[0..n), count = st[2] (the
// tokens chosen so far in this run of steps), while count < cap.  Enqueued
// before the step's token choice, it keeps every step's logits so that the
// host can hash them after a graph replay.
__global__ __launch_bounds__(256) void k_step_record(const int *__restrict__ st,
                                                    int64_t *__restrict__ rec, int cap,
                                                    const int64_t *__restrict__ v, int n)
{
    const int k = st[2];
    if (k < 0 || k >= cap)
        return;
    int64_t *dst = rec + (size_t)k * n;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
        dst[i] = v[i];
}

// SwiGLU over interleaved (gate, up) pairs: out[i] = fp_mul(silu(t[2i]), t[2i+1])
__global__ __launch_bounds__(256) void k_silu_mul_pairs(int64_t *__restrict__ out,
                                                       const int64_t *__restrict__ t, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        out[i] = q48_mul(q48_silu(t[2 * i]), t[2 * i + 1]);
}

// SwiGLU, llama_int.c:1549-1552: out = fp_mul(fp_silu(g), u)
__global__ __launch_bounds__(256) void k_silu_mul(int64_t *__restrict__ out,
                                                 const int64_t *__restrict__ g,
                                                 const int64_t *__restrict__ u, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        out[i] = q48_mul(q48_silu(g[i]), u[i]);
}

// Residual add, llama_int.c:1535 and :1556 (int64, wrapping)
__global__ __launch_bounds__(256) void k_add(int64_t *__restrict__ acc,
                                            const int64_t *__restrict__ d, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        acc[i] = (int64_t)((uint64_t)acc[i] + (uint64_t)d[i]);
}

// hidden = embed_tokens[token] (llama_int.c:2822-2824)
__global__ __launch_bounds__(256) void k_embed(int64_t *__restrict__ out,
                                              const int64_t *__restrict__ table,
                                              const int *__restrict__ d_token,
                                              int token, int dim)
{
    if (d_token)
        token = *d_token;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < dim)
        out[i] = table[(size_t)token * dim + i];
}

// argmax, llama_int.c:2888-2893: first index of the maximum.
__global__ __launch_bounds__(1024) void k_argmax(int *__restrict__ out,
                                                const int64_t *__restrict__ v, int n)
{
    __shared__ int64_t bv[16];
    __shared__ int bi[16];
    const int tid = threadIdx.x;
    int64_t best = INT64_MIN;
    int idx = n;   // sentinel larger than any index
    argmax_scan(v, n, tid, best, idx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int64_t ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((tid & 63) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        *out = idx < n ? idx : 0;
    }
}

__global__ __launch_bounds__(256) void k_zero(uint64_t *__restrict__ p, size_t n8)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

__global__ void k_zero_bytes(uint8_t *__restrict__ p, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = 0;
}

// Element-wise fp_math evaluation (determinism gate and unit parity).
__global__ __launch_bounds__(256) void k_fp_eval(int func, const int64_t *__restrict__ x,
                                                const int64_t *__restrict__ y,
                                                int64_t *__restrict__ o0,
                                                int64_t *__restrict__ o1,
                                                const q48_consts *__restrict__ k, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    const int64_t a = x[i];
    int64_t r = 0, r1 = 0;
    switch (func) {
    case 0: r = q48_mul(a, y[i]); break;
    case 1: r = y[i] != 0 ? q48_div(a, y[i]) : 0; break;
    case 2: r = q48_sqrt(a); break;
    case 3: r = q48_sqrt_fast(a); break;
    case 4: r = q48_inv_sqrt(a); break;
    case 5: r = q48_exp(a); break;
    case 6: r = q48_log(a); break;
    case 7: q48_sincos(k, a, &r, &r1); break;
    case 8: r = q48_sigmoid(a); break;
    case 9: r = q48_silu(a); break;
    case 10: r = q48_safe_exp(a); break;
    case 11: r = q48_exp_dyadic(a, (int)y[i]); break;
    case 12: r = y[i] != 0 ? q48_div_by(a, q48_divisor_of(y[i])) : 0; break;
    default: break;
    }
    o0[i] = r;
    if (o1)
        o1[i] = r1;
}

} // namespace

int q48_launch_math_init(q48_ctx *c)
{
    hipLaunchKernelGGL(k_math_init, dim3(1), dim3(64), 0, c->stream, c->consts);
    return (int)hipGetLastError();
}

int q48_launch_rmsnorm(q48_ctx *c, int64_t *out, const int64_t *x,
                       const int64_t *w, int dim)
{
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(256), 0, c->stream, out, x, w, dim);
    return (int)hipGetLastError();
}

int q48_launch_pf_rmsnorm(q48_ctx *c, int64_t *out, const int64_t *X, const int64_t *w, int T,
                          int dim)
{
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(256), 0, c->stream, out, X, w, dim);
    return (int)hipGetLastError();
}

int q48_launch_rope_init(q48_ctx *c)
{
    const long n = (long)(c->rope_head_dim / 2) * c->rope_max_seq;
    hipLaunchKernelGGL(k_rope_init, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       c->stream, c->rope_cos, c->rope_sin, c->consts,
                       c->rope_head_dim, c->rope_max_seq, c->rope_theta);
    return (int)hipGetLastError();
}

int q48_launch_rope(q48_ctx *c, int64_t *vec, int n_heads, int head_dim,
                    const int *d_pos, int pos)
{
    const int n = n_heads * (head_dim / 2);
    hipLaunchKernelGGL(k_rope, dim3((n + 255) / 256), dim3(256), 0, c->stream, vec,
                       c->rope_cos, c->rope_sin, n_heads, head_dim, d_pos, pos,
                       c->rope_max_seq);
    return (int)hipGetLastError();
}

int q48_launch_attn(q48_ctx *c, int64_t *out, const int64_t *q,
                    int64_t *kcache, int64_t *vcache, const int64_t *k_new,
                    const int64_t *v_new, int layer, const int *d_pos, int pos,
                    int n_heads, int n_kv, int head_dim, int max_seq)
{
    int rc = q48_ws_reserve(c, (size_t)n_heads * max_seq * sizeof(int64_t));
    if (rc)
        return rc;
    hipLaunchKernelGGL(k_attn_decode, dim3(n_heads), dim3(ATT_NT), 0, c->stream, out, q,
                       kcache, vcache, k_new, v_new, (int64_t *)c->ws, layer, d_pos,
                       pos, n_heads, n_kv, head_dim, max_seq);
    return (int)hipGetLastError();
}

int q48_att_split_min() { return ATT_SPLIT_MIN; }
int q48_att_lds_max() { return ATT_LDS_MAX; }

// Workspace of the split attention: k_attn_s1/se/s2's scores [n_heads]
// [max_seq], chunk maxima and sums [n_heads][ATT_NCMAX].  k_attn_g's
// exchange words, epochs and error word live apart, in a region that is zero
// before the first launch (ATTG_SYNC_BYTES).
size_t q48_attn_ws_bytes(int n_heads, int max_seq, int head_dim)
{
    (void)head_dim;
    return ((size_t)n_heads * max_seq + (size_t)2 * n_heads * ATT_NCMAX) * sizeof(int64_t);
}

size_t q48_attn_sync_bytes() { return ATTG_SYNC_BYTES; }

uint64_t q48_attg_default_wait() { return ATTG_TIMEOUT; }

// Each launch with more than one chunk advances its KV heads' 32-bit epochs
// by one, and a chunk word counts when it carries the launch's epoch.  A word
// not rewritten since an earlier launch with the same epoch value (2^32
// launches before) would be taken for this launch's: so the region is zeroed,
// with the stream idle, before its count of launches reaches 2^31.
int q48_attg_account(q48_ctx *c, const unsigned *sync, uint64_t n)
{
    constexpr uint64_t kLimit = (uint64_t)1 << 31;
    uint64_t *count = sync == c->attx_sync ? &c->attg_count : q48_scratch_attg_count(c->device);
    if (!count)
        return Q48_EINVAL;
    if (*count + n >= kLimit) {
        if (hipStreamSynchronize(c->stream) != hipSuccess ||
            q48_launch_zero(c, const_cast<unsigned *>(sync), ATTG_SYNC_BYTES) != (int)hipSuccess ||
            hipStreamSynchronize(c->stream) != hipSuccess)
            return Q48_EHIP;
        *count = 0;
    }
    *count += n;
    return Q48_OK;
}

// k_attn_g needs every active block resident at once: the chunks of a full
// cache (max_seq) times the KV heads must fit the device's occupancy.
static bool attg_fits(q48_ctx *c, int hd, int n_heads, int n_kv, int max_seq)
{
    const int k = hd == 64 ? (c->attn_g_mfma ? 3 : 0) : hd == 32 ? 1 : 2;
    if (n_heads % n_kv || n_heads / n_kv > ATTG_GMAX || n_kv > ATTG_KVMAX)
        return false;
    if ((max_seq + ATTG_CH - 1) / ATTG_CH > ATTG_NCMAX)
        return false;
    if (c->attx_per_cu[k] < 0) {   // resident blocks per compute unit, asked once
        const void *fn = k == 0   ? (const void *)k_attn_g<64>
                         : k == 3 ? (const void *)k_attn_g<64, true>
                         : k == 1 ? (const void *)k_attn_g<32>
                                  : (const void *)k_attn_g<128>;
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, ATTG_NT, 0) != hipSuccess)
            n = 0;
        c->attx_per_cu[k] = n;
    }
    const long need = (long)n_kv * ((max_seq + ATTG_CH - 1) / ATTG_CH);
    return need <= (long)c->attx_per_cu[k] * c->cu_count;
}

int q48_launch_attn_v2(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                       int64_t *vcache, const int64_t *k_new, const int64_t *v_new,
                       int layer, const int *d_pos, int pos, int n_heads, int n_kv,
                       int head_dim, int max_seq, int rope, const void *prefetch,
                       size_t prefetch_bytes, int64_t *ws_ext, size_t ws_ext_bytes,
                       unsigned *sync_ext)
{
    // prefetch blocks: one per compute unit the heads leave idle
    const size_t pf_n16 = prefetch ? prefetch_bytes / 16 : 0;
    const int pf_blocks = pf_n16 ? (c->cu_count > n_heads ? c->cu_count - n_heads : 1) : 0;
    const bool lds = max_seq <= ATT_LDS_MAX;
    // the workspace: the caller's (allocation-free entry) or the context's
    auto ws_get = [&](size_t bytes, int64_t **p) -> int {
        if (ws_ext) {
            if (bytes > ws_ext_bytes)
                return Q48_ERANGE;
            *p = ws_ext;
            return Q48_OK;
        }
        int rc = q48_ws_reserve(c, bytes);
        *p = (int64_t *)c->ws;
        return rc;
    };
    int64_t *ws = nullptr;
    if (!lds) {
        int rc = ws_get((size_t)n_heads * max_seq * sizeof(int64_t), &ws);
        if (rc)
            return rc;
    }
#define ATT_LAUNCH(R, L)                                                                      \
    hipLaunchKernelGGL((k_attn_v2<R, L>), dim3(n_heads + pf_blocks), dim3(ATT_NT), 0,         \
                       c->stream, out, q, kcache, vcache, k_new, v_new, ws, c->rope_cos,      \
                       c->rope_sin, layer, d_pos, pos, n_heads, n_kv, head_dim, max_seq,      \
                       (const ulonglong2 *)prefetch, pf_n16)
    const int64_t *scale_p = c->rope_sin + (size_t)c->rope_max_seq * (c->rope_head_dim / 2);
    // long caches: split kernels (chunks of positions over many blocks) once
    // the position reaches ATT_SPLIT_MIN; a captured graph keeps the kernels
    // of the position it was captured at
    if (rope && pos >= ATT_SPLIT_MIN && (head_dim == 32 || head_dim == 64 || head_dim == 128) &&
        (max_seq + ATT_CH - 1) / ATT_CH <= ATT_NCMAX && n_heads <= 256) {
        const size_t sc_n = (size_t)n_heads * max_seq, cm_n = (size_t)n_heads * ATT_NCMAX;
        unsigned *sync = ws_ext ? sync_ext : c->attx_sync;
        if (c->attn_one_launch && sync && attg_fits(c, head_dim, n_heads, n_kv, max_seq)) {
            // KV head fastest: the blocks of the live chunks are dispatched
            // first and take one compute unit each (with chunk fastest, half of
            // them shared a unit with another live block and ran slower, and
            // both in-kernel exchanges waited for them)
            const dim3 grid(n_kv, (max_seq + ATTG_CH - 1) / ATTG_CH);
            // count the launch on its exchange region (a captured one counts
            // at every replay of its graph)
            if (c->capturing) {
                ++c->capture_attg[sync == c->attx_sync ? 0 : 1];
            } else {
                int arc = q48_attg_account(c, sync, 1);
                if (arc)
                    return arc;
            }
            c->attg_unchecked = 1;
#define ATTG_LAUNCH(HD, MFS)                                                                  \
    hipLaunchKernelGGL((k_attn_g<HD, MFS>), grid, dim3(ATTG_NT), 0, c->stream, out, q, kcache, \
                       vcache, k_new, v_new, c->rope_cos, c->rope_sin, scale_p,               \
                       reinterpret_cast<uint64_t *>(sync), layer, d_pos, pos, n_heads, n_kv,  \
                       max_seq, c->attg_wait)
            if (head_dim == 64 && c->attn_g_mfma)
                ATTG_LAUNCH(64, true);
            else if (head_dim == 64)
                ATTG_LAUNCH(64, false);
            else if (head_dim == 32)
                ATTG_LAUNCH(32, false);
            else
                ATTG_LAUNCH(128, false);
#undef ATTG_LAUNCH
            return (int)hipGetLastError();
        }
        int rc = ws_get(q48_attn_ws_bytes(n_heads, max_seq, head_dim), &ws);
        if (rc)
            return rc;
        int64_t *sc = ws, *cm = sc + sc_n, *cs = cm + cm_n;
        const dim3 grid((max_seq + ATT_CH - 1) / ATT_CH, n_heads);
#define ATTS_LAUNCH(HD)                                                                       \
    do {                                                                                      \
        hipLaunchKernelGGL((k_attn_s1<HD>), grid, dim3(256), 0, c->stream, q, kcache, vcache, \
                           k_new, v_new, c->rope_cos, c->rope_sin, scale_p, sc, cm, layer,    \
                           d_pos, pos, n_heads, n_kv, max_seq);                               \
        hipLaunchKernelGGL((k_attn_se<HD>), grid, dim3(256), 0, c->stream, out, sc, cm, cs,   \
                           d_pos, pos, n_heads, max_seq);                                     \
        hipLaunchKernelGGL((k_attn_s2<HD>), grid, dim3(256), 0, c->stream, out, vcache, sc,   \
                           cs, layer, d_pos, pos, n_heads, n_kv, max_seq);                    \
    } while (0)
        if (head_dim == 64)
            ATTS_LAUNCH(64);
        else if (head_dim == 32)
            ATTS_LAUNCH(32);
        else
            ATTS_LAUNCH(128);
#undef ATTS_LAUNCH
        return (int)hipGetLastError();
    }
#define ATT3_LAUNCH(HD)                                                                      \
    hipLaunchKernelGGL((k_attn_v3<HD, ATT_V3_NT>), dim3(n_heads + pf_blocks), dim3(ATT_V3_NT), \
                       0, c->stream,                                                         \
                       out, q, kcache, vcache, k_new, v_new, c->rope_cos, c->rope_sin,       \
                       scale_p, layer, d_pos, pos, n_heads, n_kv, max_seq,                   \
                       (const ulonglong2 *)prefetch, pf_n16)
    if (rope && lds && head_dim == 64)
        ATT3_LAUNCH(64);
    else if (rope && lds && head_dim == 32)
        ATT3_LAUNCH(32);
    else if (rope && lds && head_dim == 128)
        ATT3_LAUNCH(128);
    else if (rope && lds)
        ATT_LAUNCH(1, 1);
    else if (rope)
        ATT_LAUNCH(1, 0);
    else if (lds)
        ATT_LAUNCH(0, 1);
    else
        ATT_LAUNCH(0, 0);
#undef ATT_LAUNCH
#undef ATT3_LAUNCH
    return (int)hipGetLastError();
}

int q48_launch_attn_cached(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                           int64_t *vcache, int layer, const int *d_pos, int pos, int n_heads,
                           int n_kv, int head_dim, int max_seq, const void *prefetch,
                           size_t prefetch_bytes)
{
    // prefetch blocks: one per compute unit the heads leave idle (as
    // q48_launch_attn_v2)
    const size_t pf_n16 = prefetch ? prefetch_bytes / 16 : 0;
    const int pf_blocks = pf_n16 ? (c->cu_count > n_heads ? c->cu_count - n_heads : 1) : 0;
    const int64_t *scale_p = c->rope_sin + (size_t)c->rope_max_seq * (c->rope_head_dim / 2);
#define ATTC_LAUNCH(HD)                                                                       \
    hipLaunchKernelGGL((k_attn_v3<HD, ATT_V3_NT, true>), dim3(n_heads + pf_blocks),           \
                       dim3(ATT_V3_NT), 0, c->stream, out, q, kcache, vcache, nullptr, nullptr, \
                       nullptr, nullptr, scale_p, layer, d_pos, pos, n_heads, n_kv, max_seq,  \
                       (const ulonglong2 *)prefetch, pf_n16)
    if (head_dim == 64)
        ATTC_LAUNCH(64);
    else if (head_dim == 32)
        ATTC_LAUNCH(32);
    else if (head_dim == 128)
        ATTC_LAUNCH(128);
    else
        return (int)hipErrorInvalidValue;
#undef ATTC_LAUNCH
    return (int)hipGetLastError();
}

int q48_launch_step_set(q48_ctx *c, int token, int pos)
{
    hipLaunchKernelGGL(k_step_set, dim3(1), dim3(64), 0, c->stream, c->d_step, token, pos);
    return (int)hipGetLastError();
}

size_t q48_amax_part_bytes() { return (2 * AMAX_BLOCKS + 2) * sizeof(uint64_t); }

// n below AMAX_BLOCKS * 256 takes the one-block kernel (the record, when
// asked, as its own launch before it)
int q48_launch_step_argmax(q48_ctx *c, int *tokens, int cap, const int64_t *v, int n,
                           int64_t *rec, int rec_cap)
{
    if (n >= AMAX_BLOCKS * 256) {
        hipLaunchKernelGGL(k_step_argmax_mb, dim3(AMAX_BLOCKS), dim3(256), 0, c->stream,
                           c->d_step, tokens, cap, v, n, rec, rec_cap, c->amax_part);
        return (int)hipGetLastError();
    }
    if (rec) {
        const int rc = q48_launch_step_record(c, rec, rec_cap, v, n);
        if (rc)
            return rc;
    }
    hipLaunchKernelGGL(k_step_argmax, dim3(1), dim3(1024), 0, c->stream, c->d_step, tokens,
                       cap, v, n);
    return (int)hipGetLastError();
}

int q48_launch_step_record(q48_ctx *c, int64_t *rec, int cap, const int64_t *v, int n)
{
    const int blocks = (n + 255) / 256 < 256 ? (n + 255) / 256 : 256;
    hipLaunchKernelGGL(k_step_record, dim3(blocks), dim3(256), 0, c->stream, c->d_step, rec, cap,
                       v, n);
    return (int)hipGetLastError();
}

int q48_launch_silu_mul_pairs(q48_ctx *c, int64_t *out, const int64_t *t, int n)
{
    hipLaunchKernelGGL(k_silu_mul_pairs, dim3((n + 255) / 256), dim3(256), 0, c->stream, out, t, n);
    return (int)hipGetLastError();
}

int q48_launch_silu_mul(q48_ctx *c, int64_t *out, const int64_t *g,
                        const int64_t *u, int n)
{
    hipLaunchKernelGGL(k_silu_mul, dim3((n + 255) / 256), dim3(256), 0, c->stream, out, g, u, n);
    return (int)hipGetLastError();
}

int q48_launch_add(q48_ctx *c, int64_t *acc, const int64_t *d, int n)
{
    hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, c->stream, acc, d, n);
    return (int)hipGetLastError();
}

int q48_launch_embed(q48_ctx *c, int64_t *out, const int64_t *table,
                     const int *d_token, int token, int dim)
{
    hipLaunchKernelGGL(k_embed, dim3((dim + 255) / 256), dim3(256), 0, c->stream, out,
                       table, d_token, token, dim);
    return (int)hipGetLastError();
}

int q48_launch_argmax(q48_ctx *c, int *d_out, const int64_t *v, int n)
{
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, c->stream, d_out, v, n);
    return (int)hipGetLastError();
}

int q48_launch_zero(q48_ctx *c, void *p, size_t bytes)
{
    const size_t n8 = bytes / 8;
    if (n8) {
        size_t blocks = (n8 + 255) / 256;
        if (blocks > 65536)
            blocks = 65536;
        hipLaunchKernelGGL(k_zero, dim3((unsigned)blocks), dim3(256), 0, c->stream,
                           (uint64_t *)p, n8);
    }
    const size_t tail = bytes - n8 * 8;
    if (tail)
        hipLaunchKernelGGL(k_zero_bytes, dim3(1), dim3(64), 0, c->stream,
                           (uint8_t *)p + n8 * 8, tail);
    return (int)hipGetLastError();
}

int q48_launch_fp_eval(q48_ctx *c, int func, const int64_t *x,
                       const int64_t *y, int64_t *out0, int64_t *out1, int n)
{
    hipLaunchKernelGGL(k_fp_eval, dim3((n + 255) / 256), dim3(256), 0, c->stream, func, x, y,
                       out0, out1, c->consts, n);
    return (int)hipGetLastError();
}
