// q48_sample.hip — sample_token (llama_int.c:2958-3039) on gfx950, bit for
// bit: temperature division, top-k mask, softmax, top-p nucleus and one
// xoroshiro128+ draw (rng_next, llama_int.c:2922-2929) over device logits.
//
// The reference works sequentially: a qsort for the top-k threshold and, for
// the nucleus, a repeated first-maximum search whose running int64 sum
// decides when to stop.  Here:
//  - the top-k threshold (the k-th largest value, duplicates counted) is a
//    radix select over the order-preserving keys w ^ 2^63, 8 bits a pass;
//  - when every difference x - max is exact and the exponentials sum below
//    2^63 (always, for logits / T below 16384), each probability is at most
//    ONE and their sum at most ONE, so no running sum wraps: the nucleus is
//    then found by a radix search over the probabilities that carries the
//    sum of each bucket, and the entries equal to the cut value are kept in
//    index order, as the reference's first-maximum search takes them;
//  - otherwise (wrapping sums) the reference's loop itself runs, one
//    block-wide first-maximum per kept entry;
//  - the draw is the first index whose running (wrapping) sum exceeds r: a
//    block scan of chunk sums, then a walk of each thread's chunk.
// All arithmetic is integer; sums are mod 2^64 exactly as the reference's
// int64 additions under -fwrapv.
#include "q48_internal.h"

namespace {

constexpr int SMP_T = 256;                   // threads of the element-wise kernels
constexpr int SMP_B = 1024;                  // threads of the selection kernels
constexpr int SMP_GMAX = 256;                // blocks of the element-wise kernels at most
constexpr int64_t SMP_NEG = INT64_MIN / 2;   // the top-k mask (llama_int.c:2982)

// state words at the head of the sampling workspace
enum { ST_THR, ST_MX, ST_EXACT, ST_SUM, ST_WORDS = 8 };

struct SmpWs {
    int64_t *st;      // ST_WORDS state words
    int64_t *pmax;    // per-block max of w          [SMP_GMAX]
    int64_t *pmin;    // per-block min of w          [SMP_GMAX]
    uint64_t *psum;   // per-block sum of e, 128-bit [2 SMP_GMAX]
    int64_t *w;       // logits / T, then masked     [n]
    int64_t *p;       // exponentials, probabilities [n]
};

__device__ __forceinline__ SmpWs smp_ws(int64_t *base, int n)
{
    SmpWs s;
    s.st = base;
    s.pmax = base + ST_WORDS;
    s.pmin = s.pmax + SMP_GMAX;
    s.psum = reinterpret_cast<uint64_t *>(s.pmin + SMP_GMAX);
    s.w = s.pmin + 3 * SMP_GMAX;
    s.p = s.w + n;
    return s;
}

// ---- block reductions (NT threads, all active) ----------------------------
template <int NT>
__device__ __forceinline__ int64_t blk_max(int64_t v, int64_t *red)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int64_t o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i)
        v = red[i] > v ? red[i] : v;
    return v;
}

template <int NT>
__device__ __forceinline__ int64_t blk_min(int64_t v, int64_t *red)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int64_t o = __shfl_xor(v, off, 64);
        v = o < v ? o : v;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i)
        v = red[i] < v ? red[i] : v;
    return v;
}

template <int NT>
__device__ __forceinline__ uint64_t blk_sum(uint64_t v, int64_t *red)
{
    v = (uint64_t)q48_wave_sum64((int64_t)v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = (int64_t)v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i)
        t += (uint64_t)red[i];
    return t;
}

// (value, index) maximum, the smaller index among equal values (argmax,
// llama_int.c:2888-2893); idx = INT_MAX marks "none"
template <int NT>
__device__ __forceinline__ void blk_argmax(int64_t &v, int &idx, int64_t *redv, int *redi)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int64_t ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (oi != INT_MAX && (idx == INT_MAX || ov > v || (ov == v && oi < idx))) {
            v = ov;
            idx = oi;
        }
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        redv[threadIdx.x >> 6] = v;
        redi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    v = redv[0];
    idx = redi[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i)
        if (redi[i] != INT_MAX && (idx == INT_MAX || redv[i] > v || (redv[i] == v && redi[i] < idx))) {
            v = redv[i];
            idx = redi[i];
        }
}

// exclusive prefix sum (mod 2^64) over the threads of the block in order:
// a scan inside each wave, then the wave totals (tmp holds NT / 64 words)
template <int NT>
__device__ __forceinline__ uint64_t blk_excl_scan(uint64_t v, uint64_t *tmp)
{
    const int tid = threadIdx.x, lane = tid & 63;
    uint64_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t o = __shfl_up(incl, off, 64);
        if (lane >= off)
            incl += o;
    }
    __syncthreads();
    if (lane == 63)
        tmp[tid >> 6] = incl;
    __syncthreads();
    uint64_t before = 0;
    for (int w = 0; w < (tid >> 6); ++w)
        before += tmp[w];
    return before + incl - v;
}

// Walks of the radix selections, one wave (threads 0-63, all active): lane
// l holds buckets 4 l .. 4 l + 3 of the 256.  The bucket where the k-th
// largest lies (counts from the top: above < k <= above + cnt[b]) ...
__device__ __forceinline__ void walk_count(const int *cnt, int nb, int k, int *out_b,
                                           int *out_krem)
{
    const int l = threadIdx.x;
    int c[4], tot = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        c[j] = 4 * l + j < nb ? cnt[4 * l + j] : 0;
        tot += c[j];
    }
    int incl = tot;   // sum over lanes >= l
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_down(incl, off, 64);
        if (l + off < 64)
            incl += o;
    }
    int above = incl - tot;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
        if (above < k && k <= above + c[j]) {
            *out_b = 4 * l + j;
            *out_krem = k - above;
        }
        above += c[j];
    }
}

// ... and the highest bucket whose sum from the top reaches top_p (sums
// start at base; -1 when even the whole range stays below)
__device__ __forceinline__ void walk_sum(const int *cnt, const unsigned long long *sum, int nb,
                                         uint64_t base, int64_t top_p, int *out_b,
                                         uint64_t *out_above, int *out_ties)
{
    const int l = threadIdx.x;
    uint64_t sm[4], tot = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sm[j] = 4 * l + j < nb ? sum[4 * l + j] : 0;
        tot += sm[j];
    }
    uint64_t incl = tot;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t o = __shfl_down(incl, off, 64);
        if (l + off < 64)
            incl += o;
    }
    uint64_t above = base + incl - tot;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
        if ((int64_t)above < top_p && (int64_t)(above + sm[j]) >= top_p) {
            *out_b = 4 * l + j;
            *out_above = above;
            *out_ties = cnt[4 * l + j];
        }
        above += sm[j];
    }
}

// Passes of the single-block kernels over n values: the loads of a batch of
// SMP_U go out before any is used (one memory round trip per batch instead
// of one per element).  pass_strided visits i = tid, tid + SMP_B, ...;
// pass_chunk visits [lo, hi) in index order.
constexpr int SMP_U = 16;

template <class F>
__device__ __forceinline__ void pass_strided(const int64_t *a, int n, F f)
{
    for (int i0 = threadIdx.x; i0 < n; i0 += SMP_B * SMP_U) {
        int64_t v[SMP_U];
#pragma unroll
        for (int u = 0; u < SMP_U; ++u) {
            const int i = i0 + u * SMP_B;
            v[u] = a[i < n ? i : n - 1];
        }
#pragma unroll
        for (int u = 0; u < SMP_U; ++u)
            if (i0 + u * SMP_B < n)
                f(i0 + u * SMP_B, v[u]);
    }
}

template <class F>
__device__ __forceinline__ void pass_chunk(const int64_t *a, int lo, int hi, F f)
{
    for (int i0 = lo; i0 < hi; i0 += SMP_U) {
        int64_t v[SMP_U];
#pragma unroll
        for (int u = 0; u < SMP_U; ++u)
            v[u] = a[i0 + u < hi ? i0 + u : hi - 1];
#pragma unroll
        for (int u = 0; u < SMP_U; ++u)
            if (i0 + u < hi)
                f(i0 + u, v[u]);
    }
}

// ---- 1: w = fp_div(logit, T) (llama_int.c:2970-2971), block max / min ----
__global__ __launch_bounds__(SMP_T) void k_smp_scale(int64_t *__restrict__ base,
                                                    const int64_t *__restrict__ logits,
                                                    int n, int64_t temperature)
{
    __shared__ int64_t red[SMP_T / 64];
    SmpWs s = smp_ws(base, n);
    int64_t mx = INT64_MIN, mn = INT64_MAX;
    for (int i = blockIdx.x * SMP_T + threadIdx.x; i < n; i += gridDim.x * SMP_T) {
        const int64_t w = q48_div(logits[i], temperature);
        s.w[i] = w;
        mx = w > mx ? w : mx;
        mn = w < mn ? w : mn;
    }
    mx = blk_max<SMP_T>(mx, red);
    mn = blk_min<SMP_T>(mn, red);
    if (threadIdx.x == 0) {
        s.pmax[blockIdx.x] = mx;
        s.pmin[blockIdx.x] = mn;
    }
}

// ---- 2: top-k threshold (llama_int.c:2974-2987) and the exactness test ----
// The k-th largest w, duplicates counted (sorted[k - 1] of the reference's
// descending qsort): radix select, most significant byte first, over the
// keys w ^ 2^63 (unsigned order = signed order of w).
__global__ __launch_bounds__(SMP_B) void k_smp_topk(int64_t *__restrict__ base, int n,
                                                   int top_k, int nblk)
{
    __shared__ int64_t red[SMP_B / 64];
    __shared__ int hist[256];
    __shared__ int whist[16][256];
    __shared__ uint64_t sel_prefix;
    __shared__ int sel_krem, sel_krem2, sel_b;
    SmpWs s = smp_ws(base, n);
    const int tid = threadIdx.x;
    int64_t mx = INT64_MIN, mn = INT64_MAX;
    for (int b = tid; b < nblk; b += SMP_B) {
        mx = s.pmax[b] > mx ? s.pmax[b] : mx;
        mn = s.pmin[b] < mn ? s.pmin[b] : mn;
    }
    mx = blk_max<SMP_B>(mx, red);
    mn = blk_min<SMP_B>(mn, red);

    int64_t thr = INT64_MIN;
    if (top_k > 0 && top_k < n) {
        // keys w - min (unsigned, order-preserving), only the bits below
        // the range's top bit; one histogram per wave (LDS atomics of a
        // whole wave on one bucket would serialise), 8 bits a pass
        const uint64_t range = (uint64_t)mx - (uint64_t)mn;
        const int top = range ? 64 - __builtin_clzll(range) : 0;
        const int wave = tid >> 6;
        if (tid == 0) {
            sel_prefix = 0;
            sel_krem = top_k;
        }
        for (int hi = top; hi > 0; hi -= 8) {
            const int lo = hi > 8 ? hi - 8 : 0, width = hi - lo;
            for (int b = tid; b < 16 * 256; b += SMP_B)
                whist[b >> 8][b & 255] = 0;
            __syncthreads();
            const uint64_t prefix = sel_prefix;
            pass_strided(s.w, n, [&](int, int64_t w) {
                const uint64_t key = (uint64_t)w - (uint64_t)mn;
                if (hi >= 64 || (key >> hi) == prefix)
                    atomicAdd(&whist[wave][(key >> lo) & ((1u << width) - 1)], 1);
            });
            __syncthreads();
            if (tid < 256) {
                int h = 0;
#pragma unroll
                for (int w = 0; w < 16; ++w)
                    h += whist[w][tid];
                hist[tid] = h;
            }
            __syncthreads();
            if (tid < 64)
                walk_count(hist, 1 << width, sel_krem, &sel_b, &sel_krem2);
            __syncthreads();
            if (tid == 0) {
                sel_krem = sel_krem2;
                sel_prefix = (prefix << width) | (uint64_t)sel_b;
            }
            __syncthreads();
        }
        thr = (int64_t)((uint64_t)mn + sel_prefix);
    }
    if (tid == 0) {
        // masked entries (w < thr: some exist when thr > min w) become
        // INT64_MIN / 2, and join the maximum and the minimum of the values
        // the softmax sees; the threshold itself is kept
        const bool masked = thr > mn;
        if (masked && SMP_NEG > mx)
            mx = SMP_NEG;
        const int64_t xmin = masked ? (thr < SMP_NEG ? thr : SMP_NEG) : mn;
        s.st[ST_THR] = thr;
        s.st[ST_MX] = mx;
        // every x - mx exact in int64 (no wrap): exp(x - mx) <= ONE
        s.st[ST_EXACT] = (q48_i128)mx - (q48_i128)xmin <= ((q48_i128)1 << 63) ? 1 : 0;
    }
}

// ---- 3: e = fp_safe_exp(x - max) (softmax, llama_int.c:1060-1072) --------
__global__ __launch_bounds__(SMP_T) void k_smp_exp(int64_t *__restrict__ base, int n)
{
    __shared__ int64_t red[SMP_T / 64];
    SmpWs s = smp_ws(base, n);
    const int64_t thr = s.st[ST_THR], mx = s.st[ST_MX];
    uint64_t lo = 0, hi = 0;
    for (int i = blockIdx.x * SMP_T + threadIdx.x; i < n; i += gridDim.x * SMP_T) {
        const int64_t w = s.w[i];
        const int64_t x = w < thr ? SMP_NEG : w;
        const int64_t e = q48_safe_exp((int64_t)((uint64_t)x - (uint64_t)mx));
        s.p[i] = e;
        // e >= 0: the exact sum as 128 bits (the reference keeps its low 64)
        const uint64_t t = lo + (uint64_t)e;
        hi += t < lo;
        lo = t;
    }
    lo = blk_sum<SMP_T>(lo, red);
    hi = blk_sum<SMP_T>(hi, red);
    if (threadIdx.x == 0) {
        s.psum[2 * blockIdx.x] = lo;
        s.psum[2 * blockIdx.x + 1] = hi;
    }
}

// the exponentials' total: 128-bit sum of the per-block partials
__device__ __forceinline__ q48_u128 smp_total(const SmpWs &s, int nblk)
{
    q48_u128 t = 0;
    for (int b = 0; b < nblk; ++b)
        t += ((q48_u128)s.psum[2 * b + 1] << 64) | s.psum[2 * b];
    return t;
}

// ---- 4: p = fp_div(e, sum) when sum > 0 -----------------------------------
__global__ __launch_bounds__(SMP_T) void k_smp_div(int64_t *__restrict__ base, int n, int nblk)
{
    __shared__ int64_t sum_sh;
    SmpWs s = smp_ws(base, n);
    if (threadIdx.x == 0) {
        const q48_u128 t = smp_total(s, nblk);
        sum_sh = (int64_t)(uint64_t)t;   // the reference's wrapping int64 sum
        if (blockIdx.x == 0) {
            s.st[ST_SUM] = sum_sh;
            // no wrap anywhere after: every p <= ONE and their sum <= ONE
            if (!(t > 0 && t < ((q48_u128)1 << 63)))
                s.st[ST_EXACT] = 0;
        }
    }
    __syncthreads();
    const int64_t sum = sum_sh;
    if (sum > 0) {
        const q48_divisor dv = q48_divisor_of(sum);
        for (int i = blockIdx.x * SMP_T + threadIdx.x; i < n; i += gridDim.x * SMP_T)
            s.p[i] = q48_div_by(s.p[i], dv);
    }
}

// First index i (index order) at which the running sum of val(a[j]), j <= i,
// exceeds `target` (strict) or reaches it: INT_MAX if none.  Requires
// val >= 0 with no wrap (a monotone running sum).  Each wave first sums a
// contiguous range of the array with coalesced loads; the range where the
// sum crosses is then split over the lanes of one wave, and one lane walks
// its piece.  All threads of the block call it; every thread gets the
// result.
template <class F>
__device__ __forceinline__ int first_crossing(const int64_t *a, int n, F val, uint64_t target,
                                              bool strict, uint64_t *wtot, int *res)
{
    constexpr int NWV = SMP_B / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int R = (n + NWV - 1) / NWV;
    const int w0 = min(n, wave * R), w1 = min(n, w0 + R);
    uint64_t t = 0;
    for (int j0 = w0 + lane; j0 < w1; j0 += 64 * SMP_U) {
        int64_t v[SMP_U];
#pragma unroll
        for (int u = 0; u < SMP_U; ++u)
            v[u] = a[min(j0 + 64 * u, w1 - 1)];
#pragma unroll
        for (int u = 0; u < SMP_U; ++u)
            if (j0 + 64 * u < w1)
                t += val(v[u]);
    }
    t = (uint64_t)q48_wave_sum64((int64_t)t);
    __syncthreads();
    if (lane == 0)
        wtot[wave] = t;
    __syncthreads();
    // the crossing wave and the sum before it (identical in every thread)
    auto crossed = [&](uint64_t s) { return strict ? s > target : s >= target; };
    uint64_t before = 0;
    int wc = -1;
    for (int w = 0; w < NWV && wc < 0; ++w) {
        if (crossed(before + wtot[w]))
            wc = w;
        else
            before += wtot[w];
    }
    if (tid == 0)
        *res = INT_MAX;
    __syncthreads();
    if (wc >= 0 && wave == wc) {
        const int S = (R + 63) / 64;
        const int l0 = min(w1, w0 + lane * S), l1 = min(w1, l0 + S);
        uint64_t ls = 0;
        pass_chunk(a, l0, l1, [&](int, int64_t v) { ls += val(v); });
        uint64_t incl = ls;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint64_t o = __shfl_up(incl, off, 64);
            if (lane >= off)
                incl += o;
        }
        // the lane whose piece holds the crossing walks it
        uint64_t run = before + incl - ls;
        if (!crossed(run) && crossed(run + ls)) {
            int found = INT_MAX;
            pass_chunk(a, l0, l1, [&](int i, int64_t v) {
                if (found == INT_MAX) {
                    run += val(v);
                    if (crossed(run))
                        found = i;
                }
            });
            *res = found;
        }
    }
    __syncthreads();
    return *res;
}

// ---- 5: nucleus (llama_int.c:2993-3023) and the draw (3027-3036) ----------
// One block; thread t owns the index chunk [t C, (t + 1) C).  Step mode
// (st != nullptr, as k_step_argmax): the token feeds the next decode step.
__global__ __launch_bounds__(SMP_B) void k_smp_pick(int64_t *__restrict__ base, int n,
                                                   int64_t top_p, uint64_t *__restrict__ rng,
                                                   int *__restrict__ out_tok,
                                                   int *__restrict__ st, int *__restrict__ tokens,
                                                   int cap)
{
    __shared__ int64_t redv[SMP_B / 64];
    __shared__ int redi[SMP_B / 64];
    __shared__ uint64_t scan[SMP_B / 64];
    __shared__ int hcnt[256];
    __shared__ unsigned long long hsum[256];
    __shared__ int wcnt[16][256];
    __shared__ unsigned long long wsum[16][256];
    __shared__ uint64_t cut_prefix;
    __shared__ uint64_t cut_above, cut_above2;
    __shared__ int cut_all, cut_ties, cut_b;
    __shared__ int64_t r_sh;
    __shared__ int cross_i;
    __shared__ int64_t cv[SMP_B];
    __shared__ int ci[SMP_B];
    __shared__ int ccount;
    SmpWs s = smp_ws(base, n);
    const int tid = threadIdx.x;
    const int C = (n + SMP_B - 1) / SMP_B;
    const int lo = min(n, tid * C), hi = min(n, lo + C);
    int64_t *p = s.p;
    const bool nucleus = top_p > 0 && top_p < Q48_ONE;
    const bool exact = s.st[ST_EXACT] != 0;

    // Few positive probabilities (top-k on, or a peaked softmax): gather
    // them, with their indices, into LDS and finish there, one per thread
    if (exact) {
        if (tid == 0)
            ccount = 0;
        __syncthreads();
        const int lane = tid & 63;
        for (int i0 = tid; i0 < n; i0 += SMP_B * SMP_U) {
            int64_t v[SMP_U];
#pragma unroll
            for (int u = 0; u < SMP_U; ++u)
                v[u] = p[min(i0 + u * SMP_B, n - 1)];
#pragma unroll
            for (int u = 0; u < SMP_U; ++u) {
                const bool pos = i0 + u * SMP_B < n && v[u] > 0;
                const uint64_t m = __ballot(pos);
                if (m) {
                    const int leader = __ffsll((unsigned long long)m) - 1;
                    int b0 = 0;
                    if (lane == leader)
                        b0 = atomicAdd(&ccount, __popcll(m));
                    b0 = __shfl(b0, leader, 64);
                    const int k = b0 + __popcll(m & ((1ull << lane) - 1));
                    if (pos && k < SMP_B) {
                        cv[k] = v[u];
                        ci[k] = i0 + u * SMP_B;
                    }
                }
            }
        }
        __syncthreads();
    }
    if (exact && ccount <= SMP_B) {
        const int K = ccount;
        const bool have = tid < K;
        const int64_t v = have ? cv[tid] : 0;
        const int ix = have ? ci[tid] : INT_MAX;
        bool keep = have;
        if (nucleus) {
            // kept while the sum of the entries before it in the order
            // (p desc, index asc) is below top_p: a prefix of that order
            uint64_t before = 0;
            for (int j = 0; j < K; ++j) {
                const int64_t w = cv[j];
                if (w > v || (w == v && ci[j] < ix))
                    before += (uint64_t)w;
            }
            keep = have && (int64_t)before < top_p;
        }
        int64_t q = keep ? v : 0;
        if (nucleus) {
            const int64_t sum = (int64_t)blk_sum<SMP_B>((uint64_t)q, redv);
            if (sum > 0 && q > 0)
                q = q48_div_by(q, q48_divisor_of(sum));
        }
        __syncthreads();
        cv[tid] = q;   // slots past K hold 0
        __syncthreads();
        if (tid == 0) {
            const uint64_t a = rng[0];
            uint64_t b = rng[1];
            const uint64_t d = a + b;
            b ^= a;
            rng[0] = ((a << 55) | (a >> 9)) ^ b ^ (b << 14);
            rng[1] = (b << 36) | (b >> 28);
            r_sh = (int64_t)(d >> 16);
        }
        __syncthreads();
        // the running sum in index order reaches each entry's own index;
        // zero entries elsewhere add nothing
        uint64_t cum = 0;
        for (int j = 0; j < K; ++j)
            if (ci[j] <= ix)
                cum += (uint64_t)cv[j];
        int first = have && (int64_t)cum > r_sh ? ix : INT_MAX;
        int64_t dummy = 0;
        blk_argmax<SMP_B>(dummy, first, redv, redi);
        int tok = first;
        if (tok == INT_MAX) {
            // argmax of the whole vector: the first largest entry, or index 0
            // when every entry is 0
            int64_t bv = have ? q : INT64_MIN;
            int bi = have ? ix : INT_MAX;
            blk_argmax<SMP_B>(bv, bi, redv, redi);
            tok = bi != INT_MAX && bv > 0 ? bi : 0;
        }
        if (tid == 0) {
            if (st) {
                st[0] = tok;
                st[1] = st[1] + 1;
                const int k = st[2];
                if (k < cap)
                    tokens[k] = tok;
                st[2] = k + 1;
            } else {
                *out_tok = tok;
            }
        }
        return;
    }

    if (nucleus) {
        if (exact) {
            // every p in [0, ONE], sum <= ONE: the kept set is the top of
            // the order (p desc, index asc) up to the first running sum
            // >= top_p.  Radix search for the cut value p*, carrying the
            // sum above the current bucket.
            // keys p (>= 0) below the top bit of the largest; per-wave
            // histograms of counts and sums, 8 bits a pass
            int64_t pm = 0;
            pass_strided(p, n, [&](int, int64_t v) { pm = v > pm ? v : pm; });
            pm = blk_max<SMP_B>(pm, redv);
            const int top = pm > 0 ? 64 - __builtin_clzll((uint64_t)pm) : 0;
            const int wave = tid >> 6;
            if (tid == 0) {
                cut_prefix = 0;
                cut_above = 0;
                cut_all = top == 0;
            }
            __syncthreads();
            for (int hi = top; hi > 0 && !cut_all; hi -= 8) {
                const int lo = hi > 8 ? hi - 8 : 0, width = hi - lo;
                for (int b = tid; b < 16 * 256; b += SMP_B) {
                    wcnt[b >> 8][b & 255] = 0;
                    wsum[b >> 8][b & 255] = 0;
                }
                __syncthreads();
                const uint64_t prefix = cut_prefix;
                pass_strided(p, n, [&](int, int64_t sv) {
                    const uint64_t v = (uint64_t)sv;
                    if (sv > 0 && (hi >= 64 || (v >> hi) == prefix)) {
                        const int b = (int)((v >> lo) & ((1u << width) - 1));
                        atomicAdd(&wcnt[wave][b], 1);
                        atomicAdd(&wsum[wave][b], (unsigned long long)v);
                    }
                });
                __syncthreads();
                if (tid < 256) {
                    int c = 0;
                    unsigned long long t = 0;
#pragma unroll
                    for (int w = 0; w < 16; ++w) {
                        c += wcnt[w][tid];
                        t += wsum[w][tid];
                    }
                    hcnt[tid] = c;
                    hsum[tid] = t;
                }
                __syncthreads();
                if (tid == 0)
                    cut_b = -1;
                __syncthreads();
                if (tid < 64)
                    walk_sum(hcnt, hsum, 1 << width, cut_above, top_p, &cut_b, &cut_above2,
                             &cut_ties);
                __syncthreads();
                if (tid == 0) {
                    if (cut_b < 0) {
                        cut_all = 1;   // all positive mass below top_p: keep it all
                    } else {
                        cut_above = cut_above2;
                        cut_prefix = (prefix << width) | (uint64_t)cut_b;
                    }
                }
                __syncthreads();
            }
            __syncthreads();
            const int keep_all = cut_all;
            const int64_t pc = (int64_t)cut_prefix;
            // entries equal to p* join in index order until the sum reaches
            // top_p: m of them
            int64_t m = 0;
            if (!keep_all) {
                const uint64_t need = (uint64_t)top_p - cut_above;
                m = (int64_t)((need + (uint64_t)pc - 1) / (uint64_t)pc);
                m = m < cut_ties ? m : cut_ties;
            }
            // the m-th tie in index order is the last one kept (all of them
            // when m is their count)
            int last_tie = INT_MAX;
            if (!keep_all && m < cut_ties)
                last_tie = first_crossing(
                    p, n, [pc](int64_t v) -> uint64_t { return v == pc; }, (uint64_t)m, false,
                    scan, &cross_i);
            pass_strided(p, n, [&](int i, int64_t v) {
                const bool keep = keep_all ? v > 0 : v > pc || (v == pc && i <= last_tie);
                p[i] = keep ? v : 0;
            });
        } else {
            // the reference's own loop: while the running sum is below
            // top_p, take the largest positive entry (first index among
            // equals) and mark it by negating it
            int64_t cum = 0;
            while (cum < top_p) {
                int64_t bv = INT64_MIN;
                int bi = INT_MAX;
                pass_chunk(p, lo, hi, [&](int i, int64_t v) {
                    if (v > 0 && (bi == INT_MAX || v > bv)) {
                        bv = v;
                        bi = i;
                    }
                });
                blk_argmax<SMP_B>(bv, bi, redv, redi);
                if (bi == INT_MAX)
                    break;
                cum = (int64_t)((uint64_t)cum + (uint64_t)bv);
                __syncthreads();
                if (tid == 0)
                    p[bi] = (int64_t)(0 - (uint64_t)bv);
                __syncthreads();
            }
            pass_chunk(p, lo, hi, [&](int i, int64_t v) {
                p[i] = v < 0 ? (int64_t)(0 - (uint64_t)v) : 0;
            });
        }
        // renormalise the kept entries by their (wrapping) sum
        __syncthreads();
        uint64_t part = 0;
        pass_strided(p, n, [&](int, int64_t v) { part += (uint64_t)v; });
        const int64_t sum = (int64_t)blk_sum<SMP_B>(part, redv);
        if (sum > 0) {
            const q48_divisor dv = q48_divisor_of(sum);
            pass_strided(p, n, [&](int i, int64_t v) {
                if (v > 0)
                    p[i] = q48_div_by(v, dv);
            });
        }
    }

    // the draw: r in [0, ONE) from one rng_next (llama_int.c:2922-2929)
    if (tid == 0) {
        const uint64_t a = rng[0];
        uint64_t b = rng[1];
        const uint64_t v = a + b;
        b ^= a;
        rng[0] = ((a << 55) | (a >> 9)) ^ b ^ (b << 14);
        rng[1] = (b << 36) | (b >> 28);
        r_sh = (int64_t)(v >> 16);
    }
    __syncthreads();
    const int64_t r = r_sh;
    // first index whose running (wrapping) sum exceeds r
    __syncthreads();
    int tok;
    if (s.st[ST_EXACT]) {
        // every value >= 0 and the sum at most ONE: a monotone running sum
        tok = first_crossing(
            p, n, [](int64_t v) -> uint64_t { return (uint64_t)v; }, (uint64_t)r, true, scan,
            &cross_i);
    } else {
        uint64_t part = 0;
        pass_chunk(p, lo, hi, [&](int, int64_t v) { part += (uint64_t)v; });
        uint64_t run = blk_excl_scan<SMP_B>(part, scan);
        int first = INT_MAX;
        pass_chunk(p, lo, hi, [&](int i, int64_t v) {
            if (first == INT_MAX) {
                run += (uint64_t)v;
                if ((int64_t)run > r)
                    first = i;
            }
        });
        // minimum index over the block (values equal: argmax picks the
        // smaller index)
        int64_t dummy = 0;
        blk_argmax<SMP_B>(dummy, first, redv, redi);
        tok = first;
    }
    if (tok == INT_MAX) {
        // rounding left the mass below r: the first maximum (argmax)
        int64_t bv = INT64_MIN;
        int bi = INT_MAX;
        pass_chunk(p, lo, hi, [&](int i, int64_t v) {
            if (bi == INT_MAX || v > bv) {
                bv = v;
                bi = i;
            }
        });
        blk_argmax<SMP_B>(bv, bi, redv, redi);
        tok = bi == INT_MAX ? 0 : bi;
    }
    if (tid == 0) {
        if (st) {
            st[0] = tok;
            st[1] = st[1] + 1;
            const int k = st[2];
            if (k < cap)
                tokens[k] = tok;
            st[2] = k + 1;
        } else {
            *out_tok = tok;
        }
    }
}

} // namespace

size_t q48_sample_ws_words(int n) { return (size_t)ST_WORDS + 4 * SMP_GMAX + 2 * (size_t)n; }

int q48_launch_sample(q48_ctx *c, int64_t *ws, const int64_t *logits, int n, int64_t temperature,
                      int top_k, int64_t top_p, uint64_t *rng, int *out_tok, int *tokens, int cap)
{
    const int g = (n + SMP_T - 1) / SMP_T < SMP_GMAX ? (n + SMP_T - 1) / SMP_T : SMP_GMAX;
    hipLaunchKernelGGL(k_smp_scale, dim3(g), dim3(SMP_T), 0, c->stream, ws, logits, n,
                       temperature);
    hipLaunchKernelGGL(k_smp_topk, dim3(1), dim3(SMP_B), 0, c->stream, ws, n, top_k, g);
    hipLaunchKernelGGL(k_smp_exp, dim3(g), dim3(SMP_T), 0, c->stream, ws, n);
    hipLaunchKernelGGL(k_smp_div, dim3(g), dim3(SMP_T), 0, c->stream, ws, n, g);
    hipLaunchKernelGGL(k_smp_pick, dim3(1), dim3(SMP_B), 0, c->stream, ws, n, top_p, rng,
                       out_tok, tokens ? c->d_step : nullptr, tokens, cap);
    return (int)hipGetLastError();
}
