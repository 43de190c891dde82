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

// exclusive prefix sum (mod 2^64) over the threads of the block in order
template <int NT>
__device__ __forceinline__ uint64_t blk_excl_scan(uint64_t v, uint64_t *tmp)
{
    const int tid = threadIdx.x;
    __syncthreads();
    tmp[tid] = v;
    __syncthreads();
    // Hillis-Steele inclusive scan over NT entries
    for (int off = 1; off < NT; off <<= 1) {
        const uint64_t o = tid >= off ? tmp[tid - off] : 0;
        __syncthreads();
        tmp[tid] += o;
        __syncthreads();
    }
    return tmp[tid] - v;
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
    __shared__ uint64_t sel_prefix;
    __shared__ int sel_krem;
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
        if (tid == 0) {
            sel_prefix = 0;
            sel_krem = top_k;
        }
        uint64_t mask = 0;
        for (int shift = 56; shift >= 0; shift -= 8) {
            for (int b = tid; b < 256; b += SMP_B)
                hist[b] = 0;
            __syncthreads();
            const uint64_t prefix = sel_prefix;
            for (int i = tid; i < n; i += SMP_B) {
                const uint64_t key = (uint64_t)s.w[i] ^ 0x8000000000000000ull;
                if ((key & mask) == prefix)
                    atomicAdd(&hist[(key >> shift) & 255], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int krem = sel_krem, b = 255;
                for (; b > 0 && krem > hist[b]; --b)
                    krem -= hist[b];
                sel_krem = krem;
                sel_prefix = prefix | ((uint64_t)b << shift);
            }
            mask |= (uint64_t)255 << shift;
            __syncthreads();
        }
        thr = (int64_t)(sel_prefix ^ 0x8000000000000000ull);
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
    if (sum > 0)
        for (int i = blockIdx.x * SMP_T + threadIdx.x; i < n; i += gridDim.x * SMP_T)
            s.p[i] = q48_div(s.p[i], sum);
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
    __shared__ uint64_t scan[SMP_B];
    __shared__ int hcnt[256];
    __shared__ unsigned long long hsum[256];
    __shared__ uint64_t cut_prefix;
    __shared__ uint64_t cut_above;
    __shared__ int cut_all, cut_ties;
    __shared__ int64_t r_sh;
    SmpWs s = smp_ws(base, n);
    const int tid = threadIdx.x;
    const int C = (n + SMP_B - 1) / SMP_B;
    const int lo = min(n, tid * C), hi = min(n, lo + C);
    int64_t *p = s.p;

    if (top_p > 0 && top_p < Q48_ONE) {
        if (s.st[ST_EXACT]) {
            // every p in [0, ONE], sum <= ONE: the kept set is the top of
            // the order (p desc, index asc) up to the first running sum
            // >= top_p.  Radix search for the cut value p*, carrying the
            // sum above the current bucket.
            if (tid == 0) {
                cut_prefix = 0;
                cut_above = 0;
                cut_all = 0;
            }
            uint64_t mask = 0;
            for (int shift = 48; shift >= 0; shift -= 8) {
                for (int b = tid; b < 256; b += SMP_B) {
                    hcnt[b] = 0;
                    hsum[b] = 0;
                }
                __syncthreads();
                if (cut_all)
                    break;
                const uint64_t prefix = cut_prefix;
                for (int i = lo; i < hi; ++i) {
                    const uint64_t v = (uint64_t)p[i];
                    if ((int64_t)v > 0 && (v & mask) == prefix) {
                        const int b = (int)((v >> shift) & 255);
                        atomicAdd(&hcnt[b], 1);
                        atomicAdd(&hsum[b], (unsigned long long)v);
                    }
                }
                __syncthreads();
                if (tid == 0) {
                    uint64_t above = cut_above;
                    int b = 255;
                    for (; b >= 0; --b) {
                        if ((int64_t)(above + hsum[b]) >= top_p)
                            break;
                        above += hsum[b];
                    }
                    if (b < 0) {
                        cut_all = 1;   // all positive mass below top_p: keep it all
                    } else {
                        cut_above = above;
                        cut_prefix = prefix | ((uint64_t)b << shift);
                        cut_ties = hcnt[b];
                    }
                }
                mask |= (uint64_t)255 << shift;
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
            // rank of each tie: ties before this chunk, then in the chunk
            int my_ties = 0;
            if (!keep_all)
                for (int i = lo; i < hi; ++i)
                    my_ties += p[i] == pc;
            int64_t rank = (int64_t)blk_excl_scan<SMP_B>((uint64_t)my_ties, scan);
            for (int i = lo; i < hi; ++i) {
                const int64_t v = p[i];
                bool keep;
                if (keep_all) {
                    keep = v > 0;
                } else if (v == pc) {
                    keep = rank < m;
                    ++rank;
                } else {
                    keep = v > pc;
                }
                p[i] = keep ? v : 0;
            }
        } else {
            // the reference's own loop: while the running sum is below
            // top_p, take the largest positive entry (first index among
            // equals) and mark it by negating it
            int64_t cum = 0;
            while (cum < top_p) {
                int64_t bv = INT64_MIN;
                int bi = INT_MAX;
                for (int i = lo; i < hi; ++i)
                    if (p[i] > 0 && (bi == INT_MAX || p[i] > bv)) {
                        bv = p[i];
                        bi = i;
                    }
                blk_argmax<SMP_B>(bv, bi, redv, redi);
                if (bi == INT_MAX)
                    break;
                cum = (int64_t)((uint64_t)cum + (uint64_t)bv);
                __syncthreads();
                if (tid == 0)
                    p[bi] = (int64_t)(0 - (uint64_t)bv);
                __syncthreads();
            }
            for (int i = lo; i < hi; ++i)
                p[i] = p[i] < 0 ? (int64_t)(0 - (uint64_t)p[i]) : 0;
        }
        // renormalise the kept entries by their (wrapping) sum
        uint64_t part = 0;
        for (int i = lo; i < hi; ++i)
            part += (uint64_t)p[i];
        const int64_t sum = (int64_t)blk_sum<SMP_B>(part, redv);
        if (sum > 0)
            for (int i = lo; i < hi; ++i)
                if (p[i] > 0)
                    p[i] = q48_div(p[i], sum);
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
    uint64_t part = 0;
    for (int i = lo; i < hi; ++i)
        part += (uint64_t)p[i];
    uint64_t run = blk_excl_scan<SMP_B>(part, scan);
    int first = INT_MAX;
    for (int i = lo; i < hi; ++i) {
        run += (uint64_t)p[i];
        if ((int64_t)run > r) {
            first = i;
            break;
        }
    }
    int64_t dummy = 0;
    int fi = first;
    {
        // minimum index over the block (values equal: argmax picks the
        // smaller index)
        blk_argmax<SMP_B>(dummy, fi, redv, redi);
    }
    int tok = fi;
    if (tok == INT_MAX) {
        // rounding left the mass below r: the first maximum (argmax)
        int64_t bv = INT64_MIN;
        int bi = INT_MAX;
        for (int i = lo; i < hi; ++i)
            if (bi == INT_MAX || p[i] > bv) {
                bv = p[i];
                bi = i;
            }
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
