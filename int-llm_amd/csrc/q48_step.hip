// q48_step.hip — one greedy decode step (llama_forward + argmax,
// llama_int.c:2807-2893) as ONE persistent launch: k_step_fused.
//
// The multi-launch step (embed, then per layer the normed q|k|v GEMV,
// attention, the O GEMV with the residual, the normed gate|up GEMV with
// SwiGLU, the down GEMV with the residual, then the normed lm_head and
// argmax) pays each launch's ramp: the first weight loads of a GEMV go out
// only when the previous kernel has drained.  Here G = (compute units) x
// (blocks per unit) resident blocks walk the same phases in order and a
// block waits only for the phase it reads:
//  - phase p's blocks each take the row groups b, b + G, ... of the
//    projection (the k_gemv_p6 scheme: norm statistics and the staged x once
//    per block and phase, the next group's tiles issued during the current
//    group's last ones);
//  - a block issues its first weight tiles (read-only data) BEFORE it waits
//    for the producer of its x, so the weight stream keeps going across the
//    phase boundary while the dependency resolves;
//  - a phase is complete when each of its blocks has bumped the phase's
//    counter; the data a phase publishes for other compute units (q|k|v,
//    attention output, hidden, the norm partial sums, the FFN hidden, the
//    argmax partials) goes out with agent-coherent (write-through) stores
//    whose completion is awaited before the counter add, and is read with
//    agent-coherent loads, so no L2 write-back or invalidate is needed;
//  - every wait is bounded (wall clock): a wait that exceeds SK_TIMEOUT, or
//    sees another block's timeout, sets *err and every block leaves the
//    kernel, so a launch whose blocks cannot all be resident ends with an
//    error instead of hanging.  The host sizes G from the occupancy.
// Counters start at zero; block 0 resets them at the end of the step, after
// every block has passed its last wait.
//
// The arithmetic of every phase is that of the multi-launch kernels (same
// tile sums, same epilogues, the same attention body), so the logits and the
// token are bit-identical to them and to llama_forward.
#include "../../include/intllm_hip.h"
#include "q48_attn.hpp"
#include "q48_gemv_tiles.hpp"

namespace {

constexpr int SK_NW = 8, SK_NT = 64 * SK_NW;
constexpr int SK_SMAX = 512;                  // attention positions (scores in LDS)
constexpr int SK_CS = 16;                     // counter stride in uints (64 bytes)
constexpr int SK_GB = 64;                     // blocks per arrival group
constexpr int SK_PS = 32 * SK_CS;             // uints per phase: the phase counter, then
                                              // one arrival counter per group of SK_GB
                                              // blocks (up to 31 groups)
constexpr int SK_MAXG = 16;                   // row groups per block and phase (EPI 2)
constexpr uint64_t SK_TIMEOUT = 1ull << 26;   // wall-clock ticks (0.67 s at 100 MHz)

struct SkArgs {
    const char *wm;          // matrices: int64 or bfloat16 bits, element offsets below
    const int64_t *w64;      // int64 slab: embedding and norm weights
    long long off_embed, off_norm, off_lm, off_layers, layer_elems;
    long long lo_an, lo_fn, lo_qkv, lo_wo, lo_gu, lo_wd;
    int64_t *hidden, *qkv, *attn, *hf, *logits, *s_attn, *s_ffn;
    int64_t *kc, *vc;
    const int64_t *cos_t, *sin_t, *scale_p;
    int *st;                 // step state {token, pos, count}
    int *tokens;
    int cap;
    unsigned *sync;          // phase counters (SK_CS apart), zero at launch
    int *err;                // nonzero: a wait timed out
    int64_t *amax;           // argmax partials, (value, index) per block
    int L, dim, nh, nkv, hd, ffn, vocab, max_seq;
};

struct SkLds {
    uint64_t part[2][SK_NW][V4_RB][2];   // segment partial sums, by group parity
    int64_t pre[SK_MAXG][V4_RB];         // EPI 2: gate (0-3) / up (4-7) per group
    int64_t r;                           // rmsnorm r of the phase's x
    int64_t bv[SK_NW];                   // final argmax
    int bi[SK_NW];
};

// the block's LDS: the phase scratch and the staged x limbs (max(dim, ffn) x 3 words)
__shared__ SkLds sk_sh;
extern __shared__ __align__(16) uint32_t sk_xs[];

__device__ __forceinline__ int64_t ldc(const int64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void stc(int64_t *p, int64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Phase completion is counted in two levels, so that no counter takes more
// than SK_GB atomic adds per phase: a block adds 1 to its arrival group's
// counter, and the last of the group's participating blocks adds 1 to the
// phase counter, which the consumers poll.  A phase with P participating
// blocks (blocks 0 .. P - 1) is complete when the phase counter reaches
// sk_groups(P).
__device__ __forceinline__ unsigned sk_groups(unsigned parts)
{
    return (parts + SK_GB - 1) / SK_GB;
}

// Block-wide: wait until the phase counter *cnt >= target.  false on every
// thread when this or another block's wait timed out (then the caller
// leaves the kernel).
__device__ bool sk_wait(const unsigned *cnt, unsigned target, int *err)
{
    int ok = 1;
    if (threadIdx.x == 0) {
        const uint64_t t0 = wall_clock64();
        while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                ok = 0;
                break;
            }
            if (wall_clock64() - t0 > SK_TIMEOUT) {
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    return __syncthreads_and(ok) != 0;
}

// This block's part of a phase (of `parts` participating blocks) is done:
// its coherent stores have completed (each wave waits for its own), then the
// arrival (and, for the group's last block, the phase counter add).
__device__ __forceinline__ void sk_signal(unsigned *cnt, unsigned parts)
{
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned grp = blockIdx.x / SK_GB;
        const unsigned n = min((unsigned)SK_GB, parts - grp * SK_GB);
        if (__hip_atomic_fetch_add(cnt + SK_CS * (1 + grp), 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == n - 1)
            __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__device__ __forceinline__ unsigned sk_part(int ngroups)
{
    return (unsigned)min((int)gridDim.x, ngroups);
}

// One GEMV phase of the step for this block (the k_gemv_p6 body with the
// wait, coherent x and epilogue, and K = 8 NTF TE compile-time).
//  PRO 0: x as given; PRO 3: rmsnorm of x with r from the partial sums st_in.
//  EPI 0: y = v (AMAX: and this block's first maximum of y, into amax);
//  EPI 2: y = fp_mul(fp_silu(gate), up) over [gate; up] (M = 2 ffn);
//  EPI 4: y += v, and the partial sums of squares of the new 8 rows to st_out.
// Not inlined: each phase gets its own register allocation.
template <int UNR, int PRO, int EPI, int NTF, int WT, bool AMAX = false>
__device__ __noinline__ bool sk_gemv(int64_t *y, const char *Wv,
                        const int64_t *x, const int64_t *norm_w, const int64_t *st_in,
                        int64_t *st_out, int M, const unsigned *wcnt, unsigned wtarget,
                        unsigned *dcnt, int *err, int64_t *amax)
{
    static_assert(NTF % UNR == 0, "the window must divide the tiles");
    static_assert(!AMAX || EPI == 0, "argmax partials come with EPI 0");
    SkLds &sh = sk_sh;
    uint32_t *const xs = sk_xs;
    constexpr int NW = SK_NW, ES = WFmt<WT>::ES, SEG = WFmt<WT>::TE * NTF, K = SEG * NW;
    // opaque per phase: nothing derived from the thread index is hoisted out
    // of the layer loop (it would stay live, in registers, across every phase)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 3, l8 = lane & 7;
    const int ffn = M >> 1;
    const int k0 = wave * SEG;
    const int ngroups = EPI == 2 ? (ffn + 3) / 4 : (M + V4_RB - 1) / V4_RB;
    int grp = blockIdx.x;
    if (grp >= ngroups)
        return true;

    // this lane's weight row in group gi (EPI 2: gate rows 4 gi + g, then up
    // rows ffn + 4 gi + g - 4); rows past the end read row 0 (never stored)
    auto wrow = [&](int gi) {
        const int pr = gi * 4 + (g & 3);
        const int row = EPI == 2 ? (g < 4 ? pr : ffn + pr) : gi * V4_RB + g;
        const bool live = EPI == 2 ? pr < ffn : row < M;
        return reinterpret_cast<const ulonglong2 *>(Wv + ((size_t)(live ? row : 0) * K + k0) * ES) +
               l8;
    };
    // the first tiles: read-only weights, in flight while the producer of x
    // finishes
    const ulonglong2 *w2 = wrow(grp);
    ulonglong2 wa[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u)
        wa[u] = w2[u * 8];
    if (!sk_wait(wcnt, sk_groups(wtarget), err))
        return false;

    // PRO 3 partial sums, then x (and the norm weights), then the residual
    // rows of the first group: data of this launch, read coherently
    constexpr int PC = (K / 8 + 63) / 64, NP = K / 8;
    uint64_t plo[PC], phi[PC];
    if (PRO == 3) {
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            const int i = min(lane + c * 64, NP - 1);
            plo[c] = (uint64_t)ldc(st_in + 2 * i);
            phi[c] = (uint64_t)ldc(st_in + 2 * i + 1);
        }
    }
    constexpr int XB = (SEG + 127) / 128;
    int64_t xv[2 * XB], nw[2 * XB];
#pragma unroll
    for (int b = 0; b < XB; ++b) {
        const int j = min(2 * lane + 128 * b, SEG - 2);
        xv[2 * b] = ldc(x + k0 + j);
        xv[2 * b + 1] = ldc(x + k0 + j + 1);
        if (PRO != 0) {
            const ulonglong2 w = *reinterpret_cast<const ulonglong2 *>(norm_w + k0 + j);
            nw[2 * b] = (int64_t)w.x;
            nw[2 * b + 1] = (int64_t)w.y;
        }
    }
    int64_t yres = 0;
    if (EPI == 4 && wave == 0)
        yres = ldc(y + min(grp * V4_RB + (lane & 7), M - 1));

    int64_t r = 0;
    if (PRO == 3) {
        // wave 0 derives r for the block
        q48_u128 ss = 0;
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            const uint64_t m = lane + c * 64 < NP ? ~0ull : 0ull;
            ss += ((q48_u128)(phi[c] & m) << 64) | (plo[c] & m);
        }
        ss = q48_wave_sum128(ss);
        q48_keep128(ss);
        if (wave == 0) {
            const int64_t rv = rms_inv_of(ss, K);
            if (lane == 0)
                sh.r = rv;
        }
        __syncthreads();
        r = sh.r;
    }

    // stage this wave's segment of x as limbs; sum x over the segment
    uint64_t xsum = 0;
    uint32_t *xw = xs + (size_t)wave * SEG * 3;
#pragma unroll
    for (int b = 0; b < 2 * XB; ++b) {
        const int j = 2 * lane + 128 * (b / 2) + b % 2;
        int64_t v = xv[b];
        if (PRO != 0)
            v = q48_mul(q48_mul(v, r), nw[b]);
        v = j < SEG ? v : 0;
        xsum += (uint64_t)v;
        if (j < SEG) {
            const uint64_t X = (uint64_t)v ^ 0x8000000000000000ull;
            xw[3 * j] = (uint32_t)X & 0x3FFFFFu;
            xw[3 * j + 1] = (uint32_t)(X >> 22) & 0x1FFFFFu;
            xw[3 * j + 2] = WT == 1 ? (uint32_t)(v >> 43) : (uint32_t)(X >> 43);
        }
    }
    xsum = (uint64_t)q48_wave_sum64((int64_t)xsum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    int64_t best = INT64_MIN;
    int bidx = 0x7fffffff;
    int i = 0;
    for (; grp < ngroups; grp += gridDim.x, ++i) {
        const int nxt = grp + (int)gridDim.x;
        // the next group's rows; after the last group, group 0's (read by
        // every block, so they stay in cache: in bounds, never used)
        const ulonglong2 *w2n = wrow(nxt < ngroups ? nxt : 0);
        Acc6 A = {0, 0, 0, 0, 0, 0, 0};
        Acc3 F = {0, 0, 0, 0, 0, 0};
        q48_u16x2 chk = {0, 0};
#pragma unroll
        for (int t = 0; t < NTF; ++t) {
            if constexpr (WT == 0)
                mac_tile<0>(A, xw, l8, t, wa[t % UNR]);
            else
                b16_tile_fast(F, chk, xw, l8, t, wa[t % UNR]);
            if (t + UNR < NTF)
                wa[t % UNR] = w2[(t + UNR) * 8];
            else
                wa[t % UNR] = w2n[(t + UNR - NTF) * 8];
        }
        bool fast = false;
        q48_u128 S;
        if constexpr (WT == 1) {
            b16_pin(F);
            fast = b16_wave_ok(chk);
            if (fast) {
                S = acc3_value(F);
            } else {
#pragma unroll 1
                for (int t = 0; t < NTF; ++t)
                    mac_tile<1>(A, xw, l8, t, w2[t * 8]);
                S = acc6_value(A);
            }
        } else {
            S = acc6_value(A);
        }
        w2 = w2n;
        S = q48_sum8_u128(S);
        if (l8 == 0) {
            if (!fast)
                S -= (q48_u128)xsum << 63;
            sh.part[i & 1][wave][g][0] = (uint64_t)S;
            sh.part[i & 1][wave][g][1] = (uint64_t)(S >> 64);
        }
        __syncthreads();
        if (tid < V4_RB) {
            q48_u128 T = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w)
                T += ((q48_u128)sh.part[i & 1][w][tid][1] << 64) | sh.part[i & 1][w][tid][0];
            const int64_t v = (int64_t)((q48_i128)T >> 48);
            const int rr = grp * V4_RB + tid;
            if (EPI == 0) {
                if (rr < M) {
                    stc(y + rr, v);
                    if (AMAX && v > best) {   // rows ascend: the first maximum
                        best = v;
                        bidx = rr;
                    }
                }
            } else if (EPI == 2) {
                sh.pre[i][tid] = v;
            } else {
                // residual add (llama_int.c:1535, 1556), then the partial
                // sum of squares of the 8 new rows for the next rmsnorm
                int64_t h = 0;
                if (rr < M) {
                    h = (int64_t)((uint64_t)yres + (uint64_t)v);
                    stc(y + rr, h);
                }
                q48_u128 sq = (q48_u128)q48_smul128(h, h);
                sq = q48_sum8_u128(sq);
                if (tid == 0) {
                    stc(st_out + 2 * grp, (int64_t)(uint64_t)sq);
                    stc(st_out + 2 * grp + 1, (int64_t)(uint64_t)(sq >> 64));
                }
            }
        }
        if (EPI == 4 && wave == 0 && nxt < ngroups)
            yres = ldc(y + min(nxt * V4_RB + (lane & 7), M - 1));
    }
    if (EPI == 2) {
        __syncthreads();
        // SwiGLU (llama_int.c:1549-1552) of every pair this block produced
        if (tid < 4 * i) {
            const int gi = tid >> 2, q = tid & 3;
            const int pi = ((int)blockIdx.x + gi * (int)gridDim.x) * 4 + q;
            if (pi < ffn)
                stc(y + pi, q48_mul(q48_silu(sh.pre[gi][q]), sh.pre[gi][4 + q]));
        }
    }
    if (AMAX && tid < V4_RB) {
        // the block's first maximum over its rows (lanes 0-7 of wave 0)
#pragma unroll
        for (int off = 4; off >= 1; off >>= 1) {
            const int64_t ov = __shfl_xor(best, off, 8);
            const int oi = __shfl_xor(bidx, off, 8);
            if (ov > best || (ov == best && oi < bidx)) {
                best = ov;
                bidx = oi;
            }
        }
        if (tid == 0) {
            stc(amax + 2 * blockIdx.x, best);
            stc(amax + 2 * blockIdx.x + 1, bidx);
        }
    }
    sk_signal(dcnt, sk_part(ngroups));
    return true;
}

// The attention phase: block h < n_heads runs query head h once q|k|v is
// complete.
template <int HD>
__device__ __noinline__ bool sk_attn(const SkArgs &a, int l, int pos, const unsigned *wcnt,
                                     unsigned wtarget, unsigned *dcnt)
{
    if ((int)blockIdx.x >= a.nh)
        return true;
    if (!sk_wait(wcnt, sk_groups(wtarget), a.err))
        return false;
    const int kvd = a.nkv * HD;
    attn_v3_head<HD, SK_SMAX, true, false, true, SK_NT>(
        a.attn, a.qkv, a.kc, a.vc, a.qkv + a.dim, a.qkv + a.dim + kvd, a.cos_t, a.sin_t,
        a.scale_p, l, nullptr, pos, a.nh, a.nkv, a.max_seq, blockIdx.x);
    sk_signal(dcnt, sk_part(a.nh));
    return true;
}

// The step.  Phases (counter index): 0 embedding; per layer l, 1 + 5 l + 0..4:
// q|k|v, attention, O, gate|up, down; 1 + 5 L lm_head; 2 + 5 L every block
// done.  NTD / NTF: tiles per wave for K = dim / K = ffn.
template <int WT, int NTD, int NTF, int HD>
__global__ __launch_bounds__(SK_NT) __attribute__((amdgpu_waves_per_eu(4))) void
k_step_fused(SkArgs a)
{
    constexpr int ES = WFmt<WT>::ES;
    constexpr int UD = 4, UF = WT == 0 ? 4 : NTF;   // tile windows (divide NTD, NTF)
    SkLds &sh = sk_sh;
    const int tid = threadIdx.x;
    const int token = a.st[0], pos = a.st[1];
    const int dim = a.dim, kvd = a.nkv * HD, nq = dim + 2 * kvd;
    auto cnt = [&](int p) { return a.sync + (size_t)p * SK_PS; };
    if (pos < 0 || pos >= a.max_seq || pos >= SK_SMAX || token < 0 || token >= a.vocab) {
        if (blockIdx.x == 0 && tid == 0)
            __hip_atomic_store(a.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;   // uniform: every block sees the same state
    }

    // hidden = embed[token] (llama_int.c:2822-2824) and the partial sums of
    // squares of its 8-row groups (the first rmsnorm's statistics)
    if ((int)blockIdx.x < dim / V4_RB) {
        if (tid < V4_RB) {
            const int i = (int)blockIdx.x * V4_RB + tid;
            const int64_t v = a.w64[a.off_embed + (long long)token * dim + i];
            stc(a.hidden + i, v);
            q48_u128 sq = (q48_u128)q48_smul128(v, v);
            sq = q48_sum8_u128(sq);
            if (tid == 0) {
                stc(a.s_attn + 2 * blockIdx.x, (int64_t)(uint64_t)sq);
                stc(a.s_attn + 2 * blockIdx.x + 1, (int64_t)(uint64_t)(sq >> 64));
            }
        }
        sk_signal(cnt(0), sk_part(dim / V4_RB));
    }
    unsigned prev = sk_part(dim / V4_RB);

    for (int l = 0; l < a.L; ++l) {
        const long long lb = a.off_layers + (long long)l * a.layer_elems;
        const int64_t *wl64 = a.w64 + lb;
        const char *wl = a.wm + lb * ES;
        const int p0 = 1 + 5 * l;
        // rmsnorm + q|k|v (llama_int.c:1380-1390)
        if (!sk_gemv<UD, 3, 0, NTD, WT>(a.qkv, wl + a.lo_qkv * ES, a.hidden,
                                       wl64 + a.lo_an, a.s_attn, nullptr, nq, cnt(p0 - 1), prev,
                                       cnt(p0), a.err, nullptr))
            return;
        // RoPE, KV store, attention (llama_int.c:1392-1529), one block per head
        if (!sk_attn<HD>(a, l, pos, cnt(p0), sk_part(nq / V4_RB), cnt(p0 + 1)))
            return;
        // O projection + residual (llama_int.c:1531-1535)
        if (!sk_gemv<UD, 0, 4, NTD, WT>(a.hidden, wl + a.lo_wo * ES, a.attn, nullptr,
                                       nullptr, a.s_ffn, dim, cnt(p0 + 1), sk_part(a.nh),
                                       cnt(p0 + 2), a.err, nullptr))
            return;
        // rmsnorm + gate|up + SwiGLU (llama_int.c:1537-1552)
        if (!sk_gemv<UD, 3, 2, NTD, WT>(a.hf, wl + a.lo_gu * ES, a.hidden,
                                       wl64 + a.lo_fn, a.s_ffn, nullptr, 2 * a.ffn, cnt(p0 + 2),
                                       sk_part(dim / V4_RB), cnt(p0 + 3), a.err, nullptr))
            return;
        // down projection + residual (llama_int.c:1554-1556)
        if (!sk_gemv<UF, 0, 4, NTF, WT>(a.hidden, wl + a.lo_wd * ES, a.hf, nullptr,
                                       nullptr, a.s_attn, dim, cnt(p0 + 3),
                                       sk_part((a.ffn + 3) / 4), cnt(p0 + 4), a.err, nullptr))
            return;
        prev = sk_part(dim / V4_RB);
    }
    // final rmsnorm + lm_head (llama_int.c:2862-2880), with this block's
    // argmax partial
    const int pl = 1 + 5 * a.L;
    if (!sk_gemv<UD, 3, 0, NTD, WT, true>(a.logits, a.wm + a.off_lm * ES, a.hidden,
                                         a.w64 + a.off_norm, a.s_attn, nullptr, a.vocab,
                                         cnt(pl - 1), prev, cnt(pl), a.err, a.amax))
        return;
    // every block is past its last wait
    sk_signal(cnt(pl + 1), gridDim.x);
    if (blockIdx.x != 0)
        return;
    if (!sk_wait(cnt(pl + 1), sk_groups(gridDim.x), a.err))
        return;

    // argmax (llama_int.c:2888-2893): the first maximum over the partials
    const int nb = (int)sk_part((a.vocab + V4_RB - 1) / V4_RB);
    int64_t best = INT64_MIN;
    int idx = 0x7fffffff;
    for (int b = tid; b < nb; b += SK_NT) {
        const int64_t v = ldc(a.amax + 2 * b);
        const int i = (int)ldc(a.amax + 2 * b + 1);
        if (v > best || (v == best && i < idx)) {
            best = v;
            idx = i;
        }
    }
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
        sh.bv[tid >> 6] = best;
        sh.bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < SK_NW; ++w)
            if (sh.bv[w] > best || (sh.bv[w] == best && sh.bi[w] < idx)) {
                best = sh.bv[w];
                idx = sh.bi[w];
            }
        const int tok = idx < a.vocab ? idx : 0;
        a.st[0] = tok;
        a.st[1] = pos + 1;
        const int k = a.st[2];
        if (k < a.cap)
            a.tokens[k] = tok;
        a.st[2] = k + 1;
    }
    // every other block has left its waits: the counters go back to zero
    const int ng = 1 + (int)sk_groups(gridDim.x);
    for (int i = tid; i < (pl + 2) * ng; i += SK_NT)
        __hip_atomic_store(a.sync + (size_t)(i / ng) * SK_PS + (size_t)(i % ng) * SK_CS, 0u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int WT, int NTD, int NTF, int HD>
int sk_launch(q48_ctx *c, const SkArgs &a, int grid, size_t lds)
{
    hipLaunchKernelGGL((k_step_fused<WT, NTD, NTF, HD>), dim3(grid), dim3(SK_NT), lds, c->stream,
                       a);
    return (int)hipGetLastError();
}

template <int WT, int NTD, int NTF, int HD>
int sk_blocks_per_cu(size_t lds)
{
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_step_fused<WT, NTD, NTF, HD>, SK_NT,
                                                     lds) != hipSuccess)
        return 0;
    return nb;
}

// the shapes instantiated: TinyLlama-1.1B's dim 2048, ffn 5632, head_dim 64
constexpr int SK_DIM = 2048, SK_FFN = 5632, SK_HD = 64;

} // namespace

int q48_step_fused_max_pos(void) { return SK_SMAX; }

// 0 when the step kernel serves this model (grid and LDS set), else a
// negative code.
int q48_step_fused_plan(q48_ctx *c, const q48_step_model *m, int *grid, size_t *lds)
{
    if (m->dim != SK_DIM || m->ffn != SK_FFN || m->head_dim != SK_HD || m->n_heads <= 0 ||
        m->n_kv_heads <= 0 || m->n_heads % m->n_kv_heads || m->n_layers <= 0 ||
        m->vocab <= 0 || (m->wfmt != 0 && m->wfmt != 1))
        return Q48_EINVAL;
    *lds = (size_t)(m->dim > m->ffn ? m->dim : m->ffn) * 12;
    const int nb = m->wfmt == 0 ? sk_blocks_per_cu<0, 16, 44, SK_HD>(*lds)
                                : sk_blocks_per_cu<1, 4, 11, SK_HD>(*lds);
    if (nb <= 0)
        return Q48_EINVAL;
    const int g = c->cu_count * (nb < 2 ? nb : 2);
    // every head needs a block; the gate|up groups of a block fit its LDS;
    // at most 31 arrival groups
    if (g < m->n_heads || ((m->ffn + 3) / 4 + g - 1) / g > SK_MAXG || g > 31 * SK_GB)
        return Q48_EINVAL;
    *grid = g;
    return Q48_OK;
}

int q48_launch_step_fused(q48_ctx *c, const q48_step_model *m, int *tokens, int cap, int grid,
                          size_t lds)
{
    SkArgs a;
    a.wm = static_cast<const char *>(m->wmat);
    a.w64 = m->w;
    a.off_embed = (long long)m->off_embed;
    a.off_norm = (long long)m->off_norm;
    a.off_lm = (long long)m->off_lm;
    a.off_layers = (long long)m->off_layers;
    a.layer_elems = (long long)m->layer_elems;
    a.lo_an = (long long)m->lo_an;
    a.lo_fn = (long long)m->lo_fn;
    a.lo_qkv = (long long)m->lo_qkv;
    a.lo_wo = (long long)m->lo_wo;
    a.lo_gu = (long long)m->lo_gu;
    a.lo_wd = (long long)m->lo_wd;
    a.hidden = m->hidden;
    a.qkv = m->qkv;
    a.attn = m->attn;
    a.hf = m->h_ffn;
    a.logits = m->logits;
    a.s_attn = m->s_attn;
    a.s_ffn = m->s_ffn;
    a.kc = m->kcache;
    a.vc = m->vcache;
    a.cos_t = c->rope_cos;
    a.sin_t = c->rope_sin;
    a.scale_p = c->rope_sin + (size_t)c->rope_max_seq * (c->rope_head_dim / 2);
    a.st = c->d_step;
    a.tokens = tokens;
    a.cap = cap;
    a.sync = c->sk_sync;
    a.err = c->sk_err;
    a.amax = c->sk_amax;
    a.L = m->n_layers;
    a.dim = m->dim;
    a.nh = m->n_heads;
    a.nkv = m->n_kv_heads;
    a.hd = m->head_dim;
    a.ffn = m->ffn;
    a.vocab = m->vocab;
    a.max_seq = m->max_seq;
    return m->wfmt == 0 ? sk_launch<0, 16, 44, SK_HD>(c, a, grid, lds)
                        : sk_launch<1, 4, 11, SK_HD>(c, a, grid, lds);
}
