// q48_gemv.hip — exact Q16.48 GEMV / GEMM for gfx950 (VALU limb arithmetic).
//
// Contract (matmul_vec, llama_int.c:1014-1046):
//     y[i] = (int64)( (sum_j (int128) W[i][j] * x[j]) >> 48 )
// with W row-major [M][K].  Only bits [48, 112) of the two's-complement
// sum reach y, so any summation order mod 2^128 is bit-exact.
//
// Limb scheme (offset binary).  Flip the sign bit of both operands:
//     X' = x ^ 2^63 = x + 2^63,   W' = w ^ 2^63 = w + 2^63   (unsigned)
//     x*w = X'W' - 2^63 (X' + W') + 2^126
// X'W' is a product of unsigned 64-bit numbers, i.e. four unsigned 32x32
// partials, each one v_mad_u64_u32 with a 64-bit accumulate.  Summed over
// j, the 2^126 terms only touch bits 126-127, and 2^63 (X' + W') mod 2^112
// only depends on (sum x + sum w) mod 2^49 — one 64-bit running sum per
// lane, plus a per-row sum of x shared by every row.  Per MAC per lane:
//     a0 += xl*wl  (carry count c0)     bits   0..  (64 + log2 K)
//     a1 += xh*wl + xl*wh  (carry c1)   bits  32..
//     a2 += xh*wh  (mod 2^64)           bits  64..127
//     ws += w      (mod 2^64)
// then S = a0 + 2^64 c0 + 2^32 a1 + 2^96 c1 + 2^64 a2 - 2^63 (ws + xs).
//
// GEMV layout: one wavefront per output row (64 lanes x 16 B = 1 KiB per
// load instruction, fully coalesced), x staged once per block in LDS in
// flipped form, rows-per-block waves sharing it; 128-bit cross-lane sum.
#include "q48_internal.h"

namespace {

struct LimbAcc {
    uint64_t a0, a1, a2, ws;
    uint32_t c0, c1;
};

__device__ __forceinline__ void mac_flip(LimbAcc &A, uint32_t xl, uint32_t xh,
                                         uint64_t w)
{
    const uint32_t wl = (uint32_t)w;
    const uint32_t wh = (uint32_t)(w >> 32) ^ 0x80000000u;
    uint64_t s;
    s = (uint64_t)xl * wl + A.a0;
    A.c0 += s < A.a0;
    A.a0 = s;
    s = (uint64_t)xh * wl + A.a1;
    A.c1 += s < A.a1;
    A.a1 = s;
    s = (uint64_t)xl * wh + A.a1;
    A.c1 += s < A.a1;
    A.a1 = s;
    A.a2 += (uint64_t)xh * wh;
    A.ws += w;
}

__device__ __forceinline__ q48_u128 acc_value(const LimbAcc &A)
{
    q48_u128 S = (q48_u128)A.a0;
    S += (q48_u128)A.c0 << 64;
    S += (q48_u128)A.a1 << 32;
    S += (q48_u128)A.c1 << 96;
    S += (q48_u128)A.a2 << 64;
    S -= (q48_u128)A.ws << 63;
    return S;
}

constexpr int KCHUNK = 4096;   // x elements staged per pass (32 KiB LDS)

// RPB waves per block, one row per wave.  VEC = 2: 16-byte loads (K even,
// W 16-byte aligned); VEC = 1: 8-byte loads (any K).
template <int RPB, int VEC>
__global__ __launch_bounds__(64 * RPB) void k_gemv(int64_t *__restrict__ y,
                                                   const int64_t *__restrict__ W,
                                                   const int64_t *__restrict__ x,
                                                   int M, int K)
{
    __shared__ __align__(16) uint64_t xs[KCHUNK];
    __shared__ uint64_t xsum_w[RPB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int row = blockIdx.x * RPB + wave;
    const bool active = row < M;
    const int64_t *wr = W + (size_t)(active ? row : 0) * (size_t)K;

    LimbAcc A = {0, 0, 0, 0, 0, 0};
    uint64_t xsum = 0;

    for (int k0 = 0; k0 < K; k0 += KCHUNK) {
        const int kc = min(KCHUNK, K - k0);
        __syncthreads();
        for (int j = tid; j < kc; j += 64 * RPB) {
            uint64_t v = (uint64_t)x[k0 + j];
            xs[j] = v ^ 0x8000000000000000ull;
            xsum += v;
        }
        __syncthreads();
        if (active) {
            if (VEC == 2) {
                const ulonglong2 *w2 = reinterpret_cast<const ulonglong2 *>(wr + k0);
                const uint4 *x4 = reinterpret_cast<const uint4 *>(xs);
                const int np = kc >> 1;
                int p = lane;
                for (; p + 192 < np; p += 256) {
                    ulonglong2 wa = w2[p], wb = w2[p + 64], wc = w2[p + 128], wd = w2[p + 192];
                    uint4 xa = x4[p], xb = x4[p + 64], xc = x4[p + 128], xd = x4[p + 192];
                    mac_flip(A, xa.x, xa.y, wa.x);
                    mac_flip(A, xa.z, xa.w, wa.y);
                    mac_flip(A, xb.x, xb.y, wb.x);
                    mac_flip(A, xb.z, xb.w, wb.y);
                    mac_flip(A, xc.x, xc.y, wc.x);
                    mac_flip(A, xc.z, xc.w, wc.y);
                    mac_flip(A, xd.x, xd.y, wd.x);
                    mac_flip(A, xd.z, xd.w, wd.y);
                }
                for (; p < np; p += 64) {
                    ulonglong2 wa = w2[p];
                    uint4 xa = x4[p];
                    mac_flip(A, xa.x, xa.y, wa.x);
                    mac_flip(A, xa.z, xa.w, wa.y);
                }
            } else {
                const uint2 *x2 = reinterpret_cast<const uint2 *>(xs);
                for (int j = lane; j < kc; j += 64) {
                    uint64_t wv = (uint64_t)wr[k0 + j];
                    uint2 xa = x2[j];
                    mac_flip(A, xa.x, xa.y, wv);
                }
            }
        }
    }

    // sum of x over the whole row (shared by every row of the block)
    xsum = (uint64_t)q48_wave_sum64((int64_t)xsum);
    if (lane == 0)
        xsum_w[wave] = xsum;
    __syncthreads();
    if (!active)
        return;
    uint64_t xtot = 0;
#pragma unroll
    for (int w = 0; w < RPB; ++w)
        xtot += xsum_w[w];

    q48_u128 S = q48_wave_sum128(acc_value(A));
    S -= (q48_u128)xtot << 63;
    if (lane == 0)
        y[row] = (int64_t)((q48_i128)S >> 48);
}

// ---------------------------------------------------------------------------
// GEMV v5 (the decode kernel).
//
// Carry-free limbs.  x is shared by every row, so it is split once, when it
// is staged, into three limbs of its flipped value X' = x ^ 2^63:
//     X' = x0 + 2^22 x1 + 2^43 x2,   x0 < 2^22, x1, x2 < 2^21,
// and each weight into two 32-bit limbs of W' = w ^ 2^63.  Every partial
// product x_i * w_j is below 2^54, so a 64-bit accumulator holds the sum of
// up to 1024 of them exactly: six v_mad_u64_u32 per MAC and no carry
// handling.  A lane sums 2 products per 16-element tile of its segment,
// at most seg / 8 <= 192 per accumulator (K <= V2_MAX_K).  At the end
//     S = a00 + 2^32 a01 + 2^22 a10 + 2^54 a11 + 2^43 a20 + 2^75 a21
//         - 2^63 (sum w + sum x)                                 (mod 2^128)
// (the offset-binary identity above), and y = (int64)(S >> 48).
//
// Layout.  8 rows per block, one 8-lane group per row (each load
// instruction of a group reads one full 128-byte line of its row), NW
// waves per block each taking one K-segment of all 8 rows.  Each wave
// stages only its own segment of x, so no block-wide barrier sits between
// the prologue and the loads; the segment partials meet in LDS at the end.
//
// Latency.  A lane issues its x loads, then its first UNR weight tiles,
// and only then waits, for x alone, to stage it: the weights arrive
// meanwhile.  vmcnt retires loads in issue order, so that order and
// unconditional (clamped) loads are what keep the compiler's waits partial.
// For the decode shapes (16 or 44 tiles per wave) the tiles then flow
// through a rotating window of UNR = 4 or 6 loads: multiply tile t, issue
// tile t + UNR.  Issuing every tile up front instead stalls the wave on
// the full memory pipeline with no work to overlap (measured: 10-20% slower).
//
// Prologues (the staged x is exactly what rmsnorm, llama_int.c:1048-1058,
// would write):  PRO 0: x as given;  PRO 1: every block computes the
// rmsnorm statistics of x itself and stages fp_mul(fp_mul(x, r), norm_w);
// PRO 2: the same with r = *r_in, computed once by the producer of x;
// PRO 3: the same with r computed in the block from the producer's partial
// sums of squares (r_in points at them: ceil(K / 8) 128-bit values).
// Epilogues:  EPI 0 stores y;  EPI 1 adds y into `y` (the residual adds,
// llama_int.c:1535, 1556);  EPI 2 reads W as [gate; up] (M = 2 ffn):
// block b takes gate rows 4b..4b+3 (groups 0-3) and the matching up rows
// ffn+4b.. (groups 4-7) and stores fp_mul(fp_silu(gate), up)
// (llama_int.c:1549-1552);  EPI 3 is EPI 1 followed by the statistics of
// the next rmsnorm of the updated vector: each block writes its partial sum
// of squares, the last block to finish adds them all and writes
// r = fp_inv_sqrt((int64)((ss >> 48) / M) + 2814749767) to *r_out;
// EPI 4 is EPI 1 followed by the block's partial sum of squares of its 8
// new rows, stored at r_out[2 b], r_out[2 b + 1] (lo, hi) for a PRO 3
// consumer: no atomics, no waits, no last block.
// ---------------------------------------------------------------------------
} // namespace

#include "q48_gemv_tiles.hpp"

namespace {

// A 16-byte weight tile.  int64 weights (WT 0) are read once per token and
// far exceed the caches (8.3 GB against a 256 MB MALL), so they go out as
// non-temporal loads: measured 1.861 against 1.955 ms per TinyLlama-shape
// decode token.  bfloat16 tiles (WT 1) keep ordinary loads (their kernels are
// VALU-bound, and non-temporal loads measured slower there: 1.69 against 1.58).
template <int WT>
__device__ __forceinline__ ulonglong2 ld_wtile(const ulonglong2 *p)
{
    if constexpr (WT == 0) {
        typedef unsigned long long v2u __attribute__((ext_vector_type(2)));
        const v2u v = __builtin_nontemporal_load(reinterpret_cast<const v2u *>(p));
        return make_ulonglong2(v.x, v.y);
    } else {
        return *p;
    }
}

template <int NW, int UNR, int PRO, int EPI, int NTF, int WT = 0>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4))) void k_gemv_v5(int64_t *__restrict__ y,
                                                    const void *__restrict__ Wv,
                                                    const int64_t *__restrict__ x,
                                                    const int64_t *__restrict__ norm_w,
                                                    const int64_t *__restrict__ r_in,
                                                    int64_t *__restrict__ r_out,
                                                    uint64_t *__restrict__ rms_part,
                                                    int *__restrict__ rms_count,
                                                    int M, int K, int seg, const q48_ropekv rk)
{
    extern __shared__ __align__(16) uint32_t xs[];   // 3 limbs per staged x
    __shared__ uint64_t red_lo[NW], red_hi[NW];
    __shared__ uint64_t part[NW][V4_RB][2];
    __shared__ int64_t r_sh;
    __shared__ int last_sh;

    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform (scalar) so that the segment bounds and the tile loop
    // branch uniformly
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 3, l8 = lane & 7;
    const int row0 = blockIdx.x * V4_RB;
    const int ffn = M >> 1;
    const int k0 = wave * seg;
    const int kn = max(0, min(seg, K - k0));

    // row of group g (EPI 2: gate rows 4b+g, then up rows ffn+4b+g-4; EPI 5:
    // the RoPE pairs i = j0 + (g & 3) and i + hd / 2 of head hh, hd / 8
    // blocks per head; hd a power of two, so shifts)
    const int pr = blockIdx.x * 4 + (g & 3);
    int hh = 0, j0 = 0;
    if (EPI == 5) {
        const int sh = 28 - __builtin_clz((unsigned)rk.hd);   // log2(hd / 8)
        hh = (int)blockIdx.x >> sh;
        j0 = 4 * ((int)blockIdx.x & ((1 << sh) - 1));
    }
    const int row = EPI == 2   ? (g < 4 ? pr : ffn + pr)
                    : EPI == 5 ? hh * rk.hd + j0 + (g & 3) + (g < 4 ? 0 : rk.hd >> 1)
                               : row0 + g;
    const bool live = EPI == 2 ? pr < ffn : row < M;
    // EPI 5: the position, read first (a scalar load through the constant
    // address space, so that no vector-memory wait has to cover it)
    int p5 = 0;
    if constexpr (EPI == 5) {
        typedef const __attribute__((address_space(4))) int cint;
        p5 = rk.d_pos ? *(cint *)rk.d_pos : rk.pos;
    }
    // rows past the end read row 0 (in bounds, never accumulated)
    constexpr int ES = WFmt<WT>::ES, SEGC = WFmt<WT>::TE * NTF;
    const ulonglong2 *w2 = reinterpret_cast<const ulonglong2 *>(
                               static_cast<const char *>(Wv) +
                               ((size_t)(live ? row : 0) * K + k0) * ES) + l8;
    const int nt = kn / WFmt<WT>::TE;   // whole tiles of the segment

    // the residual rows this block adds to (EPI 1, 3, 4): read now, used last
    constexpr bool RES = EPI == 1 || EPI == 3 || EPI == 4;
    int64_t yres = 0;
    if (RES && tid < V4_RB && row0 + tid < M)
        yres = y[row0 + tid];

    // PRO 3: the norm statistics arrive as the producer's per-8-row partial
    // sums of squares (128-bit lo/hi pairs, ceil(K / 8) of them, at most 3
    // per thread); their loads go out first, with the residual's
    // With NTF known each lane preloads np / 64 of the np = K / 8 = 2 NW NTF
    // partials (16-byte aligned, checked on the host); otherwise they are
    // read in a loop when needed.
    constexpr int PC = NTF > 0 ? (NW * SEGC / 8 + 63) / 64 : 1;
    uint64_t plo[PC], phi[PC];
    const int np = (K + 7) >> 3;
    const uint64_t *st = reinterpret_cast<const uint64_t *>(r_in);
    if (PRO == 3 && NTF > 0 && wave == 0) {
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            const int i = min(lane + c * 64, np - 1);
            const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(st + 2 * i);
            plo[c] = v.x;
            phi[c] = v.y;
        }
    }

    int64_t r = 0;
    if (PRO == 1) {
        // whole-x statistics in every block (ssq over K, 64 NW threads)
        constexpr int SB = 8;
        q48_u128 ss = 0;
        for (int j0 = 0; j0 < K; j0 += 64 * NW * SB) {
            int64_t v[SB];
#pragma unroll
            for (int b = 0; b < SB; ++b) {
                const int j = j0 + tid + b * 64 * NW;
                v[b] = j < K ? x[j] : 0;
            }
#pragma unroll
            for (int b = 0; b < SB; ++b)
                ss += (q48_u128)q48_smul128(v[b], v[b]);
        }
        ss = block_sum128<64 * NW>(ss, red_lo, red_hi);
        if (tid == 0)
            r_sh = rms_inv_of(ss, K);
        __syncthreads();
        r = r_sh;
    } else if (PRO == 2) {
        r = *r_in;
    }

    // Issue order matters: vmcnt retires loads in issue order, so the x (and
    // norm weight) loads of the first staging batch go out before the first
    // batch of weights; staging then waits for x only while the weights are
    // still in flight.  Every load below is unconditional (clamped index) so
    // the wait counts stay static.
    // (A wave with an empty segment or no whole tile reads element 0 of x
    // and of W instead: in bounds, never used.)
    // x values per lane per staging batch: exactly the segment when every
    // wave has NTF tiles (16 NTF elements), else 8 or 16 per batch
    // With NTF known every wave's segment is exactly 16 NTF elements and x,
    // norm_w are 16-byte aligned (checked on the host): a lane loads element
    // pairs, 16 bytes at a time.  Otherwise single elements, 8 or 16 of them
    // per lane per staging batch.
    constexpr int XB = NTF > 0 ? (SEGC + 127) / 128 : (PRO ? 8 : 16);
    constexpr int XW = NTF > 0 ? 2 : 1;   // elements per load
    int64_t xv[XB * XW], nw[XB * XW];
    const int xk = kn > 0 ? k0 : 0, xlast = max(kn - XW, 0);
#pragma unroll
    for (int b = 0; b < XB; ++b) {
        const int j = min(XW * lane + 64 * XW * b, xlast);
        if constexpr (XW == 2) {
            const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(x + xk + j);
            xv[2 * b] = (int64_t)v.x;
            xv[2 * b + 1] = (int64_t)v.y;
            if (PRO != 0) {
                const ulonglong2 w = *reinterpret_cast<const ulonglong2 *>(norm_w + xk + j);
                nw[2 * b] = (int64_t)w.x;
                nw[2 * b + 1] = (int64_t)w.y;
            }
        } else {
            xv[b] = x[xk + j];
            if (PRO != 0)
                nw[b] = norm_w[xk + j];
        }
    }
    asm volatile("" ::: "memory");   // keep the x loads ahead of the weight loads
    const ulonglong2 *wt = nt > 0 ? w2 : reinterpret_cast<const ulonglong2 *>(Wv);
    const int tlast = max(nt - 1, 0), tstep = nt > 0 ? 8 : 0;
    ulonglong2 wa[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u)
        wa[u] = ld_wtile<WT>(&wt[min(u, tlast) * tstep]);
    // nothing that waits on a load may be scheduled above this point
    __builtin_amdgcn_sched_barrier(0);

    // EPI 5: this block's four cos / sin pairs at the position, issued
    // behind the first weight tiles and used only by the epilogue; every
    // lane loads (lane & 3's pair, clamped row) so that the loads stay here
    int64_t c5 = 0, s5 = 0;
    if constexpr (EPI == 5) {
        const int pc = min(max(p5, 0), rk.max_seq - 1), half = rk.hd >> 1;
        const size_t at = (size_t)pc * half + j0 + (lane & 3);
        c5 = rk.cos_t[at];
        s5 = rk.sin_t[at];
        __builtin_amdgcn_sched_barrier(0);
    }

    if (PRO == 3) {
        // wave 0 alone loads and adds the producer's partials and derives r;
        // the others meet it at the barrier.  Loaded by every wave, the
        // partials (4 KB per wave) would queue ahead of each wave's x and
        // weight loads in the CU's load path, and the chain of 64 x 64-bit
        // products inside rms_inv_of would contend for the SIMDs
        if (wave == 0) {
            q48_u128 ss = 0;
            if constexpr (NTF > 0) {
#pragma unroll
                for (int c = 0; c < PC; ++c) {
                    // masked, not branched: a branch would sink the load and wait
                    const uint64_t m = lane + c * 64 < np ? ~0ull : 0ull;
                    ss += ((q48_u128)(phi[c] & m) << 64) | (plo[c] & m);
                }
            } else {
                for (int i = lane; i < np; i += 64)
                    ss += ((q48_u128)st[2 * i + 1] << 64) | st[2 * i];
            }
            ss = q48_wave_sum128(ss);
            const int64_t rv = rms_inv_of(ss, K);
            if (lane == 0)
                r_sh = rv;
        }
        __syncthreads();
        r = r_sh;
    }

    // stage this wave's segment of x as limbs; sum x over the segment
    uint64_t xsum = 0;
    uint32_t *xw = xs + (size_t)wave * seg * 3;
    auto stage = [&](int j0) {
#pragma unroll
        for (int b = 0; b < XB * XW; ++b) {
            // the loaded value is used outside the branch so that its load
            // is not sunk into it (a load there would wait for the weights)
            const int j = j0 + XW * lane + 64 * XW * (b / XW) + b % XW;
            int64_t v = xv[b];
            if (PRO != 0)
                v = q48_mul(q48_mul(v, r), nw[b]);
            v = j < kn ? v : 0;
            xsum += (uint64_t)v;
            if (j < kn) {
                const uint64_t X = (uint64_t)v ^ 0x8000000000000000ull;
                xw[3 * j] = (uint32_t)X & 0x3FFFFFu;
                xw[3 * j + 1] = (uint32_t)(X >> 22) & 0x1FFFFFu;
                // bfloat16 weights: the signed top limb (b16_tile_fast)
                xw[3 * j + 2] = WT == 1 ? (uint32_t)(v >> 43) : (uint32_t)(X >> 43);
            }
        }
    };
    stage(0);   // straight-line: the loads above stay where they are
    for (int j0 = 64 * XB; NTF == 0 && j0 < kn; j0 += 64 * XB) {
#pragma unroll
        for (int b = 0; b < XB; ++b) {
            const int j = min(j0 + lane + 64 * b, kn - 1);
            xv[b] = x[k0 + j];
            if (PRO != 0)
                nw[b] = norm_w[k0 + j];
        }
        stage(j0);
    }
    xsum = (uint64_t)q48_wave_sum64((int64_t)xsum);
    // the segment is read only by the wave that wrote it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // The first UNR tiles were issued before the staging; a segment of at
    // most UNR tiles (K <= 8 * 16 * UNR) needs no further weight loads.
    // Longer segments continue in batches of UNR (clamped, unconditional
    // loads).  Rows past the end (reading row 0) accumulate too, without
    // branching, and are never stored.
    Acc6 A = {0, 0, 0, 0, 0, 0, 0};
    Acc3 F = {0, 0, 0, 0, 0, 0};
    q48_u16x2 chk = {0, 0};
    // one tile: the int64 weights, or the fast form of the bfloat16 ones
    auto tile = [&](int t, ulonglong2 w) {
        if constexpr (WT == 0)
            mac_tile<0>(A, xw, l8, t, w);
        else
            b16_tile_fast(F, chk, xw, l8, t, w);
    };
    const uint32_t *xl = xw + 6 * l8;   // this lane's pair: 6 limbs per tile of 16
    if constexpr (NTF > 0) {
        // every wave has exactly NTF tiles: a rotating window of UNR loads in
        // flight, unrolled so that each wait is for one tile and each issue
        // follows a multiply (the wave does useful work while the memory
        // pipeline is full instead of stalling on a long run of issues)
#pragma unroll
        for (int t = 0; t < NTF; ++t) {
            tile(t, wa[t % UNR]);
            if (t + UNR < NTF)
                wa[t % UNR] = ld_wtile<WT>(&w2[(t + UNR) * 8]);
        }
    } else {
#pragma unroll
        for (int u = 0; u < UNR; ++u)
            if (u < nt)
                tile(u, wa[u]);
        for (int t0 = UNR; t0 < nt; t0 += UNR) {
#pragma unroll
            for (int u = 0; u < UNR; ++u)
                wa[u] = ld_wtile<WT>(&w2[min(t0 + u, nt - 1) * 8]);
#pragma unroll
            for (int u = 0; u < UNR; ++u)
                if (t0 + u < nt)
                    tile(t0 + u, wa[u]);
        }
    }
    // bfloat16: the fast sums plus, when a pattern outside the fast window
    // is anywhere in the wave's tiles (rare), their residuals
    q48_u128 S;
    if constexpr (WT == 1) {
        b16_pin(F);
        S = acc3_value(F);
        if (!b16_wave_ok(chk)) {
            // every tile of the segment is still in the window's registers
            // when the window holds the whole segment; else read again
            // (up to 4 tiles: holding 11 spills registers)
            if constexpr (NTF > 0 && NTF == UNR && NTF <= 4)
                b16_fix_regs(S, wa, [&](int t) { return xw + 3 * (64 * t + 8 * l8); });
            else
                b16_fix_tiles(
                    S, nt, [&](int t) { return w2[t * 8]; },
                    [&](int t) { return xw + 3 * (64 * t + 8 * l8); });
        }
    } else {
        // the kn % 16 elements (even) of the segment's end, one pair per lane
        if (2 * l8 < (kn & 15)) {
            const ulonglong2 w1 = w2[nt * 8];
            const uint32_t *p = xl + 48 * nt;
            mac6(A, p[0], p[1], p[2], w1.x);
            mac6(A, p[3], p[4], p[5], w1.y);
        }
        S = acc6_value(A);
    }
    S = q48_sum8_u128(S);
    if (l8 == 0) {
        if constexpr (WT == 0)
            S -= (q48_u128)xsum << 63;
        part[wave][g][0] = (uint64_t)S;
        part[wave][g][1] = (uint64_t)(S >> 64);
    }
    __syncthreads();

    if (EPI == 4) {
        // residual add, then this block's partial sum of squares of its 8 new
        // rows for the consumer's PRO 3 (no cross-block step here)
        if (tid < V4_RB) {
            q48_u128 T = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w)
                T += ((q48_u128)part[w][tid][1] << 64) | part[w][tid][0];
            const int64_t v = (int64_t)((q48_i128)T >> 48);
            const int rr = row0 + tid;
            int64_t h = 0;
            if (rr < M) {
                h = (int64_t)((uint64_t)yres + (uint64_t)v);
                y[rr] = h;
            }
            q48_u128 sq = (q48_u128)q48_smul128(h, h);
            sq = q48_sum8_u128(sq);
            if (tid == 0) {
                uint64_t *st = reinterpret_cast<uint64_t *>(r_out);
                st[2 * blockIdx.x] = (uint64_t)sq;
                st[2 * blockIdx.x + 1] = (uint64_t)(sq >> 64);
            }
        }
        return;
    }

    if (EPI == 3) {
        // residual add, then this block's sum of squares of the new rows
        if (tid < V4_RB) {
            q48_u128 T = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w)
                T += ((q48_u128)part[w][tid][1] << 64) | part[w][tid][0];
            const int64_t v = (int64_t)((q48_i128)T >> 48);
            const int rr = row0 + tid;
            int64_t h = 0;
            if (rr < M) {
                h = (int64_t)((uint64_t)yres + (uint64_t)v);
                y[rr] = h;
            }
            q48_u128 sq = (q48_u128)q48_smul128(h, h);
            sq = q48_sum8_u128(sq);
            if (tid == 0) {
                // The partial goes out with agent-coherent (write-through)
                // stores; waiting for them to complete before the ticket
                // increment orders them before it for every block.  No other
                // data is published through the ticket, so the L2 write-back
                // and invalidate of a full agent-scope release/acquire are not
                // needed: the last block reads the partials with
                // agent-coherent loads.
                __hip_atomic_store(&rms_part[2 * blockIdx.x], (uint64_t)sq, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&rms_part[2 * blockIdx.x + 1], (uint64_t)(sq >> 64),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0);
                const int ticket = __hip_atomic_fetch_add(rms_count, 1, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
                last_sh = ticket == (int)gridDim.x - 1;
            }
        }
        __syncthreads();
        if (!last_sh)
            return;
        // last block: every partial is visible (each was complete before its
        // block's ticket); the whole block adds them (integer sum: any order
        // gives the bits)
        q48_u128 ss = 0;
        for (unsigned b = tid; b < gridDim.x; b += 64 * NW) {
            const uint64_t lo =
                __hip_atomic_load(&rms_part[2 * b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t hi = __hip_atomic_load(&rms_part[2 * b + 1], __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
            ss += ((q48_u128)hi << 64) | lo;
        }
        ss = block_sum128<64 * NW>(ss, red_lo, red_hi);
        if (tid == 0) {
            *r_out = rms_inv_of(ss, M);
            __hip_atomic_store(rms_count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    if (tid >= V4_RB)
        return;
    q48_u128 T = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w)
        T += ((q48_u128)part[w][tid][1] << 64) | part[w][tid][0];
    const int64_t v = (int64_t)((q48_i128)T >> 48);
    const int rr = row0 + tid;
    if (EPI == 0) {
        if (rr < M)
            y[rr] = v;
    } else if (EPI == 5) {
        // threads 0-3 hold dims i = j0 + tid of head hh, 4-7 dims i + hd / 2;
        // RoPE of the q and k heads (rope_apply, llama_int.c:997-1008), then
        // k and v to the caches at pos (llama_int.c:1414-1416)
        // (the partner row tid ^ 4 summed here too: no cross-lane step)
        const int half = rk.hd >> 1, d = j0 + (tid & 3) + (tid < 4 ? 0 : half);
        q48_u128 T2 = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w)
            T2 += ((q48_u128)part[w][tid ^ 4][1] << 64) | part[w][tid ^ 4][0];
        const int64_t o = (int64_t)((q48_i128)T2 >> 48);
        int64_t r5 = v;
        if (hh < rk.n_heads + rk.n_kv)
            r5 = tid < 4 ? (int64_t)((uint64_t)q48_mul(v, c5) - (uint64_t)q48_mul(o, s5))
                         : (int64_t)((uint64_t)q48_mul(v, c5) + (uint64_t)q48_mul(o, s5));
        const int rw = hh * rk.hd + d;
        if (rw < M)
            y[rw] = r5;
        if (hh >= rk.n_heads && rw < M && p5 >= 0 && p5 < rk.max_seq) {
            const bool isk = hh < rk.n_heads + rk.n_kv;
            const int kh = hh - rk.n_heads - (isk ? 0 : rk.n_kv);
            int64_t *cache = isk ? rk.kc : rk.vc;
            cache[((size_t)rk.layer * rk.max_seq + p5) * ((size_t)rk.n_kv * rk.hd) +
                  (size_t)kh * rk.hd + d] = r5;
        }
    } else if (EPI == 1) {
        if (rr < M)
            y[rr] = (int64_t)((uint64_t)yres + (uint64_t)v);
    } else {
        // threads 0-3 hold gate rows, 4-7 the matching up rows
        const int64_t up = __shfl_down(v, 4, 64);
        const int i = blockIdx.x * 4 + tid;
        if (tid < 4 && i < ffn)
            y[i] = q48_mul(q48_silu(v), up);
    }
}

// ---------------------------------------------------------------------------
// k_gemv_r1: the normed q|k|v projection with the RoPE and KV-store epilogue
// (prologue 3, epilogue 5 of k_gemv_v5) as one block per compute unit.  With
// 8-row blocks the 2560 rows of TinyLlama's q|k|v make 320 blocks on 256
// compute units: 64 of them share a unit with another block, start their
// norm statistics behind its loads and finish 1-2 us after the rest.  Here
// each wave streams one whole row (lane l holds elements 2 l + 128 t and
// 2 l + 128 t + 1 of tile t), RW = M / (compute units) waves per block, RW / 2
// RoPE pairs (rows i and i + hd / 2 of a head) per block.  Every block stages
// the whole normed x (all waves read all of it); the arithmetic is k_gemv_v5's
// (same limbs, same carry-free sums, same correction, same epilogue), so the
// bits are the same.  K = 128 NT, int64 weights; UNR tiles of the row in
// flight (8 for TinyLlama: the prologue and the block-wide staging take about
// 3 us, a window of 4 drained before them).  ROPE false: the plain q|k|v
// projection (epilogue 0, attention above 512 positions rotates itself),
// row RW b + w in wave w of block b.  WT 1: bfloat16-resident weights, 512
// per 1 KB tile (8 per lane), by k_gemv_v5's fast form with its wave check
// and exact recomputation.
// ---------------------------------------------------------------------------
template <int RW, int NT, int UNR, bool ROPE = true, int WT = 0>
__global__ __launch_bounds__(64 * RW) void k_gemv_r1(int64_t *__restrict__ y,
                                                     const void *__restrict__ Wv,
                                                     const int64_t *__restrict__ x,
                                                     const int64_t *__restrict__ norm_w,
                                                     const int64_t *__restrict__ r_in, int M,
                                                     const q48_ropekv rk)
{
    static_assert(RW % 2 == 0 && NT % UNR == 0, "row pairs, whole windows");
    constexpr int TE = WFmt<WT>::TE * 8;                // elements per 1 KB tile
    constexpr int K = TE * NT;
    constexpr int NP = K / 2;                           // element pairs of x
    constexpr int XB = (NP + 64 * RW - 1) / (64 * RW);  // x pairs per thread
    constexpr int PC = (K / 8 + 63) / 64;               // partial sums per lane (wave 0)
    extern __shared__ __align__(16) uint32_t xs[];      // 3 limbs per element, all of K
    __shared__ uint64_t xsum_w[RW];
    __shared__ int64_t vrow[RW];
    __shared__ int64_t r_sh;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the row of this wave: pair p of the projection (hd / 2 pairs per head),
    // its first row (even waves) or its partner hd / 2 rows on (odd waves)
    const int half = ROPE ? rk.hd >> 1 : 1, sh = 31 - __builtin_clz((unsigned)half);
    const int p = (RW / 2) * (int)blockIdx.x + (wave >> 1);
    const int hh = p >> sh, j = p & (half - 1);
    const int row = ROPE ? hh * rk.hd + j + ((wave & 1) ? half : 0) : RW * (int)blockIdx.x + wave;
    const bool live = row < M;
    // the position, read first through the constant address space (a scalar
    // load: no vector-memory wait covers it)
    typedef const __attribute__((address_space(4))) int cint;
    const int p5 = !ROPE ? 0 : rk.d_pos ? *(cint *)rk.d_pos : rk.pos;

    // issue order: wave 0's partial sums, then every thread's x and norm
    // weight pairs, then the wave's first UNR weight tiles
    const uint64_t *st = reinterpret_cast<const uint64_t *>(r_in);
    uint64_t plo[PC], phi[PC];
    if (wave == 0) {
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            const int i = min(lane + c * 64, K / 8 - 1);
            const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(st + 2 * i);
            plo[c] = v.x;
            phi[c] = v.y;
        }
    }
    int64_t xv[2 * XB], nw[2 * XB];
#pragma unroll
    for (int b = 0; b < XB; ++b) {
        const int pi = min(tid + 64 * RW * b, NP - 1);
        const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(x + 2 * pi);
        const ulonglong2 w = *reinterpret_cast<const ulonglong2 *>(norm_w + 2 * pi);
        xv[2 * b] = (int64_t)v.x;
        xv[2 * b + 1] = (int64_t)v.y;
        nw[2 * b] = (int64_t)w.x;
        nw[2 * b + 1] = (int64_t)w.y;
    }
    // every wave's x loads ahead of any wave's weight loads in the compute
    // unit's load path (measured: 5-10 us per token with the 8-tile window)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const ulonglong2 *w2 = reinterpret_cast<const ulonglong2 *>(
                               static_cast<const char *>(Wv) +
                               (size_t)(live ? row : 0) * K * WFmt<WT>::ES) + lane;
    ulonglong2 wa[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u)
        wa[u] = ld_wtile<WT>(&w2[64 * u]);
    __builtin_amdgcn_sched_barrier(0);
    // the wave's cos / sin pair at the position (scalar loads)
    typedef const __attribute__((address_space(4))) int64_t cint64;
    int64_t c5 = 0, s5 = 0;
    if constexpr (ROPE) {
        const int pc = min(max(p5, 0), rk.max_seq - 1);
        c5 = *(cint64 *)(rk.cos_t + (size_t)pc * half + j);
        s5 = *(cint64 *)(rk.sin_t + (size_t)pc * half + j);
    }

    // r from the producer's partial sums, on wave 0 alone (as k_gemv_v5)
    if (wave == 0) {
        q48_u128 ss = 0;
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            const uint64_t m = lane + c * 64 < K / 8 ? ~0ull : 0ull;
            ss += ((q48_u128)(phi[c] & m) << 64) | (plo[c] & m);
        }
        ss = q48_wave_sum128(ss);
        const int64_t rv = rms_inv_of(ss, K);
        if (lane == 0)
            r_sh = rv;
    }
    __syncthreads();
    const int64_t r = r_sh;

    // stage fp_mul(fp_mul(x, r), w) as limbs (offset binary, as k_gemv_v5)
    uint64_t xsum = 0;
#pragma unroll
    for (int b = 0; b < XB; ++b) {
        const int pi = tid + 64 * RW * b;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            int64_t v = q48_mul(q48_mul(xv[2 * b + e], r), nw[2 * b + e]);
            v = pi < NP ? v : 0;
            xsum += (uint64_t)v;
            if (pi < NP) {
                const int k = 2 * pi + e;
                const uint64_t X = (uint64_t)v ^ 0x8000000000000000ull;
                xs[3 * k] = (uint32_t)X & 0x3FFFFFu;
                xs[3 * k + 1] = (uint32_t)(X >> 22) & 0x1FFFFFu;
                // bfloat16 weights: the signed top limb (b16_tile_fast)
                xs[3 * k + 2] = WT == 1 ? (uint32_t)(v >> 43) : (uint32_t)(X >> 43);
            }
        }
    }
    xsum = (uint64_t)q48_wave_sum64((int64_t)xsum);
    if (lane == 0)
        xsum_w[wave] = xsum;
    __syncthreads();
    uint64_t xtot = 0;
#pragma unroll
    for (int w = 0; w < RW; ++w)
        xtot += xsum_w[w];

    // the row: a rotating window of UNR tiles in flight; lane l's elements
    // of tile t start at TE t + (TE / 64) l
    Acc6 A = {0, 0, 0, 0, 0, 0, 0};
    Acc3 F = {0, 0, 0, 0, 0, 0};
    q48_u16x2 chk = {0, 0};
    const uint32_t *xl = xs + 3 * (TE / 64) * lane;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t *q = xl + 3 * TE * t;
        const ulonglong2 w = wa[t % UNR];
        if constexpr (WT == 0) {
            mac6(A, q[0], q[1], q[2], w.x);
            mac6(A, q[3], q[4], q[5], w.y);
        } else {
            b16_tile_fast(F, chk, q, 0, 0, w);
        }
        if (t + UNR < NT)
            wa[t % UNR] = ld_wtile<WT>(&w2[64 * (t + UNR)]);
    }
    // bfloat16: the fast sums plus, when a pattern outside the fast window
    // is anywhere in the wave's row (rare), their residuals
    q48_u128 Sl;
    if constexpr (WT == 1) {
        b16_pin(F);
        Sl = acc3_value(F);
        if (!b16_wave_ok(chk)) {
            // the window holds the whole row when UNR == NT: no second read
            if constexpr (NT == UNR)
                b16_fix_regs(Sl, wa, [&](int t) { return xl + 3 * TE * t; });
            else
                b16_fix_tiles(
                    Sl, NT, [&](int t) { return w2[64 * t]; },
                    [&](int t) { return xl + 3 * TE * t; });
        }
    } else {
        Sl = acc6_value(A);
    }
    q48_u128 S = q48_wave_sum128(Sl);
    if constexpr (WT == 0)
        S -= (q48_u128)xtot << 63;
    const int64_t v = (int64_t)((q48_i128)S >> 48);
    if constexpr (!ROPE) {
        if (lane == 0 && live)
            y[row] = v;
        return;
    }
    if (lane == 0)
        vrow[wave] = v;
    __syncthreads();

    // RoPE of the q and k rows (rope_apply, llama_int.c:997-1008), then k
    // and v to the caches at pos (llama_int.c:1414-1416): lane 0 of each wave
    if (lane != 0 || !live)
        return;
    const int64_t o = vrow[wave ^ 1];
    int64_t r5 = v;
    if (hh < rk.n_heads + rk.n_kv)
        r5 = (wave & 1) == 0 ? (int64_t)((uint64_t)q48_mul(v, c5) - (uint64_t)q48_mul(o, s5))
                             : (int64_t)((uint64_t)q48_mul(v, c5) + (uint64_t)q48_mul(o, s5));
    y[row] = r5;
    if (hh >= rk.n_heads && p5 >= 0 && p5 < rk.max_seq) {
        const bool isk = hh < rk.n_heads + rk.n_kv;
        const int kh = hh - rk.n_heads - (isk ? 0 : rk.n_kv);
        int64_t *cache = isk ? rk.kc : rk.vc;
        const int d = j + ((wave & 1) ? half : 0);
        cache[((size_t)rk.layer * rk.max_seq + p5) * ((size_t)rk.n_kv * rk.hd) +
              (size_t)kh * rk.hd + d] = r5;
    }
}

// ---------------------------------------------------------------------------
// k_gemv_p6: the persistent form of k_gemv_v5 for the long projections whose
// blocks would otherwise repeat a costly prologue in lockstep rounds (the
// normed gate|up with SwiGLU, the normed lm_head).  Block b takes the row
// groups b, b + G, b + 2G, ... (G = gridDim.x):
//  - the norm statistics, r and the staged x limbs are computed once per
//    block, not once per 8 rows;
//  - the next group's first UNR weight tiles are issued during the current
//    group's last ones, so the weight stream does not stop between groups;
//  - EPI 2 keeps each group's gate/up pre-activations in LDS and applies
//    SwiGLU to all of them after the last group (one latency chain per
//    block instead of one per group).
// Every wave has exactly NTF tiles (K = 16 NTF NW, checked on the host).
// Results are those of k_gemv_v5 (same sums, same epilogue arithmetic).
// ---------------------------------------------------------------------------
constexpr int P6_MAXG = 16;   // row groups per block at most

template <int NW, int UNR, int PRO, int EPI, int NTF, int WT = 0>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4))) void
k_gemv_p6(int64_t *__restrict__ y, const void *__restrict__ Wv,
          const int64_t *__restrict__ x, const int64_t *__restrict__ norm_w,
          const int64_t *__restrict__ r_in, int M, int K, int seg)
{
    static_assert(NTF > 0 && (PRO == 0 || PRO == 3) && (EPI == 0 || EPI == 2), "p6 forms");
    // the window crosses into the next group in the slots it frees: tile t of
    // the next group must land in slot t % UNR
    static_assert(NTF % UNR == 0, "p6 window must divide the tiles");
    constexpr int ES = WFmt<WT>::ES, SEGC = WFmt<WT>::TE * NTF;
    extern __shared__ __align__(16) uint32_t xs[];   // 3 limbs per staged x
    __shared__ uint64_t part[2][NW][V4_RB][2];
    __shared__ int64_t pre[P6_MAXG][V4_RB];          // EPI 2: gate (0-3) / up (4-7)
    __shared__ int64_t r_sh;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 3, l8 = lane & 7;
    const int ffn = M >> 1;
    const int k0 = wave * seg;
    const int ngroups = EPI == 2 ? (ffn + 3) / 4 : (M + V4_RB - 1) / V4_RB;

    // this lane's weight row in group grp (EPI 2: gate rows 4 grp + g, then
    // up rows ffn + 4 grp + g - 4); rows past the end read row 0 (in bounds,
    // never stored)
    auto wrow = [&](int grp) {
        const int pr = grp * 4 + (g & 3);
        const int row = EPI == 2 ? (g < 4 ? pr : ffn + pr) : grp * V4_RB + g;
        const bool live = EPI == 2 ? pr < ffn : row < M;
        return reinterpret_cast<const ulonglong2 *>(static_cast<const char *>(Wv) +
                                                    ((size_t)(live ? row : 0) * K + k0) * ES) +
               l8;
    };

    // PRO 3 partial sums first, then x (and the norm weights), then the
    // first group's weight tiles: vmcnt retires in issue order
    constexpr int PC = (NW * SEGC / 8 + 63) / 64;
    uint64_t plo[PC], phi[PC];
    const int np = (K + 7) >> 3;
    const uint64_t *st = reinterpret_cast<const uint64_t *>(r_in);
    if (PRO == 3 && wave == 0) {
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            const int i = min(lane + c * 64, np - 1);
            const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(st + 2 * i);
            plo[c] = v.x;
            phi[c] = v.y;
        }
    }
    constexpr int XB = (SEGC + 127) / 128;
    int64_t xv[2 * XB], nw[2 * XB];
#pragma unroll
    for (int b = 0; b < XB; ++b) {
        const int j = min(2 * lane + 128 * b, seg - 2);
        const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(x + k0 + j);
        xv[2 * b] = (int64_t)v.x;
        xv[2 * b + 1] = (int64_t)v.y;
        if (PRO != 0) {
            const ulonglong2 w = *reinterpret_cast<const ulonglong2 *>(norm_w + k0 + j);
            nw[2 * b] = (int64_t)w.x;
            nw[2 * b + 1] = (int64_t)w.y;
        }
    }
    asm volatile("" ::: "memory");   // keep the x loads ahead of the weight loads
    int grp = blockIdx.x;
    const ulonglong2 *w2 = wrow(grp < ngroups ? grp : 0);
    ulonglong2 wa[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u)
        wa[u] = ld_wtile<WT>(&w2[u * 8]);
    __builtin_amdgcn_sched_barrier(0);

    int64_t r = 0;
    if (PRO == 3) {
        // wave 0 alone loads the partials and derives r (as in k_gemv_v5)
        if (wave == 0) {
            q48_u128 ss = 0;
#pragma unroll
            for (int c = 0; c < PC; ++c) {
                const uint64_t m = lane + c * 64 < np ? ~0ull : 0ull;
                ss += ((q48_u128)(phi[c] & m) << 64) | (plo[c] & m);
            }
            ss = q48_wave_sum128(ss);
            const int64_t rv = rms_inv_of(ss, K);
            if (lane == 0)
                r_sh = rv;
        }
        __syncthreads();
        r = r_sh;
    }

    // stage this wave's segment of x as limbs; sum x over the segment
    uint64_t xsum = 0;
    uint32_t *xw = xs + (size_t)wave * seg * 3;
#pragma unroll
    for (int b = 0; b < 2 * XB; ++b) {
        const int j = 2 * lane + 128 * (b / 2) + b % 2;
        int64_t v = xv[b];
        if (PRO != 0)
            v = q48_mul(q48_mul(v, r), nw[b]);
        v = j < seg ? v : 0;
        xsum += (uint64_t)v;
        if (j < seg) {
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

    int i = 0;
    for (; grp < ngroups; grp += gridDim.x, ++i) {
        const int nxt = grp + (int)gridDim.x;
        // the next group's rows; after the last group, group 0's (read by
        // every block there, so they stay in cache: in bounds, never used)
        const ulonglong2 *w2n = wrow(nxt < ngroups ? nxt : 0);
        Acc6 A = {0, 0, 0, 0, 0, 0, 0};
        Acc3 F = {0, 0, 0, 0, 0, 0};
        q48_u16x2 chk = {0, 0};
        // bfloat16: this group's tiles, kept after the window moves on to
        // the next group's (for the residual pass, without a second read)
        ulonglong2 wc[WT == 1 ? NTF : 1];
#pragma unroll
        for (int t = 0; t < NTF; ++t) {
            if constexpr (WT == 0) {
                mac_tile<0>(A, xw, l8, t, wa[t % UNR]);
            } else {
                b16_tile_fast(F, chk, xw, l8, t, wa[t % UNR]);
                wc[t] = wa[t % UNR];
            }
            if (t + UNR < NTF)
                wa[t % UNR] = ld_wtile<WT>(&w2[(t + UNR) * 8]);
            else
                wa[t % UNR] = ld_wtile<WT>(&w2n[(t + UNR - NTF) * 8]);
        }
        // bfloat16 outside the fast window: the residuals of this group's
        // tiles (the next group's tiles stay in the window)
        q48_u128 S;
        if constexpr (WT == 1) {
            b16_pin(F);
            S = acc3_value(F);
            if (!b16_wave_ok(chk))
                b16_fix_regs(S, wc, [&](int t) { return xw + 3 * (64 * t + 8 * l8); });
        } else {
            S = acc6_value(A);
        }
        w2 = w2n;
        S = q48_sum8_u128(S);
        if (l8 == 0) {
            if constexpr (WT == 0)
                S -= (q48_u128)xsum << 63;
            part[i & 1][wave][g][0] = (uint64_t)S;
            part[i & 1][wave][g][1] = (uint64_t)(S >> 64);
        }
        // partial sums double-buffered by group: one barrier per group
        __syncthreads();
        if (tid < V4_RB) {
            q48_u128 T = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w)
                T += ((q48_u128)part[i & 1][w][tid][1] << 64) | part[i & 1][w][tid][0];
            const int64_t v = (int64_t)((q48_i128)T >> 48);
            if (EPI == 0) {
                const int rr = grp * V4_RB + tid;
                if (rr < M)
                    y[rr] = v;
            } else {
                pre[i][tid] = v;
            }
        }
    }
    if (EPI == 2) {
        __syncthreads();
        // SwiGLU of every pair this block produced, one pair per thread
        if (tid < 4 * i) {
            const int gi = tid >> 2, q = tid & 3;
            const int pi = ((int)blockIdx.x + gi * (int)gridDim.x) * 4 + q;
            if (pi < ffn)
                y[pi] = q48_mul(q48_silu(pre[gi][q]), pre[gi][4 + q]);
        }
    }
}

// Standalone rmsnorm statistics r of x (one block): for the fallbacks and
// for the first hidden vector of a token.  With table != nullptr it also
// copies table[*d_token or token] to out first (the embedding row,
// llama_int.c:2822-2824) and takes the statistics of that row.
__global__ __launch_bounds__(256) void k_rms_inv(int64_t *__restrict__ r_out,
                                                int64_t *__restrict__ out,
                                                const int64_t *__restrict__ x,
                                                const int64_t *__restrict__ table,
                                                const int *__restrict__ d_token, int token,
                                                int dim)
{
    __shared__ uint64_t red_lo[4], red_hi[4];
    const int tid = threadIdx.x;
    if (table) {
        if (d_token)
            token = *d_token;
        x = table + (size_t)token * dim;
    }
    q48_u128 ss = 0;
    constexpr int B = 8;
    for (int i0 = 0; i0 < dim; i0 += 256 * B) {
        int64_t v[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int i = i0 + tid + 256 * b;
            v[b] = i < dim ? x[i] : 0;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int i = i0 + tid + 256 * b;
            if (table && i < dim)
                out[i] = v[b];
            ss += (q48_u128)q48_smul128(v[b], v[b]);
        }
    }
    ss = q48_wave_sum128(ss);
    if ((tid & 63) == 0) {
        red_lo[tid >> 6] = (uint64_t)ss;
        red_hi[tid >> 6] = (uint64_t)(ss >> 64);
    }
    __syncthreads();
    if (tid == 0) {
        q48_u128 t = 0;
        for (int w = 0; w < 4; ++w)
            t += ((q48_u128)red_hi[w] << 64) | red_lo[w];
        *r_out = rms_inv_of(t, dim);
    }
}

// Partial sums of squares of x over rows 8i..8i+7 (stats[2i], stats[2i+1]
// = lo, hi), the input of a PRO 3 consumer; with table != nullptr x is the
// embedding row table[*d_token or token], copied to out first
// (llama_int.c:2822-2824).
__global__ __launch_bounds__(256) void k_rms_stats(int64_t *__restrict__ stats,
                                                  int64_t *__restrict__ out,
                                                  const int64_t *__restrict__ x,
                                                  const int64_t *__restrict__ table,
                                                  const int *__restrict__ d_token, int token,
                                                  int dim)
{
    if (table) {
        if (d_token)
            token = *d_token;
        x = table + (size_t)token * dim;
    }
    const int np = (dim + 7) >> 3;
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < np; p += gridDim.x * blockDim.x) {
        int64_t v[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const int i = 8 * p + b;
            v[b] = i < dim ? x[i] : 0;
        }
        q48_u128 ss = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const int i = 8 * p + b;
            if (table && i < dim)
                out[i] = v[b];
            ss += (q48_u128)q48_smul128(v[b], v[b]);
        }
        reinterpret_cast<uint64_t *>(stats)[2 * p] = (uint64_t)ss;
        reinterpret_cast<uint64_t *>(stats)[2 * p + 1] = (uint64_t)(ss >> 64);
    }
}

// r of the rmsnorm of a dim-vector from its partial sums (one block).
__global__ __launch_bounds__(256) void k_stats_r(int64_t *__restrict__ r_out,
                                                const int64_t *__restrict__ stats, int dim)
{
    __shared__ uint64_t red_lo[4], red_hi[4];
    const int np = (dim + 7) >> 3;
    const uint64_t *st = reinterpret_cast<const uint64_t *>(stats);
    q48_u128 ss = 0;
    for (int p = threadIdx.x; p < np; p += 256)
        ss += ((q48_u128)st[2 * p + 1] << 64) | st[2 * p];
    ss = block_sum128<256>(ss, red_lo, red_hi);
    if (threadIdx.x == 0)
        *r_out = rms_inv_of(ss, dim);
}

// out = fp_mul(fp_mul(x, *r), w): the per-element part of rmsnorm.
__global__ __launch_bounds__(256) void k_rms_apply(int64_t *__restrict__ out,
                                                  const int64_t *__restrict__ x,
                                                  const int64_t *__restrict__ w,
                                                  const int64_t *__restrict__ r, int dim)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < dim)
        out[i] = q48_mul(q48_mul(x[i], *r), w[i]);
}

// Grid of the persistent form: at most two blocks per compute unit, and no
// more blocks than make every block take the same number of row groups
// (rounds) up to one: 1408 groups run as 470 blocks x 3, not 512 blocks of
// which a quarter idle through the last round.
static int p6_grid(const q48_ctx *c, int groups)
{
    const int full = 2 * c->cu_count;
    const int rounds = (groups + full - 1) / full;
    return (groups + rounds - 1) / rounds;
}

template <int PRO, int EPI>
static int launch_v4(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                     const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M, int K,
                     const q48_ropekv *rk = nullptr)
{
    const q48_ropekv rkv = rk ? *rk : q48_ropekv{};
    constexpr int NW = 8;
    // segment: K / NW rounded up to a multiple of 16 elements
    const int seg = ((K + NW - 1) / NW + 15) / 16 * 16;
    const size_t lds = (size_t)seg * NW * 3 * sizeof(uint32_t);
    const int blocks = EPI == 2 ? (M / 2 + 3) / 4 : (M + V4_RB - 1) / V4_RB;
    if (EPI == 3) {
        int rc = q48_rms_reserve(c, blocks);
        if (rc)
            return rc;
    }
    // K = 2048 and K = 5632 (every wave: 16 or 44 whole tiles) take the
    // unrolled rotating pipeline; other K the batched loop
    const bool al = ((uintptr_t)x & 15) == 0 && (PRO == 0 || ((uintptr_t)norm_w & 15) == 0) &&
                    (PRO != 3 || ((uintptr_t)r_in & 15) == 0);
    // more row groups than two rounds of blocks: the persistent form
    if constexpr ((PRO == 0 || PRO == 3) && (EPI == 0 || EPI == 2)) {
        const int grid = 2 * c->cu_count;
        if (al && K == NW * seg && seg == 16 * 16 && blocks > 2 * grid &&
            blocks <= P6_MAXG * grid && c->gemv_persistent) {
            hipLaunchKernelGGL((k_gemv_p6<NW, 4, PRO, EPI, 16>), dim3(p6_grid(c, blocks)),
                               dim3(64 * NW), lds,
                               c->stream, y, W, x, norm_w, r_in, M, K, seg);
            return (int)hipGetLastError();
        }
    }
    // the normed q|k|v projection (with or without RoPE) at 10 rows per
    // compute unit (TinyLlama on 256 units): one block per unit, one row per
    // wave
    if constexpr (PRO == 3 && (EPI == 5 || EPI == 0)) {
        if (al && K == 2048 && c->cu_count > 0 && M == 10 * c->cu_count) {
            hipLaunchKernelGGL((k_gemv_r1<10, 16, 8, EPI == 5, 0>), dim3(c->cu_count),
                               dim3(64 * 10), (size_t)3 * K * sizeof(uint32_t), c->stream, y,
                               (const void *)W, x, norm_w, r_in, M, rkv);
            return (int)hipGetLastError();
        }
    }
    if (al && K == NW * seg && seg == 16 * 16)
        hipLaunchKernelGGL((k_gemv_v5<NW, 4, PRO, EPI, 16>), dim3(blocks), dim3(64 * NW), lds,
                           c->stream, y, W, x, norm_w, r_in, r_out, c->rms_part, c->rms_count,
                           M, K, seg, rkv);
    else if (al && K == NW * seg && seg == 16 * 44)
        hipLaunchKernelGGL((k_gemv_v5<NW, 6, PRO, EPI, 44>), dim3(blocks), dim3(64 * NW), lds,
                           c->stream, y, W, x, norm_w, r_in, r_out, c->rms_part, c->rms_count,
                           M, K, seg, rkv);
    else
        hipLaunchKernelGGL((k_gemv_v5<NW, 16, PRO, EPI, 0>), dim3(blocks), dim3(64 * NW), lds,
                           c->stream, y, W, x, norm_w, r_in, r_out, c->rms_part, c->rms_count,
                           M, K, seg, rkv);
    return (int)hipGetLastError();
}

// The bfloat16-weight forms (WT 1): every wave takes K / 512 whole tiles of 64
// weights (K a multiple of 512), x and norm_w 16-byte aligned; other shapes
// are refused (Q48_EINVAL from the caller).  Long normed projections take the
// persistent form like the int64 weights.
template <int PRO, int EPI, int NTF>
static int launch_b16_ntf(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                          const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M,
                          int K, const q48_ropekv *rk = nullptr)
{
    const q48_ropekv rkv = rk ? *rk : q48_ropekv{};
    // the window: every tile of the segment in flight when it divides no
    // other way (11 tiles for K = 5632), else 4
    constexpr int NW = 8, UNR = NTF < 4 ? NTF : NTF % 4 == 0 ? 4 : NTF;
    const int seg = K / NW;
    const size_t lds = (size_t)seg * NW * 3 * sizeof(uint32_t);
    const int blocks = EPI == 2 ? (M / 2 + 3) / 4 : (M + V4_RB - 1) / V4_RB;
    if constexpr ((PRO == 0 || PRO == 3) && (EPI == 0 || EPI == 2) && UNR <= 4 && NTF % UNR == 0) {
        const int grid = 2 * c->cu_count;
        if (blocks > 2 * grid && blocks <= P6_MAXG * grid && c->gemv_persistent) {
            hipLaunchKernelGGL((k_gemv_p6<NW, UNR, PRO, EPI, NTF, 1>), dim3(p6_grid(c, blocks)),
                               dim3(64 * NW), lds, c->stream, y, W, x, norm_w, r_in, M, K, seg);
            return (int)hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_gemv_v5<NW, UNR, PRO, EPI, NTF, 1>), dim3(blocks), dim3(64 * NW), lds,
                       c->stream, y, W, x, norm_w, r_in, r_out, c->rms_part, c->rms_count, M,
                       K, seg, rkv);
    return (int)hipGetLastError();
}

template <int PRO, int EPI>
static int launch_b16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                      const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M, int K,
                      const q48_ropekv *rk = nullptr)
{
    const q48_ropekv rkv = rk ? *rk : q48_ropekv{};
    // the normed q|k|v projection at 10 rows per compute unit: one block per
    // unit, one row per wave (as for int64 weights)
    if constexpr (PRO == 3 && (EPI == 5 || EPI == 0)) {
        const bool al = ((uintptr_t)x & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 &&
                        ((uintptr_t)r_in & 15) == 0 && ((uintptr_t)W & 15) == 0;
        if (al && K == 2048 && c->cu_count > 0 && M == 10 * c->cu_count) {
            hipLaunchKernelGGL((k_gemv_r1<10, 4, 4, EPI == 5, 1>), dim3(c->cu_count),
                               dim3(64 * 10), (size_t)3 * K * sizeof(uint32_t), c->stream, y,
                               (const void *)W, x, norm_w, r_in, M, rkv);
            return (int)hipGetLastError();
        }
    }
    switch (K) {
    case 512:
        return launch_b16_ntf<PRO, EPI, 1>(c, y, W, x, norm_w, r_in, r_out, M, K, rk);
    case 1024:
        return launch_b16_ntf<PRO, EPI, 2>(c, y, W, x, norm_w, r_in, r_out, M, K, rk);
    case 2048:
        return launch_b16_ntf<PRO, EPI, 4>(c, y, W, x, norm_w, r_in, r_out, M, K, rk);
    case 5632:
        // all 11 tiles in flight: registers allow it without the norm prologue
        if constexpr (PRO == 0)
            return launch_b16_ntf<PRO, EPI, 11>(c, y, W, x, norm_w, r_in, r_out, M, K, rk);
        [[fallthrough]];
    default: {
        // other K (a multiple of 512): batches of 4 tiles in a loop (an
        // unrolled chain of more tiles runs out of registers)
        constexpr int NW = 8;
        const int seg = K / NW;
        const size_t lds = (size_t)seg * NW * 3 * sizeof(uint32_t);
        const int blocks = EPI == 2 ? (M / 2 + 3) / 4 : (M + V4_RB - 1) / V4_RB;
        hipLaunchKernelGGL((k_gemv_v5<NW, 4, PRO, EPI, 0, 1>), dim3(blocks), dim3(64 * NW), lds,
                           c->stream, y, W, x, norm_w, r_in, r_out, c->rms_part, c->rms_count,
                           M, K, seg, rkv);
        return (int)hipGetLastError();
    }
    }
}

// Per-row sums mod 2^64 (one wave per row): the 2^63 correction terms of
// the flipped-limb GEMM.
__global__ __launch_bounds__(256) void k_rowsum(uint64_t *__restrict__ out,
                                               const int64_t *__restrict__ A,
                                               int rows, int K)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const int64_t *r = A + (size_t)row * K;
    uint64_t s = 0;
    for (int j = lane; j < K; j += 64)
        s += (uint64_t)r[j];
    s = (uint64_t)q48_wave_sum64((int64_t)s);
    if (lane == 0)
        out[row] = s;
}

// GEMM Y[T][N] = X[T][K] . W[N][K]^T >> 48, per element exactly the GEMV.
// Block 256 threads = 16 x 16, tile 64 tokens x 64 rows, 4x4 outputs per
// thread, K staged 16 at a time in LDS in flipped form (zero padding
// flips to 2^63 and contributes 2^126 per product: bits >= 126 only).
constexpr int GT = 64, GN = 64, GK = 16;

__global__ __launch_bounds__(256) void k_gemm(int64_t *__restrict__ Y,
                                             const int64_t *__restrict__ W,
                                             const int64_t *__restrict__ X,
                                             const uint64_t *__restrict__ wsum,
                                             const uint64_t *__restrict__ xsum,
                                             int T, int N, int K)
{
    __shared__ __align__(16) uint64_t Xs[GK][GT];
    __shared__ __align__(16) uint64_t Ws[GK][GN];

    const int tid = threadIdx.x;
    const int tx = tid & 15;       // row group
    const int ty = tid >> 4;       // token group
    const int t0 = blockIdx.y * GT;
    const int n0 = blockIdx.x * GN;

    uint64_t a0[4][4], a1[4][4], a2[4][4];
    uint32_t c0[4][4], c1[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a0[i][j] = a1[i][j] = a2[i][j] = 0;
            c0[i][j] = c1[i][j] = 0;
        }

    for (int k0 = 0; k0 < K; k0 += GK) {
        __syncthreads();
        // stage 64 x 16 of X and of W: 1024 elements each, 4 per thread
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int idx = tid + 256 * e;
            int r = idx >> 4, k = idx & 15;
            int kk = k0 + k;
            uint64_t xv = 0, wv = 0;
            if (t0 + r < T && kk < K)
                xv = (uint64_t)X[(size_t)(t0 + r) * K + kk];
            if (n0 + r < N && kk < K)
                wv = (uint64_t)W[(size_t)(n0 + r) * K + kk];
            Xs[k][r] = xv ^ 0x8000000000000000ull;
            Ws[k][r] = wv ^ 0x8000000000000000ull;
        }
        __syncthreads();
#pragma unroll 4
        for (int k = 0; k < GK; ++k) {
            uint32_t xl[4], xh[4], wl[4], wh[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint64_t xv = Xs[k][ty * 4 + i];
                uint64_t wv = Ws[k][tx * 4 + i];
                xl[i] = (uint32_t)xv;
                xh[i] = (uint32_t)(xv >> 32);
                wl[i] = (uint32_t)wv;
                wh[i] = (uint32_t)(wv >> 32);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint64_t s;
                    s = (uint64_t)xl[i] * wl[j] + a0[i][j];
                    c0[i][j] += s < a0[i][j];
                    a0[i][j] = s;
                    s = (uint64_t)xh[i] * wl[j] + a1[i][j];
                    c1[i][j] += s < a1[i][j];
                    a1[i][j] = s;
                    s = (uint64_t)xl[i] * wh[j] + a1[i][j];
                    c1[i][j] += s < a1[i][j];
                    a1[i][j] = s;
                    a2[i][j] += (uint64_t)xh[i] * wh[j];
                }
        }
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int t = t0 + ty * 4 + i;
        if (t >= T)
            continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int n = n0 + tx * 4 + j;
            if (n >= N)
                continue;
            q48_u128 S = (q48_u128)a0[i][j];
            S += (q48_u128)c0[i][j] << 64;
            S += (q48_u128)a1[i][j] << 32;
            S += (q48_u128)c1[i][j] << 96;
            S += (q48_u128)a2[i][j] << 64;
            S -= (q48_u128)(xsum[t] + wsum[n]) << 63;
            Y[(size_t)t * N + n] = (int64_t)((q48_i128)S >> 48);
        }
    }
}

} // namespace

// Largest K the v2 kernel stages in LDS (64 KiB of x).
// K the v4 kernel takes: staged limbs (12 B per x) stay under 144 KiB of LDS and a
// lane sums at most K / 64 <= 1023 partial products per accumulator.
constexpr int V2_MAX_K = 12288;

bool q48_gemv_v2_ok(const int64_t *W, int K)
{
    return K % 2 == 0 && K <= V2_MAX_K && (((uintptr_t)W & 15) == 0);
}

int q48_launch_gemv_fused(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                          const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M,
                          int K, int pro, int epi)
{
    if (pro == 1)
        return epi == 2 ? launch_v4<1, 2>(c, y, W, x, norm_w, nullptr, nullptr, M, K)
                        : launch_v4<1, 0>(c, y, W, x, norm_w, nullptr, nullptr, M, K);
    if (pro == 2)
        return epi == 2 ? launch_v4<2, 2>(c, y, W, x, norm_w, r_in, nullptr, M, K)
                        : launch_v4<2, 0>(c, y, W, x, norm_w, r_in, nullptr, M, K);
    if (pro == 3)
        return epi == 2 ? launch_v4<3, 2>(c, y, W, x, norm_w, r_in, nullptr, M, K)
                        : launch_v4<3, 0>(c, y, W, x, norm_w, r_in, nullptr, M, K);
    if (epi == 4)
        return launch_v4<0, 4>(c, y, W, x, nullptr, nullptr, r_out, M, K);
    if (epi == 3)
        return launch_v4<0, 3>(c, y, W, x, nullptr, nullptr, r_out, M, K);
    return epi == 1 ? launch_v4<0, 1>(c, y, W, x, nullptr, nullptr, nullptr, M, K)
                    : launch_v4<0, 0>(c, y, W, x, nullptr, nullptr, nullptr, M, K);
}

bool q48_gemv_bf16_ok(int K) { return K > 0 && K % 512 == 0 && K <= V2_MAX_K; }

int q48_launch_gemv_fused_bf16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                               const int64_t *norm_w, const int64_t *r_in, int64_t *r_out, int M,
                               int K, int pro, int epi)
{
    if (pro == 3)
        return epi == 2 ? launch_b16<3, 2>(c, y, W, x, norm_w, r_in, nullptr, M, K)
                        : launch_b16<3, 0>(c, y, W, x, norm_w, r_in, nullptr, M, K);
    if (epi == 4)
        return launch_b16<0, 4>(c, y, W, x, nullptr, nullptr, r_out, M, K);
    return launch_b16<0, 0>(c, y, W, x, nullptr, nullptr, nullptr, M, K);
}

int q48_launch_gemv_rope_kv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                            const int64_t *norm_w, const int64_t *stats,
                            const q48_ropekv *rk, int M, int K)
{
    return launch_v4<3, 5>(c, y, W, x, norm_w, stats, nullptr, M, K, rk);
}

int q48_launch_gemv_rope_kv_bf16(q48_ctx *c, int64_t *y, const uint16_t *W, const int64_t *x,
                                 const int64_t *norm_w, const int64_t *stats,
                                 const q48_ropekv *rk, int M, int K)
{
    return launch_b16<3, 5>(c, y, W, x, norm_w, stats, nullptr, M, K, rk);
}

// int64 -> bfloat16 bits where exact: b is the candidate with 8 significant
// bits (bfloat16_to_q1648's exponent rule inverted), then q48_bf16(b) == v
// is checked; any element that does not round-trip sets *inexact.
__global__ __launch_bounds__(256) void k_bf16_pack(uint16_t *__restrict__ out,
                                                  const int64_t *__restrict__ in, size_t n,
                                                  int *__restrict__ inexact)
{
    bool bad = false;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (size_t)gridDim.x * 256) {
        const int64_t v = in[i];
        uint32_t b = 0;
        if (v != 0) {
            const uint64_t mag = v < 0 ? 0ull - (uint64_t)v : (uint64_t)v;
            const int p = 63 - __builtin_clzll(mag);
            const int sh = p - 7;   // shift of the 8-bit significand
            const uint32_t sig = sh >= 0 ? (uint32_t)(mag >> sh) : (uint32_t)(mag << (-sh));
            const int e = sh + 86;
            b = (v < 0 ? 0x8000u : 0u) | ((uint32_t)(e & 0xff) << 7) | (sig & 0x7fu);
            if (e < 1 || e > 254)
                bad = true;
        }
        bad |= q48_bf16(b) != v;
        out[i] = (uint16_t)b;
    }
    if (bad)
        __hip_atomic_store(inexact, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int q48_launch_bf16_pack(q48_ctx *c, uint16_t *out, const int64_t *in, size_t n, int *inexact)
{
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_bf16_pack, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256),
                       0, c->stream, out, in, n, inexact);
    return (int)hipGetLastError();
}

int q48_launch_rms_inv(q48_ctx *c, int64_t *r_out, int64_t *out, const int64_t *x,
                       const int64_t *table, const int *d_token, int token, int dim)
{
    hipLaunchKernelGGL(k_rms_inv, dim3(1), dim3(256), 0, c->stream, r_out, out, x, table,
                       d_token, token, dim);
    return (int)hipGetLastError();
}

int q48_launch_rms_stats(q48_ctx *c, int64_t *stats, int64_t *out, const int64_t *x,
                         const int64_t *table, const int *d_token, int token, int dim)
{
    const int np = (dim + 7) / 8;
    hipLaunchKernelGGL(k_rms_stats, dim3((np + 255) / 256), dim3(256), 0, c->stream, stats, out,
                       x, table, d_token, token, dim);
    return (int)hipGetLastError();
}

int q48_launch_stats_r(q48_ctx *c, int64_t *r_out, const int64_t *stats, int dim)
{
    hipLaunchKernelGGL(k_stats_r, dim3(1), dim3(256), 0, c->stream, r_out, stats, dim);
    return (int)hipGetLastError();
}

int q48_launch_rms_apply(q48_ctx *c, int64_t *out, const int64_t *x, const int64_t *w,
                         const int64_t *r, int dim)
{
    hipLaunchKernelGGL(k_rms_apply, dim3((dim + 255) / 256), dim3(256), 0, c->stream, out, x, w,
                       r, dim);
    return (int)hipGetLastError();
}

int q48_launch_gemv(q48_ctx *c, int64_t *y, const int64_t *W, const int64_t *x,
                    int M, int K)
{
    if (q48_gemv_v2_ok(W, K))
        return launch_v4<0, 0>(c, y, W, x, nullptr, nullptr, nullptr, M, K);
    const bool vec = (K % 2 == 0) && (((uintptr_t)W & 15) == 0);
    if (M >= 1024) {
        dim3 grid((M + 7) / 8);
        if (vec)
            hipLaunchKernelGGL((k_gemv<8, 2>), grid, dim3(512), 0, c->stream, y, W, x, M, K);
        else
            hipLaunchKernelGGL((k_gemv<8, 1>), grid, dim3(512), 0, c->stream, y, W, x, M, K);
    } else {
        dim3 grid((M + 3) / 4);
        if (vec)
            hipLaunchKernelGGL((k_gemv<4, 2>), grid, dim3(256), 0, c->stream, y, W, x, M, K);
        else
            hipLaunchKernelGGL((k_gemv<4, 1>), grid, dim3(256), 0, c->stream, y, W, x, M, K);
    }
    return (int)hipGetLastError();
}

int q48_launch_gemm(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X,
                    int T, int N, int K)
{
    size_t need = ((size_t)T + (size_t)N) * sizeof(uint64_t);
    int rc = q48_ws_reserve(c, need);
    if (rc)
        return rc;
    uint64_t *wsum = (uint64_t *)c->ws;
    uint64_t *xsum = wsum + N;
    hipLaunchKernelGGL(k_rowsum, dim3((N + 3) / 4), dim3(256), 0, c->stream, wsum, W, N, K);
    hipLaunchKernelGGL(k_rowsum, dim3((T + 3) / 4), dim3(256), 0, c->stream, xsum, X, T, K);
    dim3 grid((N + GN - 1) / GN, (T + GT - 1) / GT);
    hipLaunchKernelGGL(k_gemm, grid, dim3(256), 0, c->stream, Y, W, X, wsum, xsum, T, N, K);
    return (int)hipGetLastError();
}
