// q48_gemv_tiles.hpp — the tile arithmetic of the decode GEMVs (k_gemv_v5,
// k_gemv_p6): carry-free limb products of staged x against int64 or bfloat16
// weight tiles, the rmsnorm scalar r, and 128-bit block sums.  Included by the HIP sources of
// libintllm_hip only.
#pragma once

#include "q48_internal.h"

namespace {

constexpr int V4_RB = 8;

// (ss >> 48) / dim + eps, then fp_inv_sqrt: the scalar part of rmsnorm
// (llama_int.c:1049-1055).  A power-of-two dim divides by shifting
// (truncating, like the division, for a negative wrapped sum too).
__device__ __forceinline__ int64_t rms_inv_of(q48_u128 ss, int dim)
{
    const q48_i128 a = (q48_i128)ss >> 48;
    int64_t ms;
    if ((dim & (dim - 1)) == 0) {
        const int sh = __builtin_ctz((unsigned)dim);
        ms = (int64_t)(a >= 0 ? a >> sh : -((-a) >> sh));
    } else {
        ms = (int64_t)q48_divs_128_64(a, (int64_t)dim);
    }
    ms = (int64_t)((uint64_t)ms + 2814749767ull);
    return q48_inv_sqrt(ms);
}

// 128-bit sum over the block (NT threads); result valid in thread 0.
template <int NT>
__device__ __forceinline__ q48_u128 block_sum128(q48_u128 v, uint64_t *red_lo, uint64_t *red_hi)
{
    v = q48_wave_sum128(v);
    const int tid = threadIdx.x;
    if ((tid & 63) == 0) {
        red_lo[tid >> 6] = (uint64_t)v;
        red_hi[tid >> 6] = (uint64_t)(v >> 64);
    }
    __syncthreads();
    q48_u128 t = 0;
    if (tid == 0)
        for (int w = 0; w < NT / 64; ++w)
            t += ((q48_u128)red_hi[w] << 64) | red_lo[w];
    return t;
}

typedef unsigned short q48_u16x2 __attribute__((ext_vector_type(2)));

struct Acc6 {
    uint64_t a00, a01, a10, a11, a20, a21, ws;
};

__device__ __forceinline__ void mac6(Acc6 &A, uint32_t x0, uint32_t x1, uint32_t x2,
                                     uint64_t w)
{
    const uint32_t wl = (uint32_t)w, wh = (uint32_t)(w >> 32) ^ 0x80000000u;
    A.a00 += (uint64_t)x0 * wl;
    A.a01 += (uint64_t)x0 * wh;
    A.a10 += (uint64_t)x1 * wl;
    A.a11 += (uint64_t)x1 * wh;
    A.a20 += (uint64_t)x2 * wl;
    A.a21 += (uint64_t)x2 * wh;
    A.ws += w;
}

__device__ __forceinline__ q48_u128 acc6_value(const Acc6 &A)
{
    return (q48_u128)A.a00 + ((q48_u128)A.a01 << 32) + ((q48_u128)A.a10 << 22) +
           ((q48_u128)A.a11 << 54) + ((q48_u128)A.a20 << 43) + ((q48_u128)A.a21 << 75) -
           ((q48_u128)A.ws << 63);
}

// bfloat16_to_q1648 (safetensors.h:115-152), bit for bit: zero and subnormal
// exponents give 0, exponent 255 gives +-32000 << 48, otherwise (128 + m)
// shifted by e - 86 (left shifts wrap mod 2^64, right shifts truncate,
// shifts of 64 or more give 0), then the sign (two's complement negation).
// Branch-free (selects and masks only): it runs once per weight inside the
// unrolled GEMV loop.
__device__ __forceinline__ int64_t q48_bf16(uint32_t b)
{
    const int e = (int)((b >> 7) & 0xffu);
    const uint64_t sig = 128u + (b & 0x7fu);
    const int sh = e - 86;
    const uint64_t lft = sig << (sh & 63), rgt = sig >> ((-sh) & 63);
    const uint64_t left = 0ull - (uint64_t)(sh >= 0);
    // a shift of 64 or more either way, or a zero / subnormal exponent: 0
    const uint64_t ok = 0ull - (uint64_t)((unsigned)(sh + 63) < 127u && e != 0);
    uint64_t r = (rgt ^ ((lft ^ rgt) & left)) & ok;
    const uint64_t inf = 0ull - (uint64_t)(e == 0xff);
    r = (r & ~inf) | (((uint64_t)32000 << 48) & inf);
    const uint64_t neg = 0ull - (uint64_t)(b >> 15);
    return (int64_t)((r ^ neg) - neg);
}

// Weight formats of the decode GEMVs: WT 0 = int64 Q16.48 (a 128-byte tile of
// a row is 16 weights, 2 per lane); WT 1 = bfloat16 bits (a tile is 64
// weights, 8 per lane), expanded exactly with q48_bf16.  A wave's segment is
// TE[WT] * NTF elements.
template <int WT> struct WFmt;
template <> struct WFmt<0> { static constexpr int ES = 8, TE = 16; };
template <> struct WFmt<1> { static constexpr int ES = 2, TE = 64; };

// One 128-byte tile t of this lane's row of int64 weights against the staged
// x limbs (3 per element at xw[3 j]).
template <int WT>
__device__ __forceinline__ void mac_tile(Acc6 &A, const uint32_t *xw, int l8, int t, ulonglong2 w)
{
    static_assert(WT == 0, "the bfloat16 tiles use b16_tile_fast and b16_tile_fix");
    const uint32_t *p = xw + 6 * l8 + 48 * t;
    mac6(A, p[0], p[1], p[2], w.x);
    mac6(A, p[3], p[4], p[5], w.y);
}

// Fast form of the bfloat16 tiles.  A pattern with exponent e in [103, 126]
// has the Q16.48 value w = t 2^17 with t = s (128 + m) 2^(e - 103), an
// integer of at most 31 bits: t is the pattern read as an f32 with 31 added
// to its exponent, converted exactly by v_cvt_i32_f32.  Then
// w x = (t x0 + t x1 2^22 + t x2s 2^43) 2^17 with x split into the limbs x0
// (22 bits), x1 (21 bits) and the signed top limb x2s, three signed 32 x 32
// multiply-adds per weight into 64-bit sums (a lane sums at most K / 64
// <= 192 products below 2^53: no overflow).  Every other pattern (zero and
// subnormal, |w| < 2^-24, |w| >= 1, inf, NaN) is caught by a range check
// folded into a running packed 16-bit maximum: 2 b mod 2^16 drops the sign,
// and 2 b - (103 << 8) wraps to at least 24 << 8 outside the window.  A
// wave whose check fails adds the residuals of b16_tile_fix.
struct Acc3 {
    int64_t f0, f1, f2, g0, g1, g2;   // even / odd weights of a pair
};
constexpr uint32_t B16_EXP = 31u << 23;                 // 2^31 in the f32 exponent
constexpr unsigned short B16_DLO = (unsigned short)(0x10000 - (103 << 8));
constexpr unsigned B16_DMAX = (24u << 8) - 1;           // largest in-window value

// v_cvt_i32_f32 of the bits fb: the fast form's t.  Written out so that its
// value outside the window (saturated, or 0 for NaN, as the ISA defines it)
// is the same in the fast sums and in b16_tile_fix.
__device__ __forceinline__ int32_t b16_t(uint32_t fb)
{
    int32_t t;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(t) : "v"(fb));
    return t;
}

__device__ __forceinline__ void b16_tile_fast(Acc3 &F, q48_u16x2 &chk, const uint32_t *xw,
                                              int l8, int t, ulonglong2 w)
{
    __builtin_amdgcn_sched_barrier(0);
    // 8 elements x 3 limbs = 96 bytes at a 96-byte multiple of the 16-byte
    // aligned segment: six 16-byte reads
    const uint4 *p4 = reinterpret_cast<const uint4 *>(xw + 3 * (64 * t + 8 * l8));
    uint4 q4[6];
#pragma unroll
    for (int i = 0; i < 6; ++i)
        q4[i] = p4[i];
    const int32_t *q = reinterpret_cast<const int32_t *>(q4);
    const uint32_t u[4] = {(uint32_t)w.x, (uint32_t)(w.x >> 32), (uint32_t)w.y,
                           (uint32_t)(w.y >> 32)};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const q48_u16x2 d = __builtin_bit_cast(q48_u16x2, u[h]) * (q48_u16x2)(2) +
                            (q48_u16x2)(B16_DLO);
        chk = __builtin_elementwise_max(chk, d);
        const int32_t ta = b16_t((u[h] << 16) + B16_EXP);
        const int32_t tb = b16_t((u[h] & 0xffff0000u) + B16_EXP);
        F.f0 += (int64_t)ta * q[6 * h];
        F.f1 += (int64_t)ta * q[6 * h + 1];
        F.f2 += (int64_t)ta * q[6 * h + 2];
        F.g0 += (int64_t)tb * q[6 * h + 3];
        F.g1 += (int64_t)tb * q[6 * h + 4];
        F.g2 += (int64_t)tb * q[6 * h + 5];
    }
}

// The exact residual of one tile's patterns outside the fast window, added
// to S.  The fast sums hold t 2^17 x for every weight, t = b16_t of the
// shifted pattern, and stay exact outside the window too (|t| <= 2^31 keeps
// every product below 2^53); adding w x - t 2^17 x for exactly those
// weights, w = q48_bf16(b) and x rebuilt from its limbs, gives sum w x mod
// 2^128.  Per weight under a per-lane test: the wave runs a body only when
// one of its lanes holds such a pattern there.
__device__ __forceinline__ void b16_tile_fix(q48_u128 &S, const uint32_t *p, ulonglong2 w)
{
    const uint32_t u[4] = {(uint32_t)w.x, (uint32_t)(w.x >> 32), (uint32_t)w.y,
                           (uint32_t)(w.y >> 32)};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t b = (u[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        const uint32_t ex = (b >> 7) & 0xffu;
        if (ex < 103u || ex > 126u) {
            const uint32_t fb = (e & 1) ? (u[e >> 1] & 0xffff0000u) + B16_EXP
                                        : (u[e >> 1] << 16) + B16_EXP;
            const int64_t x = (int64_t)((uint64_t)p[3 * e] + ((uint64_t)p[3 * e + 1] << 22) +
                                        ((uint64_t)(int64_t)(int32_t)p[3 * e + 2] << 43));
            S += (q48_u128)q48_smul128(q48_bf16(b), x) -
                 ((q48_u128)q48_smul128(b16_t(fb), x) << 17);
        }
    }
}

// true on every lane when some lane of the wave holds a pattern of the tile
// w outside the fast window (the range check of b16_tile_fast)
__device__ __forceinline__ bool b16_tile_out(ulonglong2 w)
{
    const uint32_t u[4] = {(uint32_t)w.x, (uint32_t)(w.x >> 32), (uint32_t)w.y,
                           (uint32_t)(w.y >> 32)};
    q48_u16x2 m = (q48_u16x2)(0);
#pragma unroll
    for (int h = 0; h < 4; ++h)
        m = __builtin_elementwise_max(m, __builtin_bit_cast(q48_u16x2, u[h]) * (q48_u16x2)(2) +
                                             (q48_u16x2)(B16_DLO));
    const unsigned mx = m.x > m.y ? m.x : m.y;
    return __builtin_amdgcn_ballot_w64(mx > B16_DMAX) != 0;
}

// The residual pass of a wave whose range check failed: its nt tiles again,
// ld(t) the lane's 16 bytes of tile t and px(t) their staged limbs, read 8
// tiles at a time (one round of load latency per 8) and fixed only where a
// lane holds a pattern outside the window.
template <class Ld, class Px>
__device__ __forceinline__ void b16_fix_tiles(q48_u128 &S, int nt, Ld ld, Px px)
{
    constexpr int B = 8;
#pragma unroll 1
    for (int t0 = 0; t0 < nt; t0 += B) {
        ulonglong2 wb[B];
#pragma unroll
        for (int u = 0; u < B; ++u)
            wb[u] = ld(t0 + u < nt ? t0 + u : nt - 1);
#pragma unroll
        for (int u = 0; u < B; ++u)
            if (t0 + u < nt && b16_tile_out(wb[u]))
                b16_tile_fix(S, px(t0 + u), wb[u]);
    }
}

// The same residual pass over tiles still held in registers (w[0 .. N)):
// no second read of the weights, so a wave with a pattern outside the window
// costs its fix alone, not a memory round trip.
template <int N, class Px>
__device__ __forceinline__ void b16_fix_regs(q48_u128 &S, const ulonglong2 (&w)[N], Px px)
{
#pragma unroll
    for (int t = 0; t < N; ++t)
        if (b16_tile_out(w[t]))
            b16_tile_fix(S, px(t), w[t]);
}

// Pins the fast sums in registers before the wave's range check: otherwise
// the compiler sinks the fast multiply-adds below the check and keeps every
// tile's staged limbs live across it.
__device__ __forceinline__ void b16_pin(Acc3 &F)
{
    asm volatile("" : "+v"(F.f0), "+v"(F.f1), "+v"(F.f2), "+v"(F.g0), "+v"(F.g1), "+v"(F.g2));
}

// true on every lane when no lane of the wave saw a pattern outside the window
__device__ __forceinline__ bool b16_wave_ok(q48_u16x2 chk)
{
    const unsigned m = chk.x > chk.y ? chk.x : chk.y;
    return __builtin_amdgcn_ballot_w64(m > B16_DMAX) == 0;
}

__device__ __forceinline__ q48_u128 acc3_value(const Acc3 &F)
{
    const q48_i128 v = (q48_i128)F.f0 + (q48_i128)F.g0 + (((q48_i128)F.f1 + F.g1) << 22) +
                       (((q48_i128)F.f2 + F.g2) << 43);
    return (q48_u128)v << 17;
}

} // namespace
