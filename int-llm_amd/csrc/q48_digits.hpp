// q48_digits.hpp — int64 values as eight int8 digits for the int8 matrix
// cores, and the 24-bit limb products of truncated Q16.48 products.  Included
// by the HIP sources of libintllm_hip only.
//
// Digits.  Every int64 v is written v = S(v) + C with C = 0x0080808080808080
// and S(v) = sum_i s_i 256^i, s_i the bytes of v ^ C read as int8 (bytes 0..6
// are offset by 128, byte 7 is v's own signed top byte).  Then over any
// index range of length n
//   sum_k x_k w_k = sum_{a,b} 256^(a+b) P_ab + C sum_k x_k + C sum_k w_k - n C^2,
//   P_ab = sum_k s_a(x_k) s_b(w_k),
// exactly (mod 2^128).  Only bits [48,112) are ever observed, so the pair
// a = b = 7 (weight 2^112) is dropped and the other 63 products are grouped
// by d = a + b into 14 int32 accumulators.  An index whose digits are all
// zero (the value C) adds nothing to any P_ab.
#pragma once

#include "q48_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr uint64_t kDig = 0x0080808080808080ull;

// 4 x 4 byte transpose: out_j = [a_j, b_j, c_j, d_j] (v_perm_b32 selects
// bytes 0-3 from its second operand and 4-7 from its first).
__device__ __forceinline__ void tr4(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                    uint32_t (&o)[4])
{
    const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x06020400u);   // a0 b0 a2 b2
    const uint32_t t1 = __builtin_amdgcn_perm(b, a, 0x07030501u);   // a1 b1 a3 b3
    const uint32_t t2 = __builtin_amdgcn_perm(d, c, 0x06020400u);   // c0 d0 c2 d2
    const uint32_t t3 = __builtin_amdgcn_perm(d, c, 0x07030501u);   // c1 d1 c3 d3
    o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    o[2] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Digits of four values: w[a] holds digit a of v[0..3] in bytes 0..3.
__device__ __forceinline__ void digits4(const uint64_t (&v)[4], uint32_t (&w)[8])
{
    uint32_t lo[4], hi[4];
    tr4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3], lo);
    tr4((uint32_t)(v[0] >> 32), (uint32_t)(v[1] >> 32), (uint32_t)(v[2] >> 32),
        (uint32_t)(v[3] >> 32), hi);
#pragma unroll
    for (int a = 0; a < 4; ++a)
        w[a] = lo[a] ^ 0x80808080u;
#pragma unroll
    for (int a = 0; a < 3; ++a)
        w[4 + a] = hi[a] ^ 0x80808080u;
    w[7] = hi[3];
}

// sum_d 256^d q[d][i] (int128) of 14 digit-product accumulators
__device__ __forceinline__ q48_u128 digits_total(const v4i (&q)[14], int i)
{
    // four int64 partial sums of at most four terms each (|q| < 2^31)
    int64_t part[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        int64_t s = 0;
#pragma unroll
        for (int d = 4 * g + 3; d >= 4 * g; --d)
            if (d < 14)
                s = s * 256 + (int64_t)q[d][i];
        part[g] = s;
    }
    q48_u128 tot = (q48_u128)(q48_i128)part[3];
#pragma unroll
    for (int g = 2; g >= 0; --g)
        tot = (tot << 32) + (q48_u128)(q48_i128)part[g];
    return tot;
}

// sum over the lanes of a group of N = 2, 4, 8 or 16 (lane % N varies)
template <int N>
__device__ __forceinline__ uint64_t group_sum64(uint64_t v)
{
    v += q48_dpp64<Q48_DPP_XOR1>(v);
    if (N >= 4)
        v += q48_dpp64<Q48_DPP_XOR2>(v);
    if (N >= 8)
        v += q48_dpp64<Q48_DPP_HALF_MIRROR>(v);
    if (N >= 16)
        v += q48_dpp64<Q48_DPP_MIRROR>(v);
    return v;
}

// v ^ (the same value on lane l ^ m), 128 bits as four 32-bit shuffles
__device__ __forceinline__ q48_u128 shfl_xor128(q48_u128 v, int m)
{
    q48_u128 r = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        r |= (q48_u128)(uint32_t)__shfl_xor((int)(uint32_t)(v >> (32 * k)), m) << (32 * k);
    return r;
}

// sum_e v[e] over the four words of each of the 16 lanes of a row group
// (lane % 16 varies), on every lane: 64 int64 in exact 128-bit arithmetic,
// as the 64-bit sums of their signed high and unsigned low 32-bit halves
// (in-row DPP adds, no cross-lane round trip through LDS)
__device__ __forceinline__ q48_u128 row16_sum4(const uint64_t (&v)[4])
{
    uint64_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        lo += (uint32_t)v[e];
        hi += (uint64_t)((int64_t)v[e] >> 32);
    }
    lo = group_sum64<16>(lo);
    hi = group_sum64<16>(hi);
    return (q48_u128)((q48_i128)(int64_t)hi << 32) + lo;
}

// sum_d 256^d a[d] (int128) of 14 digit-product sums
__device__ __forceinline__ q48_u128 digits_total14(const int (&a)[14])
{
    int64_t part[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        int64_t s = 0;
#pragma unroll
        for (int d = 4 * g + 3; d >= 4 * g; --d)
            if (d < 14)
                s = s * 256 + (int64_t)a[d];
        part[g] = s;
    }
    q48_u128 tot = (q48_u128)(q48_i128)part[3];
#pragma unroll
    for (int g = 2; g >= 0; --g)
        tot = (tot << 32) + (q48_u128)(q48_i128)part[g];
    return tot;
}

// v_mad_u32_u24: a * b + c over the low 24 bits of a and b (full rate)
__device__ __forceinline__ uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c)
{
    uint32_t r;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Low limbs of a truncated product.  For a = p mod 2^48 = a0 + 2^24 a1 and
// b = v mod 2^48 = b0 + 2^24 b1 (24-bit limbs; a limb word may carry higher
// bits, the 24-bit multiplies ignore them), t = floor(((p v) mod 2^48) / 2^24)
//   = (a0 b1 + a1 b0 + floor(a0 b0 / 2^24)) mod 2^24;
// returns acc + t.  Then for any n terms (n < 2^24)
//   sum_j floor(p_j v_j / 2^48) = floor((sum_j p_j v_j - 2^24 sum_j t_j) / 2^48),
// since each (p_j v_j) mod 2^48 lies in [2^24 t_j, 2^24 t_j + 2^24).
__device__ __forceinline__ uint32_t trunc_low_acc(uint2 a, uint2 b, uint32_t acc)
{
    const uint64_t p00 = (uint64_t)(a.x & 0xFFFFFFu) * (b.x & 0xFFFFFFu);
    uint32_t t = __builtin_amdgcn_alignbit((uint32_t)(p00 >> 32), (uint32_t)p00, 24);
    t = mad_u24(a.x, b.y, t);
    t = mad_u24(a.y, b.x, t);
    return mad_u24(t, 1u, acc);
}

// the limb words (bits 0..31, bits 24..55) of v for trunc_low_acc
__device__ __forceinline__ uint2 low_limbs(uint64_t v)
{
    return make_uint2((uint32_t)v, __builtin_amdgcn_alignbit((uint32_t)(v >> 32), (uint32_t)v, 24));
}

} // namespace
