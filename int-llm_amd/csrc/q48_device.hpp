// q48_device.hpp — Q16.48 integer math as gfx950 device functions.
//
// Bit-identical to the reference's fp_math.h (native __int128 backend,
// fp_math.h:184-290) and to llama_int.c's use of it.  Every function
// below cites the reference lines it reproduces.  All int64 adds wrap
// (two's complement), as the reference's -fwrapv build does.
//
// 128-bit values: signed 64 x 64 -> 128 products come from q48_smul_parts
// (four 32 x 32 -> 64 products; clang's own expansion of a sign-extended
// __int128 multiply issues nine quarter-rate multiplies); division goes
// through q48_udiv128_64 below (128 / 64 -> 128 quotient, exact, from FP64
// estimates).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __int128 q48_i128;
typedef unsigned __int128 q48_u128;

#define Q48_ONE ((int64_t)1 << 48)
#define Q48_HALF ((int64_t)1 << 47)

// The signed product a * b mod 2^128: hi = bits 64..127, mid = bits 32..63
// (the low 32 bits of the returned value), lo32 = bits 0..31.  Schoolbook
// over 32-bit halves of the unsigned words (no partial sum overflows 64
// bits), then the two's-complement correction of the high word: a negative
// operand contributes -2^64 times the other operand's unsigned word.
__device__ __forceinline__ void q48_smul_parts(int64_t a, int64_t b, uint64_t &hi, uint32_t &mid,
                                               uint32_t &lo32)
{
    const uint64_t ua = (uint64_t)a, ub = (uint64_t)b;
    const uint32_t al = (uint32_t)ua, ah = (uint32_t)(ua >> 32);
    const uint32_t bl = (uint32_t)ub, bh = (uint32_t)(ub >> 32);
    const uint64_t lo = (uint64_t)al * bl;
    const uint64_t t = (uint64_t)ah * bl + (lo >> 32);
    const uint64_t u = (uint64_t)al * bh + (uint32_t)t;
    hi = (uint64_t)ah * bh + (t >> 32) + (u >> 32);
    hi -= (a < 0 ? ub : 0) + (b < 0 ? ua : 0);
    mid = (uint32_t)u;
    lo32 = (uint32_t)lo;
}

// (q48_i128)a * b
__device__ __forceinline__ q48_i128 q48_smul128(int64_t a, int64_t b)
{
    uint64_t hi;
    uint32_t mid, lo32;
    q48_smul_parts(a, b, hi, mid, lo32);
    return (q48_i128)(((q48_u128)hi << 64) | ((uint64_t)mid << 32) | lo32);
}

// (int64_t)(((q48_i128)a * b) >> S) for 32 <= S < 64: bits S .. S + 63
template <int S>
__device__ __forceinline__ int64_t q48_mul_shr(int64_t a, int64_t b)
{
    static_assert(S >= 32 && S < 64, "shift");
    uint64_t hi;
    uint32_t mid, lo32;
    q48_smul_parts(a, b, hi, mid, lo32);
    return (int64_t)((hi << (64 - S)) | (uint64_t)(mid >> (S - 32)));
}

// Constants computed by fp_math_init (fp_math.h:833-858) on the device at
// context creation: FP_PI, fp_cordic_gain, fp_cordic_angles[48].
struct q48_consts {
    int64_t pi;
    int64_t gain;
    int64_t angles[48];
    int ready;
};

// ---------------------------------------------------------------------------
// Exact unsigned 128 / 64 division (quotient up to 128 bits).
//
// Two base-2^64 long-division digits, each an exact 128/64 step done by
// restoring division on 64-bit words (shift-subtract).  The safety net of
// q48_udiv128_64 below; never reached when the FP64 unit rounds correctly.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t q48_udiv128_step(uint64_t hi, uint64_t lo,
                                                     uint64_t d, uint64_t *rem)
{
    // Precondition hi < d: the quotient fits in 64 bits.
    uint64_t q = 0;
    if (hi == 0) {
        q = lo / d;
        *rem = lo - q * d;
        return q;
    }
    // restoring division: 64 iterations of (hi:lo) << 1, compare, subtract
    for (int i = 0; i < 64; ++i) {
        uint64_t top = hi >> 63;
        hi = (hi << 1) | (lo >> 63);
        lo <<= 1;
        q <<= 1;
        if (top || hi >= d) {
            hi -= d;
            q |= 1;
        }
    }
    *rem = hi;
    return q;
}

__device__ __forceinline__ q48_u128 q48_udiv128_64_slow(q48_u128 n, uint64_t d)
{
    uint64_t nh = (uint64_t)(n >> 64), nl = (uint64_t)n;
    uint64_t qh = nh / d;
    uint64_t r1 = nh - qh * d;
    uint64_t r;
    uint64_t ql = q48_udiv128_step(r1, nl, d, &r);
    return ((q48_u128)qh << 64) | ql;
}

// A non-negative double (at most 2^128) to an unsigned 128-bit integer,
// truncating.  Above 2^64 the value is a multiple of 2^12, so hi * 2^64 and
// the difference are exact in double.
__device__ __forceinline__ q48_u128 q48_f64_to_u128(double v)
{
    if (v < 18446744073709551616.0)
        return (uint64_t)v;
    const uint64_t hi = (uint64_t)(v * 5.421010862427522e-20);   // 2^-64
    const uint64_t lo = (uint64_t)(v - (double)hi * 18446744073709551616.0);
    return ((q48_u128)hi << 64) | lo;
}

// floor(n / d), exact, d > 0, for quotients of 2^52 and above.  Each pass
// takes an FP64 estimate of the remaining quotient, scaled by (1 - 2^-46)
// so that it stays at or below the true quotient (the estimate's relative
// error is below 2^-51), subtracts estimate * d exactly, and so removes at
// least 45 bits of the quotient: three passes cover any 128-bit quotient
// and leave at most one unit for the final step (checked on the host over
// 75 million random and edge cases).  Should an estimate ever overshoot,
// the long division above takes over, so the result is exact whatever the
// FP64 unit does.
__device__ __noinline__ q48_u128 q48_udiv128_64_big(q48_u128 n, uint64_t d)
{
    const q48_u128 n0 = n;
    const double dd = (double)d;
    q48_u128 q = 0;
#pragma unroll
    for (int it = 0; it < 3; ++it) {
        if (n < (q48_u128)d)
            break;
        const double nd =
            (double)(uint64_t)(n >> 64) * 18446744073709551616.0 + (double)(uint64_t)n;
        const q48_u128 qi = q48_f64_to_u128(nd / dd * (1.0 - 1.4210854715202004e-14));
        const q48_u128 p = qi * d;
        if (p > n)
            return q48_udiv128_64_slow(n0, d);
        n -= p;
        q += qi;
    }
#pragma unroll
    for (int it = 0; it < 2; ++it)
        if (n >= (q48_u128)d) {
            n -= d;
            ++q;
        }
    if (n >= (q48_u128)d)
        return q48_udiv128_64_slow(n0, d);
    return q;
}

// floor(n / d), exact.  Fast path when the quotient is below 2^52 (every
// division of the forward pass but rmsnorm's mean of large activations:
// fp_div(ONE, e^x), the softmax and the sigmoid all have quotients <=
// 2^48): one FP64 estimate, within a few units of the true quotient, fixed
// up by exact 128-bit remainder steps.  Otherwise the multi-pass version.
__device__ __forceinline__ q48_u128 q48_udiv128_64(q48_u128 n, uint64_t d)
{
    const q48_u128 hi52 = n >> 52;
    if ((uint64_t)(hi52 >> 64) == 0 && (uint64_t)hi52 < d) {
        const double nd = (double)(uint64_t)(n >> 64) * 18446744073709551616.0 +
                          (double)(uint64_t)n;
        uint64_t q = (uint64_t)(nd / (double)d);
        q48_i128 r = (q48_i128)(n - (q48_u128)q * d);
        while (r < 0) {
            --q;
            r += d;
        }
        while (r >= (q48_i128)d) {
            ++q;
            r -= d;
        }
        return q;
    }
    return q48_udiv128_64_big(n, d);
}

// fp_w_divs (fp_math.h:249-256) for a divisor that fits int64: truncating
// signed division; b == -1 wraps like negation.
__device__ __forceinline__ q48_i128 q48_divs_128_64(q48_i128 a, int64_t b)
{
    if (b == -1)
        return (q48_i128)(0 - (q48_u128)a);
    bool na = a < 0, nb = b < 0;
    q48_u128 ua = na ? (0 - (q48_u128)a) : (q48_u128)a;
    uint64_t ub = nb ? (uint64_t)0 - (uint64_t)b : (uint64_t)b;
    q48_u128 q = q48_udiv128_64(ua, ub);
    return (na != nb) ? (q48_i128)(0 - q) : (q48_i128)q;
}

// ---------------------------------------------------------------------------
// fp_math.h primitives
// ---------------------------------------------------------------------------

// fp_mul, fp_math.h:491-506
__device__ __forceinline__ int64_t q48_mul(int64_t a, int64_t b)
{
    return q48_mul_shr<48>(a, b);
}

// sum_t fp_mul(p_t, v_t) (mod 2^64) for 0 <= p_t < 2^63 (softmax weights),
// as two words: with p = ph 2^32 + pl and v = vh 2^32 + vl (vh signed),
//   p v = pl vl + (pl vh_u + ph vl) 2^32 + (ph vh - pl [vh < 0]) 2^64
// (vh_u: vh's bits unsigned), and with mid + cy 2^64 = pl vh_u + hi(pl vl)
// + ph vl, floor(p v / 2^48) = (mid >> 16) + (ph vh + cy 2^32 - pl [vh < 0])
// 2^16.  So a1 sums mid >> 16, a2 the second factor, and the sum is a1 +
// (a2 << 16): three 32 x 32 products per term instead of a signed
// 64 x 64 -> 128 product.
struct q48_pv_acc {
    uint64_t a1, a2;
};

__device__ __forceinline__ void q48_pv_mac(q48_pv_acc &acc, int64_t p, int64_t v)
{
    const uint32_t pl = (uint32_t)(uint64_t)p, ph = (uint32_t)((uint64_t)p >> 32);
    const uint32_t vl = (uint32_t)(uint64_t)v, vh = (uint32_t)((uint64_t)v >> 32);
    const uint64_t b = (uint64_t)pl * vh + __umulhi(pl, vl);   // < 2^64
    uint64_t mid;
    const bool cy = __builtin_add_overflow(b, (uint64_t)ph * vl, &mid);
    acc.a1 += mid >> 16;
    acc.a2 += (uint64_t)((int64_t)(int32_t)ph * (int64_t)(int32_t)vh) + ((uint64_t)cy << 32) -
              ((int32_t)vh < 0 ? (uint64_t)pl : 0);
}

__device__ __forceinline__ int64_t q48_pv_total(const q48_pv_acc &acc)
{
    return (int64_t)(acc.a1 + (acc.a2 << 16));
}

// fp_mul(r, r): r * r = u^2 with u = |r| <= 2^63 as an unsigned word;
// u^2 = hh 2^64 + 2 lh 2^32 + ll, and w = 2 lh + (ll >> 32) stays below 2^64,
// so bits 48..111 are (hh << 16) + (w >> 16) mod 2^64: three 32 x 32 -> 64
// products.
__device__ __forceinline__ int64_t q48_usqr(uint64_t u)
{
    const uint32_t l = (uint32_t)u, h = (uint32_t)(u >> 32);
    const uint64_t ll = (uint64_t)l * l, lh = (uint64_t)l * h, hh = (uint64_t)h * h;
    const uint64_t w = (lh << 1) + (ll >> 32);
    return (int64_t)((hh << 16) + (w >> 16));
}
__device__ __forceinline__ int64_t q48_sqr(int64_t r)
{
    return q48_usqr(r < 0 ? (uint64_t)0 - (uint64_t)r : (uint64_t)r);
}

// floor(mag * 2^48 / ub) for 0 < ub and mag < 16 ub (a quotient below
// 2^52).  mag / ub from the hardware reciprocal refined by one Newton step
// (relative error near 2^-52, so the estimate is within 2 units of the
// quotient), then exact 128-bit remainder steps; should the estimate ever be
// further off, the long division takes over, so the result is exact
// whatever the FP64 unit does.  About a third of the latency of the
// correctly rounded FP64 division plus unit remainder loops.
__device__ __forceinline__ uint64_t q48_udiv_shl48(uint64_t mag, uint64_t ub)
{
    const double bd = (double)ub;
    double r = __builtin_amdgcn_rcp(bd);
    r = __builtin_fma(r, __builtin_fma(-bd, r, 1.0), r);
    const double est = (double)mag * r * 281474976710656.0;   // 2^48
    int64_t q = (int64_t)est;                                 // below 2^53
    const q48_u128 num = (q48_u128)mag << 48;
    q48_i128 rem = (q48_i128)(num - (q48_u128)(uint64_t)q * ub);
    if (rem < 0) {
        --q;
        rem += ub;
        if (rem < 0) {
            --q;
            rem += ub;
        }
    } else if (rem >= (q48_i128)ub) {
        ++q;
        rem -= ub;
        if (rem >= (q48_i128)ub) {
            ++q;
            rem -= ub;
        }
    }
    if (rem < 0 || rem >= (q48_i128)ub)
        return (uint64_t)q48_udiv128_64_slow(num, ub);
    return (uint64_t)q;
}

// fp_div, fp_math.h:508-524
__device__ __forceinline__ int64_t q48_div(int64_t a, int64_t b)
{
    uint64_t mag = a < 0 ? (uint64_t)0 - (uint64_t)a : (uint64_t)a;
    const uint64_t ub = b < 0 ? (uint64_t)0 - (uint64_t)b : (uint64_t)b;
    if (b != -1 && ub != 0 && (mag >> 4) < ub) {
        // |num / b| = floor(mag 2^48 / |b|) < 2^52; the sign of a / b
        const uint64_t q = q48_udiv_shl48(mag, ub);
        return (a < 0) != (b < 0) ? (int64_t)((uint64_t)0 - q) : (int64_t)q;
    }
    q48_i128 num = (q48_i128)((q48_u128)mag << 48);
    if (a < 0)
        num = (q48_i128)(0 - (q48_u128)num);
    return (int64_t)q48_divs_128_64(num, b);
}

// The nearest integer to 0 <= v < 2^51, minus 1, from the FP64 word of v + 2^52
// (whose low 52 bits are that integer); as a word, -1 for v below 1/2.
__device__ __forceinline__ uint64_t q48_round_m1(double v)
{
    return (uint64_t)__builtin_bit_cast(int64_t, v + 0x1p52) - 0x4330000000000001ull;
}

// floor(2^96 / r) = fp_div(ONE, r) for 2^48 <= r < 2^63: the reciprocal in
// fp_exp of a negative argument and in fp_sigmoid (fp_math.h:516-523 with a
// = ONE).  y = 1 / r from the hardware reciprocal and two Newton steps has a
// relative error of a few units of 2^-53 (from any first approximation
// within 2^-20), so qe = y 2^96 is within 1/16 of 2^96 / r <= 2^48 and q0 =
// round(qe) - 1 is the quotient or one less.  The remainder 2^96 - q0 r then
// lies in [0, 2 r), below 2^64, so its low word 0 - q0 r (mod 2^64) is the
// remainder itself and one compare finishes the quotient.  A remainder that
// does not settle (an FP64 unit outside those bounds) goes to q48_div.
__device__ __forceinline__ int64_t q48_recip(int64_t r)
{
    const uint64_t u = (uint64_t)r;
    const double rd = (double)u;
    double y = __builtin_amdgcn_rcp(rd);
    y = __builtin_fma(y, __builtin_fma(-rd, y, 1.0), y);
    y = __builtin_fma(y, __builtin_fma(-rd, y, 1.0), y);
    const uint64_t q0 = q48_round_m1(y * 0x1p96);
    const uint64_t rem = (uint64_t)0 - q0 * u;
    const bool up = rem >= u;
    if (rem - (up ? u : 0) >= u)
        return q48_div(Q48_ONE, r);
    return (int64_t)(q0 + up);
}

// A divisor prepared for many fp_div(e, d) with the same d (a softmax row's
// sum, a renormalisation): 2^48 / d in FP64 (two Newton steps, as in
// q48_recip) when 1 <= d < 2^62, and the largest e the fast quotient takes,
// min(d, 2^52 - 1) (0 for any other d).
struct q48_divisor {
    uint64_t d, lim;
    double y48;
};
__device__ __forceinline__ q48_divisor q48_divisor_of(int64_t d)
{
    q48_divisor v = {(uint64_t)d, 0, 0.0};
    if (d >= 1 && d < ((int64_t)1 << 62)) {
        const double dd = (double)d;
        double y = __builtin_amdgcn_rcp(dd);
        y = __builtin_fma(y, __builtin_fma(-dd, y, 1.0), y);
        y = __builtin_fma(y, __builtin_fma(-dd, y, 1.0), y);
        v.y48 = y * 0x1p48;
        v.lim = d < ((int64_t)1 << 52) ? (uint64_t)d : ((uint64_t)1 << 52) - 1;
    }
    return v;
}

// fp_div(e, d) (fp_math.h:508-524) for a divisor from q48_divisor_of.  For 0 <=
// e <= lim the quotient e 2^48 / d is at most 2^48, e is exact in FP64, qe =
// e y48 is within 0.1 of the quotient, q0 = round(qe) - 1 is it or one less,
// and the remainder e 2^48 - q0 d, in [0, 2 d), is its own low word, as in
// q48_recip.  (With lim = 0, e = 0 gives q0 = -1, remainder d and quotient 0,
// which is fp_div(0, d) for every d != 0.)  Any other e goes to q48_div.
__device__ __forceinline__ int64_t q48_div_by(int64_t e, const q48_divisor &v)
{
    if ((uint64_t)e > v.lim)
        return q48_div(e, (int64_t)v.d);
    const double ed = __builtin_bit_cast(double, (uint64_t)e | 0x4330000000000000ull) - 0x1p52;
    const uint64_t q0 = q48_round_m1(ed * v.y48);
    const uint64_t rem = ((uint64_t)e << 48) - q0 * v.d;
    const bool up = rem >= v.d;
    if (rem - (up ? v.d : 0) >= v.d)
        return q48_div(e, (int64_t)v.d);
    return (int64_t)(q0 + up);
}

// fp_from_int, fp_math.h:530-538
__device__ __forceinline__ int64_t q48_from_int(int x)
{
    uint64_t mag = x < 0 ? (uint64_t)0 - (uint64_t)(int64_t)x : (uint64_t)x;
    q48_u128 r = (q48_u128)mag << 48;
    if (x < 0)
        r = 0 - r;
    return (int64_t)r;
}

__device__ __forceinline__ int64_t q48_abs(int64_t a) { return a >= 0 ? a : (int64_t)(0 - (uint64_t)a); }

// fp_sqrt_fast, fp_math.h:605-622
__device__ __forceinline__ int64_t q48_sqrt_fast(int64_t x)
{
    if (x <= 0)
        return 0;
    uint64_t ux = (uint64_t)x;
    int bw = 64 - __builtin_clzll(ux);
    uint64_t r = (uint64_t)1 << ((bw + 1) / 2);
    for (int i = 0; i < 5; ++i) {
        uint64_t nr = (r + ux / r) >> 1;
        if (nr >= r)
            break;
        r = nr;
    }
    return (int64_t)(r << 24);
}

// fp_sqrt, fp_math.h:626-652
__device__ __forceinline__ int64_t q48_sqrt(int64_t x)
{
    if (x <= 0)
        return 0;
    q48_u128 n = (q48_u128)(uint64_t)x << 48;
    uint64_t hi = (uint64_t)(n >> 64), lo = (uint64_t)n;
    int bw = hi ? 128 - __builtin_clzll(hi) : (lo ? 64 - __builtin_clzll(lo) : 0);
    uint64_t r = (uint64_t)1 << ((bw + 1) / 2);
    for (int i = 0; i < 7; ++i) {
        if (r == 0)
            return 0;
        uint64_t q = (uint64_t)q48_udiv128_64(n, r);
        uint64_t nr = (r + q) >> 1;
        if (nr >= r)
            break;
        r = nr;
    }
    while ((q48_i128)(int64_t)r * (int64_t)r > (q48_i128)n)
        r--;
    return (int64_t)r;
}

// fp_inv_sqrt, fp_math.h:658-707
__device__ __forceinline__ int64_t q48_inv_sqrt(int64_t x)
{
    if (x <= 0)
        return 0;
    int msb = 63 - __builtin_clzll((uint64_t)x);
    int k = (msb - 48) >> 1;
    int64_t xn = k >= 0 ? (x >> (2 * k)) : (int64_t)((uint64_t)x << (-2 * k));
    int msb_n = 63 - __builtin_clzll((uint64_t)xn);
    int64_t y = msb_n == 48 ? Q48_ONE : Q48_HALF;
    const int64_t three = (int64_t)3 << 48;
    // The first step in closed form: from ONE (xn in [2^48, 2^49)) the
    // square is ONE and xn * ONE >> 48 is xn, so yn = (3 ONE - xn) >> 1; from
    // HALF (xn in [2^49, 2^50)) the square is ONE / 4, so yn = (3 ONE -
    // (xn >> 2)) >> 2.  Both factors are positive and yn > 0.
    const int64_t y1 = msb_n == 48 ? (three - xn) >> 1 : (three - (xn >> 2)) >> 2;
    int i = 8;   // index of the next step (8: the first step was a fixed point)
    if (y1 != y) {
        y = y1;
        i = 1;
    }
    // Steps 1..7 on exact doubles, straight-line.  y, y2 = floor(y^2 /
    // 2^48), xy2 = floor(xn y2 / 2^48), the factor and the next y are
    // integers below 2^53 while y < 2^49 (xn < 2^50), and each truncated
    // product a b / 2^s (|a b| <= 2^(s + 52)) is exact:
    //   with bs = b 2^-s (exact), P = a bs = RN(a b) 2^-s has ulp(P) <= 1,
    //   so a b 2^-s lies in [f - 1, f + 1) for f = floor(P), and
    //   fma(a, bs, -f) = (a b - f 2^s) 2^-s exactly (a multiple of 2^-s in
    //   [-1, 1)): floor(a b / 2^s) = f + floor(fma(a, bs, -f)).
    // No compare or branch: the chain stays on the vector unit.  A fixed
    // point stays fixed, and so does 1 (the reference's value once a step
    // gives y <= 0), so running every remaining step gives the reference's
    // y.  Should y ever reach 2^49 the integer steps below run instead.
    if (i < 8) {
        const double xs = (double)xn * 0x1p-48;                 // exact
        const double tq = 844424930131968.0 * 0x1p-49;          // 3 * 2^48 * 2^-49
        double yd = (double)y, mx = yd;
#pragma unroll
        for (int j = 0; j < 7; ++j) {
            const double ys = yd * 0x1p-48;
            double P = yd * ys, f = __builtin_floor(P);
            const double y2 = f + __builtin_floor(__fma_rn(yd, ys, -f));
            P = y2 * xs;
            f = __builtin_floor(P);
            const double xy2 = f + __builtin_floor(__fma_rn(y2, xs, -f));
            const double fs = __fma_rn(xy2, -0x1p-49, tq);     // (3 * 2^48 - xy2) 2^-49
            P = yd * fs;
            f = __builtin_floor(P);
            yd = __builtin_fmax(f + __builtin_floor(__fma_rn(yd, fs, -f)), 1.0);
            mx = __builtin_fmax(mx, yd);
        }
        if (mx < 562949953421312.0) {   // 2^49
            y = (int64_t)yd;
            i = 8;
        }
    }
    for (; i < 8; ++i) {
        int64_t y2 = q48_sqr(y);
        int64_t xy2 = q48_mul_shr<48>(xn, y2);
        int64_t factor = three - xy2;
        const int64_t yn = q48_mul_shr<49>(y, factor);
        if (yn <= 0) {
            y = 1;
            break;
        }
        // a fixed point: every remaining step maps y to itself (usually
        // reached after 4-6 of the 8 steps)
        if (yn == y)
            break;
        y = yn;
    }
    if (k >= 0) {
        int64_t r = y >> k;
        return r < 0 ? 0 : r;
    }
    q48_i128 r = (q48_i128)((q48_u128)(q48_i128)y << (-k));
    if (r > (q48_i128)INT64_MAX)
        return INT64_MAX;
    if (r < 0)
        return 0;
    return (int64_t)r;
}

// fp_exp_dyadic, fp_math.h:714-720
__device__ __forceinline__ int64_t q48_exp_dyadic(int64_t x, int k)
{
    int64_t r = (int64_t)((uint64_t)Q48_ONE + (uint64_t)(x >> k));
#pragma unroll
    for (int i = 0; i < k; ++i)
        r = q48_sqr(r);
    return r;
}

// fp_exp, fp_math.h:724-732, as one path for every lane: the squarings of
// |x| (the reference's -x, wrapping), then the reciprocal unless x > 0.  At
// x = 0 the reference squares 0 and gets ONE; here ONE / ONE, also ONE.  With
// the reference's two branches a wave whose lanes hold both signs (a softmax
// row around its maximum, SiLU arguments) would run the 14 squarings twice.
__device__ __forceinline__ int64_t q48_exp(int64_t x)
{
    const uint64_t m = x >= 0 ? (uint64_t)x : (uint64_t)0 - (uint64_t)x;
    const int64_t r = q48_exp_dyadic((int64_t)m, 14);
    if (x > 0)
        return r;
    if (r == 0)
        return 0;
    return q48_div(Q48_ONE, r);
}

// fp_exp for |x| <= 10 ONE, the range fp_safe_exp leaves (fp_math.h:739-744):
// the same squarings, the first 12 on exact doubles.  r0 = ONE + (|x| >> 14)
// and r_k = floor(r_{k-1}^2 / 2^48) <= e^(10 2^(k - 14)) ONE, so r_0 .. r_11
// stay below 3.5 ONE < 2^50, each of their squares is below 2^100 and r_12 is
// below 12.2 ONE < 2^52: with rs = r 2^-48 (exact), f = floor(r rs) and
// fma(r, rs, -f) = (r^2 - f 2^48) 2^-48 exactly (a multiple of 2^-48 in [-1,
// 1)), floor(r^2 / 2^48) = f + floor(fma(r, rs, -f)), an integer double.
// Full-rate FP64 instead of three quarter-rate 32 x 32 -> 64 products per
// square; the last two squares (up to e^10 ONE < 2^63) stay integer, and the
// reciprocal of a negative argument is q48_recip (r >= ONE).
__device__ __forceinline__ int64_t q48_exp_small(int64_t x)
{
    const uint64_t m = x >= 0 ? (uint64_t)x : (uint64_t)0 - (uint64_t)x;
    double rd = (double)(int64_t)((uint64_t)Q48_ONE + (m >> 14));
#pragma unroll
    for (int k = 0; k < 12; ++k) {
        const double rs = rd * 0x1p-48;
        const double f = __builtin_floor(rd * rs);
        rd = f + __builtin_floor(__fma_rn(rd, rs, -f));
    }
    // rd is an integer below 2^52: the low bits of rd + 2^52's word
    uint64_t u = (uint64_t)__builtin_bit_cast(int64_t, rd + 0x1p52) - 0x4330000000000000ull;
    u = (uint64_t)q48_usqr(u);
    u = (uint64_t)q48_usqr(u);
    if (x > 0)
        return (int64_t)u;
    return q48_recip((int64_t)u);
}

// fp_safe_exp, fp_math.h:739-744
__device__ __forceinline__ int64_t q48_safe_exp(int64_t x)
{
    const int64_t max_x = (int64_t)10 << 48;
    if (x > max_x)
        x = max_x;
    if (x < -max_x)
        return 0;
    return q48_exp_small(x);
}

// fp_log, fp_math.h:752-773
__device__ __forceinline__ int64_t q48_log(int64_t x)
{
    if (x <= 0)
        return -((int64_t)50 << 48);
    const int64_t ln2 = 195103586505167LL;
    int lz = __builtin_clzll((uint64_t)x);
    int log2_approx = 63 - lz - 48;
    int64_t y = (int64_t)((uint64_t)(int64_t)log2_approx * (uint64_t)ln2);
    for (int i = 0; i < 10; ++i) {
        int64_t ey = q48_exp(y);
        if (ey == 0)
            break;
        int64_t y_new = (int64_t)((uint64_t)y - (uint64_t)Q48_ONE + (uint64_t)q48_div(x, ey));
        int64_t diff = q48_abs((int64_t)((uint64_t)y_new - (uint64_t)y));
        if (diff < 2)
            break;
        y = y_new;
    }
    return y;
}

// fp_atan_taylor, fp_math.h:789-800
__device__ __forceinline__ int64_t q48_atan_taylor(int64_t x, int max_terms)
{
    int64_t x_sq = q48_mul(x, x);
    int64_t term = x, sum = x;
    for (int n = 1; n <= max_terms; ++n) {
        term = (int64_t)(0 - (uint64_t)q48_mul(term, x_sq));
        int64_t c = term / (2 * n + 1);
        if (c == 0)
            break;
        sum = (int64_t)((uint64_t)sum + (uint64_t)c);
    }
    return sum;
}

// fp_compute_pi (fp_math.h:804-812), fp_atan_pow2 (:823-827),
// fp_math_init (:833-858).  Run by one thread at context creation.
__device__ inline void q48_math_init(q48_consts *k)
{
    int64_t atan5 = q48_atan_taylor(Q48_ONE / 5, 40);
    int64_t atan239 = q48_atan_taylor(Q48_ONE / 239, 15);
    k->pi = (int64_t)(((uint64_t)atan5 << 4) - ((uint64_t)atan239 << 2));
    k->angles[0] = k->pi >> 2;
    for (int i = 1; i < 48; ++i)
        k->angles[i] = i >= 25 ? (Q48_ONE >> i) : q48_atan_taylor(Q48_ONE >> i, 40);
    int64_t k_sq = Q48_ONE;
    for (int i = 0; i < 48; ++i) {
        int64_t sv = (2 * i < 63) ? (Q48_ONE >> (2 * i)) : 0;
        k_sq = q48_mul(k_sq, Q48_ONE + sv);
    }
    k->gain = q48_div(Q48_ONE, q48_sqrt(k_sq));
    k->ready = 1;
}

// fp_sincos, fp_math.h:861-902
__device__ __forceinline__ void q48_sincos(const q48_consts *__restrict__ k,
                                           int64_t angle, int64_t *c, int64_t *s)
{
    const int64_t pi = k->pi;
    const int64_t two_pi = (int64_t)((uint64_t)pi << 1);
    while (angle > pi)
        angle = (int64_t)((uint64_t)angle - (uint64_t)two_pi);
    while (angle < -pi)
        angle = (int64_t)((uint64_t)angle + (uint64_t)two_pi);
    const int64_t pi_half = pi >> 1;
    bool neg_cos = false;
    if (angle > pi_half) {
        angle = pi - angle;
        neg_cos = true;
    } else if (angle < -pi_half) {
        angle = -pi - angle;
        neg_cos = true;
    }
    int64_t x = k->gain, y = 0, z = angle;
    for (int i = 0; i < 48; ++i) {
        int64_t xs = x >> i, ys = y >> i;
        int64_t a = k->angles[i];
        if (z >= 0) {
            int64_t xn = (int64_t)((uint64_t)x - (uint64_t)ys);
            int64_t yn = (int64_t)((uint64_t)y + (uint64_t)xs);
            z = (int64_t)((uint64_t)z - (uint64_t)a);
            x = xn;
            y = yn;
        } else {
            int64_t xn = (int64_t)((uint64_t)x + (uint64_t)ys);
            int64_t yn = (int64_t)((uint64_t)y - (uint64_t)xs);
            z = (int64_t)((uint64_t)z + (uint64_t)a);
            x = xn;
            y = yn;
        }
    }
    *c = neg_cos ? (int64_t)(0 - (uint64_t)x) : x;
    *s = y;
}

// fp_sigmoid, fp_math.h:911-916
__device__ __forceinline__ int64_t q48_sigmoid(int64_t x)
{
    const int64_t ten = (int64_t)10 << 48;
    if (x > ten)
        return Q48_ONE;
    if (x < -ten)
        return 0;
    // ONE + e^-x lies in [ONE, (1 + e^10) ONE], within q48_recip's range
    int64_t en = q48_safe_exp((int64_t)(0 - (uint64_t)x));
    return q48_recip((int64_t)((uint64_t)Q48_ONE + (uint64_t)en));
}

// fp_silu, fp_math.h:919-921
__device__ __forceinline__ int64_t q48_silu(int64_t x)
{
    return q48_mul(x, q48_sigmoid(x));
}

// ---------------------------------------------------------------------------
// Wave-level reductions (wave64)
// ---------------------------------------------------------------------------

// Lane moves within a row of 16 lanes by DPP (no LDS round trip, unlike a
// shuffle): every lane reads the lane given by the control word.
constexpr int Q48_DPP_XOR1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int Q48_DPP_XOR2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int Q48_DPP_HALF_MIRROR = 0x141;  // lane i <- 7 - i within 8 lanes
constexpr int Q48_DPP_MIRROR = 0x140;       // lane i <- 15 - i within 16 lanes

template <int CTRL>
__device__ __forceinline__ uint64_t q48_dpp64(uint64_t v)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf,
                                                              0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32),
                                                              CTRL, 0xf, 0xf, false);
    return ((uint64_t)hi << 32) | lo;
}

template <int CTRL>
__device__ __forceinline__ q48_u128 q48_dpp128(q48_u128 v)
{
    return ((q48_u128)q48_dpp64<CTRL>((uint64_t)(v >> 64)) << 64) |
           q48_dpp64<CTRL>((uint64_t)v);
}

// 128-bit sum over each aligned group of 8 lanes; every lane of the group
// returns the group's total (all 8 lanes must be active).  After the two
// quad exchanges each lane holds its quad's sum; the half-row mirror pairs
// every lane with a lane of the other quad.
__device__ __forceinline__ q48_u128 q48_sum8_u128(q48_u128 v)
{
    v += q48_dpp128<Q48_DPP_XOR1>(v);
    v += q48_dpp128<Q48_DPP_XOR2>(v);
    v += q48_dpp128<Q48_DPP_HALF_MIRROR>(v);
    return v;
}

// 128-bit two's-complement sum across the 64 lanes of a wave (all active);
// every lane returns the total.  Integer addition mod 2^128 is associative,
// so any order gives the bits of the reference's serial loop.  Rows of 16
// lanes are summed by DPP, then the four row sums are read as scalars.
__device__ __forceinline__ q48_u128 q48_wave_sum128(q48_u128 v)
{
    v = q48_sum8_u128(v);
    v += q48_dpp128<Q48_DPP_MIRROR>(v);
    q48_u128 t = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> (32 * k)), 16 * r);
        t += ((q48_u128)(((uint64_t)w[3] << 32) | w[2]) << 64) | (((uint64_t)w[1] << 32) | w[0]);
    }
    return t;
}

__device__ __forceinline__ int64_t q48_wave_sum64(int64_t x)
{
    uint64_t v = (uint64_t)x;
    v += q48_dpp64<Q48_DPP_XOR1>(v);
    v += q48_dpp64<Q48_DPP_XOR2>(v);
    v += q48_dpp64<Q48_DPP_HALF_MIRROR>(v);
    v += q48_dpp64<Q48_DPP_MIRROR>(v);
    uint64_t t = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * r);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 16 * r);
        t += ((uint64_t)hi << 32) | lo;
    }
    return (int64_t)t;
}

// maximum across the 64 lanes of a wave (all active), every lane returns
// it: DPP within rows of 16 lanes, then the four row maxima as scalars
__device__ __forceinline__ int64_t q48_wave_max64(int64_t v)
{
    int64_t o = (int64_t)q48_dpp64<Q48_DPP_XOR1>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_XOR2>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_HALF_MIRROR>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_MIRROR>((uint64_t)v);
    v = o > v ? o : v;
    int64_t t = INT64_MIN;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * r);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32),
                                                               16 * r);
        const int64_t m = (int64_t)(((uint64_t)hi << 32) | lo);
        t = m > t ? m : t;
    }
    return t;
}
