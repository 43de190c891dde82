// q48_gemm.hip — token-batched Q16.48 GEMM on the int8 matrix cores (gfx950).
//
// Y[t][n] = (int64)((sum_k (int128)X[t][k] * W[n][k]) >> 48), per output
// exactly matmul_vec (llama_int.c:1014-1046) applied to each token row.
//
// Digits.  Every int64 v is written with nine signed digits,
//   v = sum_{i<=7} d_i 256^i + 2^64 d_8,
// from u = v + C mod 2^64, C = 0x0080808080808080: d_i = byte_i(u) - 128 for
// i <= 6 (in [-128, 127]), d_7 = byte_7(u) read as int8, and d_8 = 1 when v + C
// overflowed int64 (v >= 2^63 - C, so u < 0 <= v), else 0.  Zero has all digits
// zero, and so have the high digits of a small value and the low digits of a
// value with few significant bits (a bfloat16 weight in Q16.48 has three or
// four nonzero digits, an activation below 2^55 none above d_6).  Then
//   sum_k X W = sum_{a,b<=8} 256^(a+b) P_ab,   P_ab = sum_k d_a(X_k) d_b(W_k),
// an exact integer identity over any k range with no correction terms.  Only
// bits [48,112) are observable, so the pairs with a + b >= 14 are dropped and
// the rest are grouped by d = a + b into 14 int32 accumulators Q_d; |Q_d| <=
// 8 * 2^14 * K < 2^31 while K < 16384 per accumulation run (the plane-8
// products are at most 2^7 each; longer K is split across blocks and summed in
// int128).
//
// Block: 4 waves, 64 tokens x 64 rows; wave w owns 32 tokens x 32 rows as 14
// v_mfma_i32_32x32x32_i8 accumulators (224 registers, one wave per SIMD).
// Per k-step of 32 elements the block splits the int64 tiles into nine byte
// planes in LDS (double-buffered) and records which planes of each tile hold a
// nonzero digit.  k_gemm_i8 multiplies X planes 0..6 by a window of W planes
// LO..LO + 3 (28 MFMAs a step, 7 more in a step whose W tile reaches plane
// LO - 1), LO chosen from the block's first W tile; a block meeting a tile
// outside that (X digits in planes 7-8, W digits outside LO - 1 .. LO + 3)
// writes nothing and k_gemm_i8_full redoes it with every pair (63, plus the
// plane-8 pairs of a tile holding an overflowed value).  Activations below
// 2^55 and bfloat16-exact weights always fit.  The global loads run two steps
// ahead and the byte split of the next step is interleaved with the MFMAs of
// the current one.
#include "q48_digits.hpp"
#include "../../include/intllm_hip.h"

namespace {

constexpr int MT = 64;             // tokens per block
constexpr int MN = 64;             // rows per block
constexpr int MK = 32;             // k per step: one MFMA depth
constexpr int MAXK_RUN = 16320;    // k per accumulation run: |Q_d| < 2^31
constexpr int NPAIR = MK / 32;     // (row, 8 elements) pieces per thread per operand
constexpr int CH = MK / 16;        // 16-byte k chunks per row and plane
constexpr int NPL = 9;             // digit planes per operand

// Byte planes of one stage: [plane][32-row slice][k chunk][32 rows][16 bytes].
// The 64 lanes of an MFMA operand read (row l % 32, chunk 2h + l / 32) touch
// 1 KiB of consecutive bytes, and the 32 lanes of a half-wave store 256
// consecutive bytes: no bank conflicts either way.
constexpr int SLICE = CH * 512;    // one 32-row slice of one plane
constexpr int PLANE = 2 * SLICE;   // 64 rows of one plane
constexpr int STAGE = NPL * PLANE; // one operand: 18 KiB

// Piece p (0 .. 64 CH - 1) of a tile: row r, elements [k8, k8 + 8) of the
// step, and its byte offset in a plane.  Lanes 2i, 2i + 1 take one 16-byte
// chunk of row i: a half-wave covers 16 rows x 16 bytes.
struct Piece {
    int r, k8, off;
};
__device__ __forceinline__ Piece piece(int p)
{
    const int lo = p & 1, rl = (p >> 1) & 15, c = (p >> 5) % CH, rh = (p >> 5) / CH;
    const int r = rh * 16 + rl;
    return {r, (2 * c + lo) * 8, (r >> 5) * SLICE + c * 512 + (r & 31) * 16 + 8 * lo};
}

// Eight consecutive int64 of one row -> nine 8-byte digit words, digit a of
// element e in byte e of word a, stored at plane a.  Returns the planes that
// hold a nonzero digit (bit a).
__device__ __forceinline__ uint32_t split_store(uint8_t *stage, int off, const uint64_t (&v)[8])
{
    uint64_t u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        u[e] = v[e] + kDig;
    uint32_t l0[4], l1[4], h0[4], h1[4];
    tr4((uint32_t)u[0], (uint32_t)u[1], (uint32_t)u[2], (uint32_t)u[3], l0);
    tr4((uint32_t)u[4], (uint32_t)u[5], (uint32_t)u[6], (uint32_t)u[7], l1);
    tr4((uint32_t)(u[0] >> 32), (uint32_t)(u[1] >> 32), (uint32_t)(u[2] >> 32),
        (uint32_t)(u[3] >> 32), h0);
    tr4((uint32_t)(u[4] >> 32), (uint32_t)(u[5] >> 32), (uint32_t)(u[6] >> 32),
        (uint32_t)(u[7] >> 32), h1);
    uint2 d[NPL];
#pragma unroll
    for (int a = 0; a < 4; ++a)
        d[a] = make_uint2(l0[a] ^ 0x80808080u, l1[a] ^ 0x80808080u);
#pragma unroll
    for (int a = 0; a < 3; ++a)
        d[4 + a] = make_uint2(h0[a] ^ 0x80808080u, h1[a] ^ 0x80808080u);
    d[7] = make_uint2(h0[3], h1[3]);
    // overflow flags: bit 31 of u's high word set where v's is clear
    uint32_t f0 = 0, f1 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f0 |= (((uint32_t)(u[e] >> 32) & ~(uint32_t)(v[e] >> 32)) >> 31) << (8 * e);
        f1 |= (((uint32_t)(u[e + 4] >> 32) & ~(uint32_t)(v[e + 4] >> 32)) >> 31) << (8 * e);
    }
    d[8] = make_uint2(f0, f1);
    uint8_t *p = stage + off;
    uint32_t m = 0;
#pragma unroll
    for (int a = 0; a < NPL; ++a) {
        *reinterpret_cast<uint2 *>(p + a * PLANE) = d[a];
        m |= ((d[a].x | d[a].y) != 0 ? 1u : 0u) << a;
    }
    return m;
}

// The window pass's split of eight consecutive int64: only planes P0..P1 are
// stored.  Returns bit 0 when a digit outside P0..P1 is nonzero or a value may
// have overflowed (v >= 2^63 - C needs v's high word >= 0x7F7F7F7F: tested on
// that word alone, so a few values below the bound are caught too), and bit 1
// when plane EXT (-1: none) holds a nonzero digit.
template <int P0, int P1, int EXT>
__device__ __forceinline__ uint32_t split_store_win(uint8_t *stage, int off,
                                                   const uint64_t (&v)[8])
{
    uint64_t u[8];
    bool big = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        u[e] = v[e] + kDig;
        big |= (int32_t)(uint32_t)(v[e] >> 32) >= 0x7f7f7f7f;
    }
    uint32_t l0[4], l1[4], h0[4], h1[4];
    tr4((uint32_t)u[0], (uint32_t)u[1], (uint32_t)u[2], (uint32_t)u[3], l0);
    tr4((uint32_t)u[4], (uint32_t)u[5], (uint32_t)u[6], (uint32_t)u[7], l1);
    tr4((uint32_t)(u[0] >> 32), (uint32_t)(u[1] >> 32), (uint32_t)(u[2] >> 32),
        (uint32_t)(u[3] >> 32), h0);
    tr4((uint32_t)(u[4] >> 32), (uint32_t)(u[5] >> 32), (uint32_t)(u[6] >> 32),
        (uint32_t)(u[7] >> 32), h1);
    uint2 d[8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
        d[a] = make_uint2(l0[a] ^ 0x80808080u, l1[a] ^ 0x80808080u);
#pragma unroll
    for (int a = 0; a < 3; ++a)
        d[4 + a] = make_uint2(h0[a] ^ 0x80808080u, h1[a] ^ 0x80808080u);
    d[7] = make_uint2(h0[3], h1[3]);
    uint8_t *p = stage + off;
    uint32_t out = 0;
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        if (a >= P0 && a <= P1)
            *reinterpret_cast<uint2 *>(p + a * PLANE) = d[a];
        else
            out |= d[a].x | d[a].y;
    }
    uint32_t r = (out != 0 || big) ? 1u : 0u;
    if (EXT >= 0)
        r |= (d[EXT < 0 ? 0 : EXT].x | d[EXT < 0 ? 0 : EXT].y) != 0 ? 2u : 0u;
    return r;
}

// Eight elements [k, k + 8) of a row; positions at or past kend read as 0
// (all digits zero, so they add nothing to any Q_d).
template <bool VEC, bool TAIL>
__device__ __forceinline__ void load8(uint64_t (&v)[8], const int64_t *row, int k, int kend)
{
    if (!TAIL && VEC) {
        const ulonglong2 *p = reinterpret_cast<const ulonglong2 *>(row + k);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const ulonglong2 u = p[e];
            v[2 * e] = u.x;
            v[2 * e + 1] = u.y;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = (!TAIL || k + e < kend) ? (uint64_t)row[TAIL ? min(k + e, kend - 1) : k + e]
                                           : 0;
    }
}

// OR of a 32-bit value over the wave (DPP within rows of 16, then the rows)
__device__ __forceinline__ uint32_t wave_or(uint32_t v)
{
    v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Q48_DPP_XOR1, 0xf, 0xf, false);
    v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Q48_DPP_XOR2, 0xf, 0xf, false);
    v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Q48_DPP_HALF_MIRROR, 0xf, 0xf, false);
    v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Q48_DPP_MIRROR, 0xf, 0xf, false);
    return (uint32_t)(__builtin_amdgcn_readlane((int)v, 0) | __builtin_amdgcn_readlane((int)v, 16) |
                      __builtin_amdgcn_readlane((int)v, 32) | __builtin_amdgcn_readlane((int)v, 48));
}

// Operand offset of lane l in a 32-row slice of a plane (one 32-deep half)
__device__ __forceinline__ int opnd_off(int lane) { return (lane >> 5) * 512 + (lane & 31) * 16; }

// The 28 MFMAs of a step whose X digits lie in planes 0..6 and W digits in
// planes LO..LO + 3.
template <int LO>
__device__ __forceinline__ void mfma_window(v16i (&acc)[14], const uint8_t *xs, const uint8_t *ws,
                                            int lane)
{
    static_assert(LO >= 0 && LO + 3 <= 7, "window within planes 0..7");
    const int off = opnd_off(lane);
    v4i A[7], B[4];
#pragma unroll
    for (int a = 0; a < 7; ++a)
        A[a] = *reinterpret_cast<const v4i *>(xs + a * PLANE + off);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        B[j] = *reinterpret_cast<const v4i *>(ws + (LO + j) * PLANE + off);
#pragma unroll
    for (int a = 0; a < 7; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[a + LO + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[a], B[j], acc[a + LO + j],
                                                                    0, 0, 0);
}

// X planes 0..6 against one more W plane B (B <= 7).
template <int B>
__device__ __forceinline__ void mfma_plane_w(v16i (&acc)[14], const uint8_t *xs,
                                             const uint8_t *ws, int lane)
{
    const int off = opnd_off(lane);
    const v4i Bv = *reinterpret_cast<const v4i *>(ws + B * PLANE + off);
#pragma unroll
    for (int a = 0; a < 7; ++a)
        if (a + B <= 13) {
            const v4i A = *reinterpret_cast<const v4i *>(xs + a * PLANE + off);
            acc[a + B] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bv, acc[a + B], 0, 0, 0);
        }
}

// The 63 MFMAs of planes 0..7 x 0..7 (a + b <= 13).
__device__ __forceinline__ void mfma_all(v16i (&acc)[14], const uint8_t *xs, const uint8_t *ws,
                                         int lane)
{
    const int off = opnd_off(lane);
    v4i A[8], B[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        A[a] = *reinterpret_cast<const v4i *>(xs + a * PLANE + off);
        B[a] = *reinterpret_cast<const v4i *>(ws + a * PLANE + off);
    }
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b)
            if (a + b <= 13)
                acc[a + b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[a], B[b], acc[a + b], 0, 0, 0);
}

// The plane-8 pairs: X planes 0..5 with W plane 8 (wide: W overflowed) and X
// plane 8 with W planes 0..5.
__device__ __forceinline__ void mfma_plane8(v16i (&acc)[14], const uint8_t *xs,
                                            const uint8_t *ws, int lane, bool w8, bool x8)
{
    const int off = opnd_off(lane);
    if (w8) {
        const v4i B8 = *reinterpret_cast<const v4i *>(ws + 8 * PLANE + off);
#pragma unroll
        for (int a = 0; a < 6; ++a) {
            const v4i A = *reinterpret_cast<const v4i *>(xs + a * PLANE + off);
            acc[a + 8] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B8, acc[a + 8], 0, 0, 0);
        }
    }
    if (x8) {
        const v4i A8 = *reinterpret_cast<const v4i *>(xs + 8 * PLANE + off);
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            const v4i B = *reinterpret_cast<const v4i *>(ws + b * PLANE + off);
            acc[b + 8] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A8, B, acc[b + 8], 0, 0, 0);
        }
    }
}

// Tile of block b in a grid of nn row tiles x nt token tiles.  Blocks go
// round-robin to the 8 XCDs (each with its own L2), so b is first renumbered
// to give every XCD a contiguous range, and that range is walked in groups of
// GROUP row tiles: a group's W tiles stay in cache while its token tiles pass.
constexpr int GROUP = 8;
__device__ __forceinline__ void tile_of(int b, int nn, int nt, int &n_tile, int &t_tile)
{
    const int total = nn * nt, q = total / 8, r = total % 8, x = b % 8, l = b / 8;
    const int pid = x < r ? x * (q + 1) + l : r * (q + 1) + (x - r) * q + l;
    const int per = GROUP * nt, g = pid / per, first = g * GROUP;
    const int gs = min(nn - first, GROUP), in = pid - g * per;
    n_tile = first + in % gs;
    t_tile = in / gs;
}

// Register i of the 14 digit-sum accumulators as the 128-bit sum
// S = sum_d acc[d][i] 256^d (mod 2^128, words lo and hi), where only digit
// sums D0..D1 can be nonzero.  Groups of four digit sums are exact int64
// (|g| < 2^31 (1 + 2^8 + 2^16 + 2^24) < 2^56), then
// S = g0 + 2^32 g1 + 2^64 g2 + 2^96 g3 in two words with one carry.
template <int D0, int D1>
__device__ __forceinline__ void acc_sum128(const v16i (&acc)[14], int i, uint64_t &lo,
                                           uint64_t &hi)
{
    int64_t g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint64_t v = 0;
#pragma unroll
        for (int e = 3; e >= 0; --e) {
            const int d = 4 * j + e;
            v <<= 8;
            if (d >= D0 && d <= D1 && d < 14)
                v += (uint64_t)(int64_t)acc[d][i];
        }
        g[j] = (int64_t)v;
    }
    lo = (uint64_t)g[0] + ((uint64_t)g[1] << 32);
    const uint64_t carry = lo < (uint64_t)g[0] ? 1u : 0u;
    hi = (uint64_t)(g[0] >> 63) + (uint64_t)(g[1] >> 32) + carry + (uint64_t)g[2] +
         ((uint64_t)g[3] << 32);
}

// The block's tiles, loaders and accumulators, shared by the kernel's paths.
struct GemmTile {
    int64_t *Y;
    uint64_t *P;
    int T, N, n0, t0, kbeg, kend, nfull, z, S;
    bool tail;
};

// Block b's tile and k range (split z of S, spb steps each), and the rows it
// loads: piece tid of both tiles.
__device__ __forceinline__ GemmTile gemm_tile(int b, int z, int S, int64_t *Y, uint64_t *P,
                                              const int64_t *W, const int64_t *X, int T, int N,
                                              int K, int spb, Piece (&pc)[NPAIR],
                                              const int64_t *(&xrow)[NPAIR],
                                              const int64_t *(&wrow)[NPAIR])
{
    int n_tile, t_tile;
    tile_of(b, (N + MN - 1) / MN, (T + MT - 1) / MT, n_tile, t_tile);
    GemmTile g;
    g.Y = Y;
    g.P = P;
    g.T = T;
    g.N = N;
    g.n0 = n_tile * MN;
    g.t0 = t_tile * MT;
    g.z = z;
    g.S = S;
    g.kbeg = z * spb * MK;
    g.kend = max(g.kbeg, min(K, g.kbeg + spb * MK));
    g.nfull = (g.kend - g.kbeg) / MK;
    g.tail = (g.kend - g.kbeg) % MK != 0;
#pragma unroll
    for (int j = 0; j < NPAIR; ++j) {
        pc[j] = piece((int)threadIdx.x + 256 * j);
        xrow[j] = X + (size_t)min(g.t0 + pc[j].r, T - 1) * K + pc[j].k8;
        wrow[j] = W + (size_t)min(g.n0 + pc[j].r, N - 1) * K + pc[j].k8;
    }
    return g;
}

// One pass of the block's k range.  LO >= 0: X planes 0..6 against W planes
// LO..LO + 3, plus W plane LO - 1 in the steps whose tile holds it; a step
// with digits elsewhere returns false before anything is written (the caller
// then runs LO = -1).  LO = -1: every pair, never fails.  On success the
// block's outputs are written.
template <int LO, bool VEC>
__device__ __forceinline__ bool gemm_pass(const GemmTile &g, uint8_t (&lds)[2][2][STAGE],
                                          uint32_t (&pm)[2][4], const int64_t *const (&xrow)[NPAIR],
                                          const int64_t *const (&wrow)[NPAIR],
                                          const Piece (&pc)[NPAIR])
{
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wt = w >> 1, wn = w & 1;   // wave's token slice, row slice
    const int kbeg = g.kbeg, kend = g.kend, nfull = g.nfull;
    v16i acc[14];
#pragma unroll
    for (int d = 0; d < 14; ++d)
        acc[d] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    typedef uint64_t Regs[NPAIR][8];
    auto load = [&](Regs &gx, Regs &gw, int k) {
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
            load8<VEC, false>(gx[j], xrow[j], k, kend);
            load8<VEC, false>(gw[j], wrow[j], k, kend);
        }
    };
    // split a step's tiles into stage st and publish the wave's plane masks
    // W planes a window pass stores and takes: LO - 1 .. LO + 3
    constexpr int WP0 = LO > 0 ? LO - 1 : 0, WP1 = LO + 3, WEXT = LO > 0 ? LO - 1 : -1;
    // split a step's tiles into stage st and publish the wave's plane masks:
    // every plane's (X in bits 0..8, W in 9..17) for the full pass; for a
    // window pass bit 0 = a digit outside the window, bit 1 = W plane LO - 1
    auto store = [&](int st, const Regs &gx, const Regs &gw) {
        uint32_t m;
        if constexpr (LO >= 0) {
            uint32_t r = 0;
#pragma unroll
            for (int j = 0; j < NPAIR; ++j)
                r |= split_store_win<0, 6, -1>(lds[st][0], pc[j].off, gx[j]) |
                     split_store_win<WP0, WP1, WEXT>(lds[st][1], pc[j].off, gw[j]);
            m = (__builtin_amdgcn_ballot_w64((r & 1u) != 0) != 0 ? 1u : 0u) |
                (__builtin_amdgcn_ballot_w64((r & 2u) != 0) != 0 ? 2u : 0u);
        } else {
            uint32_t mx = 0, mw = 0;
#pragma unroll
            for (int j = 0; j < NPAIR; ++j) {
                mx |= split_store(lds[st][0], pc[j].off, gx[j]);
                mw |= split_store(lds[st][1], pc[j].off, gw[j]);
            }
            m = wave_or(mx | (mw << 9));
        }
        if (lane == 0)
            pm[st][w] = m;
    };
    // the stage's masks (uniform over the block)
    auto planes = [&](int st) {
        const uint32_t m = pm[st][0] | pm[st][1] | pm[st][2] | pm[st][3];
        return (uint32_t)__builtin_amdgcn_readfirstlane((int)m);
    };
    bool ok = true;
    // MFMAs of stage st with the split of the next step interleaved (its data
    // arrived a step ago); the last step splits a clamped re-read, never used
    auto multiply = [&](int st, bool split_next, const Regs &cx_, const Regs &cw_) {
        const uint8_t *xs = &lds[st][0][0] + wt * SLICE, *ws = &lds[st][1][0] + wn * SLICE;
        const uint32_t m = planes(st);
        if constexpr (LO >= 0) {
            // a step outside the window still runs (its products are
            // discarded with the pass), so the loop body has no exit
            ok &= (m & 1u) == 0;
            mfma_window<LO < 0 ? 0 : LO>(acc, xs, ws, lane);
            if (split_next)
                store(st ^ 1, cx_, cw_);
            __builtin_amdgcn_sched_group_barrier(0x100, 11, 0);
#pragma unroll
            for (int i = 0; i < 28; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
            if (LO > 0 && (m & 2u))
                mfma_plane_w<LO < 1 ? 0 : LO - 1>(acc, xs, ws, lane);
        } else {
            const uint32_t mx = m & 0x1ffu, mw = m >> 9;
            mfma_all(acc, xs, ws, lane);
            if (split_next)
                store(st ^ 1, cx_, cw_);
            __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
            for (int i = 0; i < 63; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
            if ((mw | mx) & 0x100u)
                mfma_plane8(acc, xs, ws, lane, (mw & 0x100u) != 0, (mx & 0x100u) != 0);
        }
    };
    // Steps go two ahead: step s multiplies stage s & 1, splits step s + 1
    // (loaded during step s - 1) into the other stage and loads step s + 2.
    // Register sets alternate: step s loads into set s & 1.
    // The window pass loads three steps ahead (register sets rotating by
    // step), so a step's tiles have two steps to arrive; the full pass, at
    // the register limit, two.
    constexpr int AHEAD = LO >= 0 ? 3 : 2;
    Regs gx0, gw0, gx1, gw1, gx2, gw2;
    const int last = max(nfull - 1, 0);
    __syncthreads();   // the stages and masks of an earlier pass are consumed
    if (nfull > 0) {
        load(gx0, gw0, kbeg);
        load(gx1, gw1, kbeg + min(1, last) * MK);
        if (AHEAD == 3)
            load(gx2, gw2, kbeg + min(2, last) * MK);
        store(0, gx0, gw0);
    }
    __syncthreads();
    auto step = [&](int s, Regs &lx, Regs &lw, const Regs &cx_, const Regs &cw_) {
        // step s + AHEAD's tiles (clamped to the last step: in bounds, unused)
        load(lx, lw, kbeg + min(s + AHEAD, last) * MK);
        __builtin_amdgcn_sched_barrier(0);
        multiply(s & 1, true, cx_, cw_);
        __syncthreads();
    };
    // groups with no branch inside the loop body's loads; a failed step is
    // seen by the whole block (the masks are uniform), which leaves together
    int s = 0;
    if constexpr (AHEAD == 3) {
        for (; ok && s + 2 < nfull; s += 3) {
            step(s, gx0, gw0, gx1, gw1);
            step(s + 1, gx1, gw1, gx2, gw2);
            step(s + 2, gx2, gw2, gx0, gw0);
        }
        if (ok && s < nfull)
            step(s, gx0, gw0, gx1, gw1);
        if (ok && s + 1 < nfull)
            step(s + 1, gx1, gw1, gx2, gw2);
    } else {
        for (; ok && s + 1 < nfull; s += 2) {
            step(s, gx0, gw0, gx1, gw1);
            if (ok)
                step(s + 1, gx1, gw1, gx0, gw0);
        }
        if (ok && s < nfull)
            step(s, gx0, gw0, gx1, gw1);
    }
    if (ok && g.tail) {
        const int kt = kbeg + nfull * MK;
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
            load8<VEC, true>(gx0[j], xrow[j], kt, kend - pc[j].k8);
            load8<VEC, true>(gw0[j], wrow[j], kt, kend - pc[j].k8);
        }
        store(nfull & 1, gx0, gw0);
        __syncthreads();
        multiply(nfull & 1, false, gx0, gw0);
    }
    if (!ok)
        return false;

    // lane l, register i: token 8 (i / 4) + 4 (l / 32) + i % 4, row l % 32;
    // the window pass touches digit sums LO - 1 .. LO + 9 only
    constexpr int D0 = LO > 0 ? LO - 1 : 0, D1 = LO < 0 ? 13 : LO + 9;
    const int nl = 32 * wn + (lane & 31), n = g.n0 + nl;
    if (n >= g.N)
        return true;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int tl = 32 * wt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3), t = g.t0 + tl;
        if (t >= g.T)
            continue;
        uint64_t lo, hi;
        acc_sum128<D0, D1>(acc, i, lo, hi);
        if (g.S == 1) {
            g.Y[(size_t)t * g.N + n] = (int64_t)((hi << 16) | (lo >> 48));
        } else {
            uint64_t *p = g.P + 2 * (((size_t)g.z * g.T + t) * g.N + n);
            *reinterpret_cast<ulonglong2 *>(p) = make_ulonglong2(lo, hi);
        }
    }
    return true;
}

// grid (ceil(N/64) * ceil(T/64), 1, S): split z covers k-steps [z*spb, (z+1)*spb).
// S == 1: Y gets the shifted result;
// S > 1: P[z][t][n] gets the block's int128 partial sum (two uint64, lo first).
// The window of W planes comes from the block's first W tile (its top plane
// h gives LO = h - 3, clamped to 0..4: small weights reach lower planes, the
// largest magnitudes set the top).  A block whose tiles leave the window
// writes nothing and sets redo[block] (else clears it) for k_gemm_i8_full.
template <bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void
k_gemm_i8(int64_t *__restrict__ Y, uint64_t *__restrict__ P, int *__restrict__ redo,
          const int64_t *__restrict__ W, const int64_t *__restrict__ X, int T, int N, int K,
          int spb)
{
    __shared__ __align__(16) uint8_t lds[2][2][STAGE];   // [stage][X, W]
    __shared__ uint32_t pm[2][4];                         // [stage][wave]: planes, X | W << 9
    const int tid = threadIdx.x;
    Piece pc[NPAIR];
    const int64_t *xrow[NPAIR], *wrow[NPAIR];
    const GemmTile g = gemm_tile(blockIdx.x, blockIdx.z, gridDim.z, Y, P, W, X, T, N, K, spb,
                                 pc, xrow, wrow);

    // the first W tile's planes (every digit of the block's first step)
    uint32_t mw = 0;
    if (g.kend > g.kbeg) {
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
            uint64_t v[8];
            if (g.nfull > 0)
                load8<VEC, false>(v, wrow[j], g.kbeg, g.kend);
            else
                load8<VEC, true>(v, wrow[j], g.kbeg, g.kend - pc[j].k8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint64_t u = v[e] + kDig, dz = u ^ kDig;   // digits 0..6: bytes of dz
#pragma unroll
                for (int a = 0; a < 7; ++a)
                    mw |= ((dz >> (8 * a)) & 0xffu) != 0 ? 1u << a : 0u;
                mw |= (u >> 56) != 0 ? 1u << 7 : 0u;
            }
        }
    }
    mw = wave_or(mw);
    if ((tid & 63) == 0)
        pm[0][tid >> 6] = mw;
    __syncthreads();
    mw = (uint32_t)__builtin_amdgcn_readfirstlane((int)(pm[0][0] | pm[0][1] | pm[0][2] | pm[0][3]));
    const int h = mw ? 31 - __builtin_clz(mw) : 3;
    const int lo = min(max(h - 3, 0), 4);
    bool done;
    switch (lo) {
    case 0: done = gemm_pass<0, VEC>(g, lds, pm, xrow, wrow, pc); break;
    case 1: done = gemm_pass<1, VEC>(g, lds, pm, xrow, wrow, pc); break;
    case 2: done = gemm_pass<2, VEC>(g, lds, pm, xrow, wrow, pc); break;
    case 3: done = gemm_pass<3, VEC>(g, lds, pm, xrow, wrow, pc); break;
    default: done = gemm_pass<4, VEC>(g, lds, pm, xrow, wrow, pc); break;
    }
    if (tid == 0)
        redo[blockIdx.z * gridDim.x + blockIdx.x] = done ? 0 : 1;
}

// Every pair for the blocks k_gemm_i8 left (redo set), nb blocks of S splits:
// block b of this grid takes blocks b, b + gridDim.x, ... of that grid.
template <bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void
k_gemm_i8_full(int64_t *__restrict__ Y, uint64_t *__restrict__ P, const int *__restrict__ redo,
               const int64_t *__restrict__ W, const int64_t *__restrict__ X, int T, int N,
               int K, int spb, int nb, int S)
{
    __shared__ __align__(16) uint8_t lds[2][2][STAGE];
    __shared__ uint32_t pm[2][4];
    __shared__ int list[256], cnt;
    // the block's candidates i = blockIdx.x + c gridDim.x, 256 flags read at
    // once (one memory round trip when nothing is to be redone)
    const int tid = threadIdx.x, per = (nb * S - (int)blockIdx.x + gridDim.x - 1) / gridDim.x;
    for (int c0 = 0; c0 < per; c0 += 256) {
        if (tid == 0)
            cnt = 0;
        __syncthreads();
        const int i = (int)blockIdx.x + (c0 + tid) * (int)gridDim.x;
        if (c0 + tid < per && redo[i])
            list[atomicAdd(&cnt, 1)] = i;
        __syncthreads();
        const int n = cnt;
        for (int l = 0; l < n; ++l) {
            const int b = list[l];
            Piece pc[NPAIR];
            const int64_t *xrow[NPAIR], *wrow[NPAIR];
            const GemmTile g =
                gemm_tile(b % nb, b / nb, S, Y, P, W, X, T, N, K, spb, pc, xrow, wrow);
            gemm_pass<-1, VEC>(g, lds, pm, xrow, wrow, pc);
        }
        __syncthreads();   // list and cnt reused
    }
}

// Y[t][n] = (sum_z P[z][t][n]) >> 48
__global__ __launch_bounds__(256) void k_gemm_i8_reduce(int64_t *__restrict__ Y,
                                                       const uint64_t *__restrict__ P, int T,
                                                       int N, int S)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * N)
        return;
    q48_u128 tot = 0;
    for (int z = 0; z < S; ++z) {
        const ulonglong2 u =
            *reinterpret_cast<const ulonglong2 *>(P + 2 * ((size_t)z * T * N + i));
        tot += ((q48_u128)u.y << 64) | u.x;
    }
    Y[i] = (int64_t)((q48_i128)tot >> 48);
}

// ---------------------------------------------------------------------------
// Planes path: operands split once into digit planes in HBM, then moved
// into LDS by DMA (global_load_lds), so the k loop runs no digit split.
// ---------------------------------------------------------------------------

// Digit planes of a row-major int64 matrix (R rows, K columns) in the LDS
// stage order of the window kernels: per row tile rt (64 rows) and k-step s
// (32 columns), block rt * nsteps + s holds planes 0..7 of the nine-digit
// form, 2 KB each ([32-row slice][16-column chunk][32 rows][16 bytes]; rows
// past R and columns past K are zero), and mask[rt * nsteps + s] has bit a
// when plane a holds a nonzero digit and bit 8 when a value may have
// overflowed v + C (high word >= 0x7F7F7F7F; plane 8 itself is not stored).
__global__ __launch_bounds__(256) void k_planes(uint8_t *__restrict__ dst,
                                               uint32_t *__restrict__ mask,
                                               const int64_t *__restrict__ src, int R, int K,
                                               int nsteps)
{
    __shared__ uint32_t red[4];
    const int tid = threadIdx.x;
    const int rt = (int)blockIdx.x / nsteps, st = (int)blockIdx.x % nsteps;
    const Piece pc = piece(tid);
    const int row = rt * MN + pc.r, k0 = st * MK + pc.k8;
    uint64_t v[8];
    const int64_t *rp = src + (size_t)min(row, R - 1) * K + k0;
    if (row < R && k0 + 8 <= K && (((uintptr_t)rp) & 15) == 0) {
        const ulonglong2 *q = reinterpret_cast<const ulonglong2 *>(rp);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const ulonglong2 u = q[e];
            v[2 * e] = u.x;
            v[2 * e + 1] = u.y;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = row < R && k0 + e < K ? (uint64_t)rp[e] : 0;
    }
    uint64_t u[8];
    bool big = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        u[e] = v[e] + kDig;
        big |= (int32_t)(uint32_t)(v[e] >> 32) >= 0x7f7f7f7f;
    }
    uint32_t l0[4], l1[4], h0[4], h1[4];
    tr4((uint32_t)u[0], (uint32_t)u[1], (uint32_t)u[2], (uint32_t)u[3], l0);
    tr4((uint32_t)u[4], (uint32_t)u[5], (uint32_t)u[6], (uint32_t)u[7], l1);
    tr4((uint32_t)(u[0] >> 32), (uint32_t)(u[1] >> 32), (uint32_t)(u[2] >> 32),
        (uint32_t)(u[3] >> 32), h0);
    tr4((uint32_t)(u[4] >> 32), (uint32_t)(u[5] >> 32), (uint32_t)(u[6] >> 32),
        (uint32_t)(u[7] >> 32), h1);
    uint2 d[8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
        d[a] = make_uint2(l0[a] ^ 0x80808080u, l1[a] ^ 0x80808080u);
#pragma unroll
    for (int a = 0; a < 3; ++a)
        d[4 + a] = make_uint2(h0[a] ^ 0x80808080u, h1[a] ^ 0x80808080u);
    d[7] = make_uint2(h0[3], h1[3]);
    uint8_t *p = dst + (size_t)blockIdx.x * 8 * PLANE + pc.off;
    uint32_t m = big ? 0x100u : 0u;
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        *reinterpret_cast<uint2 *>(p + a * PLANE) = d[a];
        m |= (d[a].x | d[a].y) != 0 ? 1u << a : 0u;
    }
    m = wave_or(m);
    if ((tid & 63) == 0)
        red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0)
        mask[blockIdx.x] = red[0] | red[1] | red[2] | red[3];
}

// One LDS stage of the planes path: X planes 0..6, then W planes WP0 .. WP0 + 4.
constexpr int PX_BYTES = 7 * PLANE, PSTAGE = 12 * PLANE;

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef const __attribute__((address_space(4))) uint32_t *ConstMask;

// Workgroup barrier without the fence of __syncthreads (whose release waits
// for every DMA still in flight); the caller's s_waitcnt before it decides
// which DMA the barrier publishes.  The empty asm keeps LDS accesses on
// their side of it.
__device__ __forceinline__ void stage_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The k loop of one window (LO) over a ring of four LDS stages.  Step i:
//   wait for step i + 1's DMA (this wave's), barrier (every wave's);
//   DMA step i + 3 into the stage step i - 1 used (each wave moves six 1 KB
//   chunks: 64 lanes x 16 bytes);
//   read step i + 1's operands into the spare register set, while the MFMAs
//   of step i run on the set read during step i - 1.
// The stages are four LDS objects named statically in each step (the loop
// is unrolled by four), so the compiler's own waits for the reads of one
// stage do not count the DMA into another.
template <int LO>
__device__ __forceinline__ void planes_pass(uint8_t (&s0)[PSTAGE], uint8_t (&s1)[PSTAGE],
                                            uint8_t (&s2)[PSTAGE], uint8_t (&s3)[PSTAGE],
                                            ConstMask wm, const uint8_t *xsrc,
                                            const uint8_t *wsrc, int ns, bool rev,
                                            v16i (&acc)[14])
{
    constexpr int WP0 = LO > 0 ? LO - 1 : 0;   // first W plane in the stage
    constexpr int NB = LO > 0 ? 5 : 4;         // W planes the MFMAs read
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wt = w >> 1, wn = w & 1;
    const int off = opnd_off(lane);
    const uint8_t *ws_src = wsrc + WP0 * PLANE;
    // step s of the loop is k-step rev ? ns - 1 - s : s of the block's range
    auto dma = [&](int s, uint8_t(&dst)[PSTAGE]) {
        s = rev ? ns - 1 - s : s;
#pragma unroll
        for (int j = 0; j < 6; ++j) {
            const int c = w + 4 * j;   // chunk 0..23: X 0..13, W 14..23
            const uint8_t *g = c < 14 ? xsrc + (size_t)s * 8 * PLANE + c * 1024
                                      : ws_src + (size_t)s * 8 * PLANE + (c - 14) * 1024;
            __builtin_amdgcn_global_load_lds(g + lane * 16, dst + c * 1024, 16, 0, 0);
        }
    };
    v4i A0[7], B0[NB], A1[7], B1[NB];
    auto rd = [&](const uint8_t(&src)[PSTAGE], v4i (&A)[7], v4i (&B)[NB]) {
#pragma unroll
        for (int a = 0; a < 7; ++a)
            A[a] = *reinterpret_cast<const v4i *>(src + wt * SLICE + a * PLANE + off);
#pragma unroll
        for (int j = 0; j < NB; ++j)
            B[j] = *reinterpret_cast<const v4i *>(src + PX_BYTES + j * PLANE + wn * SLICE + off);
    };
    // the step's MFMAs; ext: its W tile reaches plane LO - 1.  The reads of
    // the next step's operands (issued just before) go out one per MFMA
    // from the start, so they finish under the MFMAs.
    auto mult = [&](bool ext, const v4i (&A)[7], const v4i (&B)[NB]) {
#pragma unroll
        for (int a = 0; a < 7; ++a)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[a + LO + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[a], B[LO - WP0 + j],
                                                                        acc[a + LO + j], 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 7 + NB; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 28 - 7 - NB, 0);
        if (LO > 0 && ext) {
#pragma unroll
            for (int a = 0; a < 7; ++a)
                acc[a + WP0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[a], B[0], acc[a + WP0], 0,
                                                                     0, 0);
        }
    };
    auto ext_of = [&](int i) {
        uint32_t e = LO > 0 ? wm[rev ? ns - 1 - i : i] : 0;
        asm volatile("" : "+s"(e));
        return ((e >> WP0) & 1u) != 0;
    };
    // wait until at most n of this wave's chunk DMAs are in flight
    auto wait_n = [&](int n) {
        if (n >= 12)
            wait_vm<12>();
        else if (n >= 6)
            wait_vm<6>();
        else
            wait_vm<0>();
    };
    // prologue: steps 0..2 in flight, step 0 landed and read
    if (ns > 0)
        dma(0, s0);
    if (ns > 1)
        dma(1, s1);
    if (ns > 2)
        dma(2, s2);
    wait_n(6 * (min(ns, 3) - 1));
    stage_barrier();
    if (ns > 0)
        rd(s0, A0, B0);
    // steady state: every step has a step i + 3 to load.  The group's four
    // step masks come in one scalar load at its top, held there by the
    // empty asm (the wave waits for its operand reads at that point anyway;
    // a wait in mid-step would also wait for the reads just issued).
    int i = 0;
    for (; i + 6 < ns; i += 4) {
        uint32_t e0 = 0, e1 = 0, e2 = 0, e3 = 0;
        if (LO > 0) {
            const ConstMask g = wm + (rev ? ns - 4 - i : i);   // steps i .. i + 3
            const uint32_t g0 = g[0], g1 = g[1], g2 = g[2], g3 = g[3];
            e0 = rev ? g3 : g0;
            e1 = rev ? g2 : g1;
            e2 = rev ? g1 : g2;
            e3 = rev ? g0 : g3;
            asm volatile("" : "+s"(e0), "+s"(e1), "+s"(e2), "+s"(e3));
        }
        wait_vm<6>();
        stage_barrier();
        dma(i + 3, s3);
        rd(s1, A1, B1);
        mult((e0 >> WP0) & 1u, A0, B0);
        wait_vm<6>();
        stage_barrier();
        dma(i + 4, s0);
        rd(s2, A0, B0);
        mult((e1 >> WP0) & 1u, A1, B1);
        wait_vm<6>();
        stage_barrier();
        dma(i + 5, s1);
        rd(s3, A1, B1);
        mult((e2 >> WP0) & 1u, A0, B0);
        wait_vm<6>();
        stage_barrier();
        dma(i + 6, s2);
        rd(s0, A0, B0);
        mult((e3 >> WP0) & 1u, A1, B1);
    }
    // the last zero to six steps (i is a multiple of four: stages continue
    // the ring)
    auto tail = [&](int k, uint8_t(&nxt_st)[PSTAGE], uint8_t(&ld_st)[PSTAGE], v4i(&Ac)[7],
                    v4i(&Bc)[NB], v4i(&An)[7], v4i(&Bn)[NB]) {
        if (k >= ns)
            return;
        wait_n(k + 1 < ns ? 6 * (min(ns - 1, k + 2) - (k + 1)) : 0);
        stage_barrier();
        if (k + 3 < ns)
            dma(k + 3, ld_st);
        const bool ext = ext_of(k);
        if (k + 1 < ns)
            rd(nxt_st, An, Bn);
        mult(ext, Ac, Bc);
    };
    tail(i, s1, s3, A0, B0, A1, B1);
    tail(i + 1, s2, s0, A1, B1, A0, B0);
    tail(i + 2, s3, s1, A0, B0, A1, B1);
    tail(i + 3, s0, s2, A1, B1, A0, B0);
    tail(i + 4, s1, s3, A0, B0, A1, B1);
    tail(i + 5, s2, s0, A1, B1, A0, B0);
}

// grid (ceil(N/64) * ceil(T/64), 1, S) over operands split by k_planes
// (nsteps k-steps): split z covers steps [z spb, (z + 1) spb).  The block
// ORs its tiles' masks over its steps; the window is LO = top W plane - 3
// (clamped to 0..4); a block whose X digits reach plane 7 (or may overflow)
// or whose W digits leave LO - 1 .. LO + 3 writes nothing and sets
// redo[block] (else clears it) for k_gemm_i8_full.  S == 1: Y gets the
// shifted result; S > 1: P[z][t][n] the int128 partial.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void
k_gemm_i8p(int64_t *__restrict__ Y, uint64_t *__restrict__ P, int *__restrict__ redo,
           const uint8_t *__restrict__ Xp, const uint32_t *__restrict__ Xm,
           const uint8_t *__restrict__ Wp, const uint32_t *__restrict__ Wm, int T, int N,
           int nsteps, int spb, int cpx)
{
    __shared__ __align__(16) uint8_t st0[PSTAGE];
    __shared__ __align__(16) uint8_t st1[PSTAGE];
    __shared__ __align__(16) uint8_t st2[PSTAGE];
    __shared__ __align__(16) uint8_t st3[PSTAGE];
    __shared__ uint32_t red[2][4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int n_tile, t_tile;
    tile_of(blockIdx.x, (N + MN - 1) / MN, (T + MT - 1) / MT, n_tile, t_tile);
    const int s0 = (int)blockIdx.z * spb, ns = max(0, min(nsteps, s0 + spb) - s0);
    uint32_t mx = 0, mw = 0;
    for (int i = tid; i < ns; i += 256) {
        mx |= Xm[(size_t)t_tile * nsteps + s0 + i];
        mw |= Wm[(size_t)n_tile * nsteps + s0 + i];
    }
    mx = wave_or(mx);
    mw = wave_or(mw);
    if (lane == 0) {
        red[0][w] = mx;
        red[1][w] = mw;
    }
    __syncthreads();
    mx = (uint32_t)__builtin_amdgcn_readfirstlane((int)(red[0][0] | red[0][1] | red[0][2] | red[0][3]));
    mw = (uint32_t)__builtin_amdgcn_readfirstlane((int)(red[1][0] | red[1][1] | red[1][2] | red[1][3]));
    const int top = (mw & 0xffu) ? 31 - __builtin_clz(mw & 0xffu) : 3;
    const int LO = min(max(top - 3, 0), 4);
    const uint32_t win = ((0x1fu << LO) >> 1) & 0xffu;
    const bool fit = (mx & ~0x7fu) == 0 && (mw & ~win) == 0;
    if (tid == 0)
        redo[blockIdx.z * gridDim.x + blockIdx.x] = fit ? 0 : 1;
    if (!fit)
        return;   // uniform over the block

    v16i acc[14];
#pragma unroll
    for (int d = 0; d < 14; ++d)
        acc[d] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const uint8_t *xsrc = Xp + ((size_t)t_tile * nsteps + s0) * 8 * PLANE;
    const uint8_t *wsrc = Wp + ((size_t)n_tile * nsteps + s0) * 8 * PLANE;
    const ConstMask wm = (ConstMask)(Wm + (size_t)n_tile * nsteps + s0);
    // Blocks run in rounds of one per compute unit; each XCD's round holds 8
    // row tiles x 4 token tiles (tile_of), and the next round's blocks take
    // the same row tiles with the next token tiles.  Odd rounds walk k
    // downwards, so they start on the W planes the round before ended on,
    // which are still in L2.
    const bool rev = ((((int)blockIdx.x >> 3) / cpx) & 1) != 0;
    // lane l, register i: token 8 (i / 4) + 4 (l / 32) + i % 4, row l % 32;
    // window LO touches digit sums LO - 1 .. LO + 9 only
    const int wt = w >> 1, wn = w & 1;
    const int n = n_tile * MN + 32 * wn + (lane & 31);
    auto store = [&](auto d0, auto d1) {
        if (n >= N)
            return;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int t = t_tile * MT + 32 * wt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            if (t >= T)
                continue;
            uint64_t lo, hi;
            acc_sum128<decltype(d0)::value, decltype(d1)::value>(acc, i, lo, hi);
            if (gridDim.z == 1) {
                Y[(size_t)t * N + n] = (int64_t)((hi << 16) | (lo >> 48));
            } else {
                uint64_t *p = P + 2 * (((size_t)blockIdx.z * T + t) * N + n);
                *reinterpret_cast<ulonglong2 *>(p) = make_ulonglong2(lo, hi);
            }
        }
    };
    using std::integral_constant;
    switch (LO) {
    case 0:
        planes_pass<0>(st0, st1, st2, st3, wm, xsrc, wsrc, ns, rev, acc);
        store(integral_constant<int, 0>{}, integral_constant<int, 9>{});
        break;
    case 1:
        planes_pass<1>(st0, st1, st2, st3, wm, xsrc, wsrc, ns, rev, acc);
        store(integral_constant<int, 0>{}, integral_constant<int, 10>{});
        break;
    case 2:
        planes_pass<2>(st0, st1, st2, st3, wm, xsrc, wsrc, ns, rev, acc);
        store(integral_constant<int, 1>{}, integral_constant<int, 11>{});
        break;
    case 3:
        planes_pass<3>(st0, st1, st2, st3, wm, xsrc, wsrc, ns, rev, acc);
        store(integral_constant<int, 2>{}, integral_constant<int, 12>{});
        break;
    default:
        planes_pass<4>(st0, st1, st2, st3, wm, xsrc, wsrc, ns, rev, acc);
        store(integral_constant<int, 3>{}, integral_constant<int, 13>{});
        break;
    }
}

} // namespace

int q48_gemm_auto_kernel(int T, int N, int K)
{
    // measured on MI355X: the int8 kernel is 7-30x faster than the VALU
    // kernel at every T >= 16 of the TinyLlama shapes
    (void)T;
    (void)N;
    (void)K;
    return Q48_GEMM_I8;
}

int q48_gemm_i8_splits(int T, int N, int K, int cu_count)
{
    const int base = ((N + MN - 1) / MN) * ((T + MT - 1) / MT);
    const int steps = (K + MK - 1) / MK;
    const int min_s = (steps + MAXK_RUN / MK - 1) / (MAXK_RUN / MK);
    int s = 1;
    // split K while the grid is under one block per compute unit and every
    // split keeps at least 8 steps
    while (base * s < cu_count && steps / (2 * s) >= 8)
        s *= 2;
    return s > min_s ? s : min_s;
}

size_t q48_gemm_planes_size(int N, int K)
{
    const size_t tiles = (size_t)((N + MN - 1) / MN) * ((K + MK - 1) / MK);
    return tiles * 8 * PLANE + ((tiles * 4 + 255) & ~(size_t)255);
}

int q48_launch_gemm_prepare(q48_ctx *c, void *Wp, const int64_t *W, int N, int K)
{
    const int steps = (K + MK - 1) / MK, nn = (N + MN - 1) / MN;
    if ((size_t)nn * steps > 0x7fffffff)
        return Q48_EINVAL;
    uint8_t *p = (uint8_t *)Wp;
    uint32_t *m = (uint32_t *)(p + (size_t)nn * steps * 8 * PLANE);
    hipLaunchKernelGGL(k_planes, dim3(nn * steps), dim3(256), 0, c->stream, p, m, W, N, K,
                       steps);
    return (int)hipGetLastError();
}

int q48_launch_gemm_i8(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X, int T,
                       int N, int K, int kernel, const void *Wpre)
{
    const int S = q48_gemm_i8_splits(T, N, K, c->cu_count);
    const int steps = (K + MK - 1) / MK;
    const int spb = (steps + S - 1) / S;
    // blocks (and their redo flags) are numbered in int
    if ((size_t)((N + MN - 1) / MN) * ((T + MT - 1) / MT) * S > 0x7fffffff)
        return Q48_EINVAL;
    const int nt = (T + MT - 1) / MT, nn = (N + MN - 1) / MN, nb = nn * nt;
    // the planes path pays one split of X (and of W unless prepared) per
    // call: it wins once tiles are reused enough (measured: T >= 512 with
    // N >= 2048 faster by 7-39%, N = 256 slower by 5-22%, T = 128 even when
    // W is split in the call); with W prepared it wins from 2 tokens, where
    // the GEMM streams W and the planes hold 5 of its 8 bytes per element
    const bool fits = (size_t)max(nt, nn) * steps <= 0x7fffffff;
    const bool planes =
        fits && (kernel == Q48_GEMM_I8_PLANES ||
                 (kernel != Q48_GEMM_I8_FUSED && T >= (Wpre ? 2 : 256) && N >= 1024));
    const bool wsplit = planes && !Wpre;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    // workspace: the blocks' redo flags, (S > 1) the int128 partials, then
    // (planes path) X and W digit planes and their masks
    const size_t flags = al((size_t)nb * S * sizeof(int));
    const size_t part = S > 1 ? 16 * (size_t)S * T * N : 0;
    const size_t xpl = planes ? (size_t)nt * steps * 8 * PLANE : 0;
    const size_t wpl = wsplit ? (size_t)nn * steps * 8 * PLANE : 0;
    const size_t xms = planes ? al((size_t)nt * steps * 4) : 0;
    const size_t wms = wsplit ? al((size_t)nn * steps * 4) : 0;
    int rc = q48_ws_reserve(c, flags + part + xpl + wpl + xms + wms);
    if (rc)
        return rc;
    char *ws = (char *)c->ws;
    int *redo = (int *)ws;
    uint64_t *P = S > 1 ? (uint64_t *)(ws + flags) : nullptr;
    const dim3 grid(nb, 1, S);
    const int fgrid = min(nb * S, c->cu_count);
    const bool vec = K % 2 == 0 && (((uintptr_t)W | (uintptr_t)X) & 15) == 0;
    if (planes) {
        uint8_t *Xp = (uint8_t *)(ws + flags + part), *Wp = Xp + xpl;
        uint32_t *Xm = (uint32_t *)(Wp + wpl), *Wm = (uint32_t *)((char *)Xm + xms);
        hipLaunchKernelGGL(k_planes, dim3(nt * steps), dim3(256), 0, c->stream, Xp, Xm, X, T, K,
                           steps);
        if (Wpre) {
            // planes from q48_launch_gemm_prepare: masks after the planes
            Wp = (uint8_t *)Wpre;
            Wm = (uint32_t *)(Wp + (size_t)nn * steps * 8 * PLANE);
        } else {
            hipLaunchKernelGGL(k_planes, dim3(nn * steps), dim3(256), 0, c->stream, Wp, Wm, W, N,
                               K, steps);
        }
        hipLaunchKernelGGL(k_gemm_i8p, grid, dim3(256), 0, c->stream, Y, P, redo, Xp, Xm, Wp, Wm,
                           T, N, steps, spb, max(1, c->cu_count / 8));
    } else if (vec) {
        hipLaunchKernelGGL((k_gemm_i8<true>), grid, dim3(256), 0, c->stream, Y, P, redo, W, X, T,
                           N, K, spb);
    } else {
        hipLaunchKernelGGL((k_gemm_i8<false>), grid, dim3(256), 0, c->stream, Y, P, redo, W, X,
                           T, N, K, spb);
    }
    if (vec)
        hipLaunchKernelGGL((k_gemm_i8_full<true>), dim3(fgrid), dim3(256), 0, c->stream, Y, P,
                           redo, W, X, T, N, K, spb, nb, S);
    else
        hipLaunchKernelGGL((k_gemm_i8_full<false>), dim3(fgrid), dim3(256), 0, c->stream, Y, P,
                           redo, W, X, T, N, K, spb, nb, S);
    if (S > 1) {
        const size_t tn = (size_t)T * N;
        hipLaunchKernelGGL(k_gemm_i8_reduce, dim3((unsigned)((tn + 255) / 256)), dim3(256), 0,
                           c->stream, Y, P, T, N, S);
    }
    return (int)hipGetLastError();
}
