// q48_gemm.hip — token-batched Q16.48 GEMM on the int8 matrix cores (gfx950).
//
// Y[t][n] = (int64)((sum_k (int128)X[t][k] * W[n][k]) >> 48), per output
// exactly matmul_vec (llama_int.c:1014-1046) applied to each token row.
//
// Digits.  Every int64 v is written v = S(v) + C with C = 0x0080808080808080
// and S(v) = sum_i s_i 256^i, s_i the bytes of v ^ C read as int8 (bytes 0..6
// are offset by 128, byte 7 is v's own signed top byte).  Then
//   sum_k W X = sum_{a,b} 256^(a+b) P_ab + C sum_k S(W) + C sum_k S(X) + K C^2,
//   P_ab = sum_k s_a(X_k) s_b(W_k),
// an exact integer identity over any k range; sum_k S(v) is the digit sums
// sum_a 256^a sum_k s_a(v_k), counted with v_dot4_i32_i8 while the tiles are
// split, so W and X are read once.  Only bits [48,112) are observable,
// so the pair a = b = 7 (weight 2^112) is dropped and the remaining 63 int8
// products are grouped by d = a + b into 14 int32 accumulators
// Q_d = sum_{a+b=d} P_ab; |Q_d| <= 8 * 2^14 * K < 2^31 while K < 16384 per
// accumulation run (longer K is split across blocks and summed in int128).
//
// Block: 4 waves, 64 tokens x 64 rows; wave w owns 32 tokens x 32 rows as 14
// v_mfma_i32_32x32x32_i8 accumulators (224 registers, one wave per SIMD).
// Per k-step of 32 elements the block splits the int64 tiles into eight byte
// planes in LDS (double-buffered) and every wave issues 63 MFMAs; the global
// loads run two steps ahead and the byte split of the next step is
// interleaved with the MFMAs of the current one.
#include "q48_digits.hpp"
#include "../../include/intllm_hip.h"

namespace {

constexpr int MT = 64;             // tokens per block
constexpr int MN = 64;             // rows per block
constexpr int MK = 32;             // k per step: one MFMA depth
constexpr int MAXK_RUN = 16320;    // k per accumulation run: |Q_d| < 2^31
constexpr int FUSE_BELOW_T = 1024; // token counts that count digit sums in the GEMM
constexpr int NPAIR = MK / 32;     // (row, 8 elements) pieces per thread per operand
constexpr int CH = MK / 16;        // 16-byte k chunks per row and limb

// Byte planes of one stage: [limb][32-row slice][k chunk][32 rows][16 bytes].
// The 64 lanes of an MFMA operand read (row l % 32, chunk 2h + l / 32) touch
// 1 KiB of consecutive bytes, and the 32 lanes of a half-wave store 256
// consecutive bytes: no bank conflicts either way.
constexpr int SLICE = CH * 512;    // one 32-row slice of one limb
constexpr int PLANE = 2 * SLICE;   // 64 rows of one limb
constexpr int STAGE = 8 * PLANE;   // one operand: 32 KiB

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

// Eight consecutive int64 of one row -> eight 8-byte digit words, limb a of
// element e in byte e of word a, stored at plane a.  sum[a] += ones-weighted
// sum of the eight limb-a digits (v_dot4_i32_i8; ones = 0x01010101 or 0).
template <bool FUSE>
__device__ __forceinline__ void split_store(uint8_t *stage, int off, const uint64_t (&v)[8],
                                            int (&sum)[8], int ones)
{
    uint32_t l0[4], l1[4], h0[4], h1[4];
    tr4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3], l0);
    tr4((uint32_t)v[4], (uint32_t)v[5], (uint32_t)v[6], (uint32_t)v[7], l1);
    tr4((uint32_t)(v[0] >> 32), (uint32_t)(v[1] >> 32), (uint32_t)(v[2] >> 32),
        (uint32_t)(v[3] >> 32), h0);
    tr4((uint32_t)(v[4] >> 32), (uint32_t)(v[5] >> 32), (uint32_t)(v[6] >> 32),
        (uint32_t)(v[7] >> 32), h1);
    uint8_t *p = stage + off;
    uint2 d[8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
        d[a] = make_uint2(l0[a] ^ 0x80808080u, l1[a] ^ 0x80808080u);
#pragma unroll
    for (int a = 0; a < 3; ++a)
        d[4 + a] = make_uint2(h0[a] ^ 0x80808080u, h1[a] ^ 0x80808080u);
    d[7] = make_uint2(h0[3], h1[3]);
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        *reinterpret_cast<uint2 *>(p + a * PLANE) = d[a];
        if (FUSE) {
            sum[a] = __builtin_amdgcn_sdot4((int)d[a].x, ones, sum[a], false);
            sum[a] = __builtin_amdgcn_sdot4((int)d[a].y, ones, sum[a], false);
        }
    }
}

// Eight elements [k, k + 8) of a row; positions at or past kend read as C
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
                                           : kDig;
    }
}

// One step: for each 32-deep half, the 8 + 8 operand limbs and 63 MFMAs.
__device__ __forceinline__ void mfma_step(v16i (&acc)[14], const uint8_t *xs,
                                          const uint8_t *ws, int lane)
{
#pragma unroll
    for (int h = 0; h < MK / 32; ++h) {
        const int off = (2 * h + (lane >> 5)) * 512 + (lane & 31) * 16;
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
                    acc[a + b] =
                        __builtin_amdgcn_mfma_i32_32x32x32_i8(A[a], B[b], acc[a + b], 0, 0, 0);
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

// grid (ceil(N/64) * ceil(T/64), 1, S): split z covers k-steps [z*spb, (z+1)*spb).
// FUSE: every block adds the digit corrections of its own k range (the digit
// sums of its rows, counted while splitting them, and its length times C^2).
// Otherwise cw[n] = C sum_k W - K C^2 and cx[t] = C sum_k X come from
// k_digit_corr and are added once: here when S == 1, else by the reduction.
// S == 1: Y gets the shifted result;
// S > 1: P[z][t][n] gets the block's int128 partial sum (two uint64, lo first).
template <bool VEC, bool FUSE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void
k_gemm_i8(int64_t *__restrict__ Y, uint64_t *__restrict__ P, const int64_t *__restrict__ W,
          const int64_t *__restrict__ X, const uint64_t *__restrict__ cw,
          const uint64_t *__restrict__ cx, int T, int N, int K, int spb)
{
    __shared__ __align__(16) uint8_t lds[2][2][STAGE];   // [stage][X, W]
    __shared__ int dsum[2][64][8];                        // [X, W][row][limb] digit sums
    __shared__ q48_u128 corr[2][64];                      // [X, W][row] corrections
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int n_tile, t_tile;
    tile_of(blockIdx.x, (N + MN - 1) / MN, (T + MT - 1) / MT, n_tile, t_tile);
    const int n0 = n_tile * MN, t0 = t_tile * MT;
    const int kbeg = blockIdx.z * spb * MK;
    const int kend = max(kbeg, min(K, kbeg + spb * MK));
    const int nfull = (kend - kbeg) / MK;
    const bool tail = (kend - kbeg) % MK != 0;

    // loader role: pieces tid and tid + 256 of both tiles
    Piece pc[NPAIR];
    const int64_t *xrow[NPAIR], *wrow[NPAIR];
#pragma unroll
    for (int j = 0; j < NPAIR; ++j) {
        pc[j] = piece(tid + 256 * j);
        xrow[j] = X + (size_t)min(t0 + pc[j].r, T - 1) * K + pc[j].k8;
        wrow[j] = W + (size_t)min(n0 + pc[j].r, N - 1) * K + pc[j].k8;
    }

    v16i acc[14];
#pragma unroll
    for (int d = 0; d < 14; ++d)
        acc[d] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = tid; i < 2 * 64 * 8; i += 256)
        (&dsum[0][0][0])[i] = 0;
    int sx[NPAIR][8], sw[NPAIR][8];
#pragma unroll
    for (int j = 0; j < NPAIR; ++j)
#pragma unroll
        for (int a = 0; a < 8; ++a)
            sx[j][a] = sw[j][a] = 0;
    constexpr int ONES = 0x01010101;

    const int wt = w >> 1, wn = w & 1;   // wave's token slice, row slice
    typedef uint64_t Regs[NPAIR][8];
    auto load = [&](Regs &gx, Regs &gw, int k) {
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
            load8<VEC, false>(gx[j], xrow[j], k, kend);
            load8<VEC, false>(gw[j], wrow[j], k, kend);
        }
    };
    auto store = [&](int st, const Regs &gx, const Regs &gw, int ones) {
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
            split_store<FUSE>(lds[st][0], pc[j].off, gx[j], sx[j], ones);
            split_store<FUSE>(lds[st][1], pc[j].off, gw[j], sw[j], ones);
        }
    };
    // Steps go two ahead: step s multiplies stage s & 1, splits step s + 1
    // (loaded during step s - 1) into the other stage and loads step s + 2.
    // Register sets alternate: step s loads into set s & 1.
    Regs gx0, gw0, gx1, gw1;
    const int last = max(nfull - 1, 0);
    if (nfull > 0) {
        load(gx0, gw0, kbeg);
        load(gx1, gw1, kbeg + min(1, last) * MK);
        store(0, gx0, gw0, ONES);
    }
    __syncthreads();
    auto step = [&](int s, Regs &lx, Regs &lw, const Regs &cx_, const Regs &cw_) {
        // step s + 2's tiles (clamped to the last step: in bounds, unused)
        load(lx, lw, kbeg + min(s + 2, last) * MK);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *st = &lds[s & 1][0][0];
        mfma_step(acc, st + wt * SLICE, st + STAGE + wn * SLICE, lane);
        // the last step splits a clamped re-read: stored, never used, not summed
        store((s + 1) & 1, cx_, cw_, s + 1 < nfull ? ONES : 0);
        // operand reads first, then the MFMAs with the digit split of the
        // next step interleaved (its data arrived a step ago)
#pragma unroll
        for (int h = 0; h < MK / 32; ++h) {
            __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
            for (int i = 0; i < 63; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2 / (MK / 32), 0);
            }
        }
        __syncthreads();
    };
    // pairs with no branch inside, so the loads stay where they are issued
    int s = 0;
    for (; s + 1 < nfull; s += 2) {
        step(s, gx0, gw0, gx1, gw1);
        step(s + 1, gx1, gw1, gx0, gw0);
    }
    if (s < nfull)
        step(s, gx0, gw0, gx1, gw1);
    if (tail) {
        const int kt = kbeg + nfull * MK;
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
            load8<VEC, true>(gx0[j], xrow[j], kt, kend - pc[j].k8);
            load8<VEC, true>(gw0[j], wrow[j], kt, kend - pc[j].k8);
        }
        store(nfull & 1, gx0, gw0, ONES);
        __syncthreads();
        const uint8_t *st = &lds[nfull & 1][0][0];
        mfma_step(acc, st + wt * SLICE, st + STAGE + wn * SLICE, lane);
    }

    // Digit corrections of this k range: per row, C * sum_k S(v) =
    // C * sum_a 256^a (digit sum of limb a); W rows also carry len * C^2.
    if (FUSE) {
#pragma unroll
        for (int j = 0; j < NPAIR; ++j)
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                atomicAdd(&dsum[0][pc[j].r][a], sx[j][a]);
                atomicAdd(&dsum[1][pc[j].r][a], sw[j][a]);
            }
    }
    __syncthreads();
    if (FUSE && tid < 128) {
        const int op = tid >> 6, row = tid & 63;
        q48_u128 sum = 0;
#pragma unroll
        for (int a = 7; a >= 0; --a)
            sum = (sum << 8) + (q48_u128)(q48_i128)dsum[op][row][a];
        q48_u128 v = sum * kDig;
        if (op == 1)
            v += (q48_u128)kDig * kDig * (q48_u128)(uint64_t)(kend - kbeg);
        corr[op][row] = v;
    }
    __syncthreads();

    // lane l, register i: token 8 (i / 4) + 4 (l / 32) + i % 4, row l % 32
    const int nl = 32 * wn + (lane & 31), n = n0 + nl;
    if (n >= N)
        return;
    q48_u128 cwn = 0;
    if (FUSE)
        cwn = corr[1][nl];
    else if (gridDim.z == 1)
        cwn = ((q48_u128)cw[2 * n + 1] << 64) | cw[2 * n];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int tl = 32 * wt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3), t = t0 + tl;
        if (t >= T)
            continue;
        q48_u128 tot = 0;
#pragma unroll
        for (int d = 13; d >= 0; --d)
            tot = (tot << 8) + (q48_u128)(q48_i128)acc[d][i];
        if (FUSE)
            tot += cwn + corr[0][tl];
        else if (gridDim.z == 1)
            tot += cwn + (((q48_u128)cx[2 * t + 1] << 64) | cx[2 * t]);
        if (gridDim.z == 1) {
            Y[(size_t)t * N + n] = (int64_t)((q48_i128)tot >> 48);
        } else {
            uint64_t *p = P + 2 * (((size_t)blockIdx.z * T + t) * N + n);
            *reinterpret_cast<ulonglong2 *>(p) = make_ulonglong2((uint64_t)tot,
                                                                 (uint64_t)(tot >> 64));
        }
    }
}

// Y[t][n] = (sum_z P[z][t][n] (+ cw[n] + cx[t] when given)) >> 48
__global__ __launch_bounds__(256) void k_gemm_i8_reduce(int64_t *__restrict__ Y,
                                                       const uint64_t *__restrict__ P,
                                                       const uint64_t *__restrict__ cw,
                                                       const uint64_t *__restrict__ cx,
                                                       int T, int N, int S)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * N)
        return;
    q48_u128 tot = 0;
    if (cw) {
        const int t = (int)(i / N), n = (int)(i % N);
        tot = (((q48_u128)cw[2 * n + 1] << 64) | cw[2 * n]) +
              (((q48_u128)cx[2 * t + 1] << 64) | cx[2 * t]);
    }
    for (int z = 0; z < S; ++z) {
        const ulonglong2 u =
            *reinterpret_cast<const ulonglong2 *>(P + 2 * ((size_t)z * T * N + i));
        tot += ((q48_u128)u.y << 64) | u.x;
    }
    Y[i] = (int64_t)((q48_i128)tot >> 48);
}

// out[row] = C * sum_k A[row][k] (exact int128, mod 2^128), minus K C^2 when
// sub_kc2: the digit corrections of the identity above.  One wave per row.
__global__ __launch_bounds__(256) void k_digit_corr(uint64_t *__restrict__ out,
                                                   const int64_t *__restrict__ A, int rows,
                                                   int K, int sub_kc2)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const int64_t *p = A + (size_t)row * K;
    q48_i128 s = 0;
    for (int k = lane; k < K; k += 64)
        s += p[k];
    s = (q48_i128)q48_wave_sum128((q48_u128)s);
    if (lane == 0) {
        q48_u128 v = (q48_u128)s * kDig;
        if (sub_kc2)
            v -= (q48_u128)kDig * kDig * (q48_u128)(uint64_t)K;
        out[2 * row] = (uint64_t)v;
        out[2 * row + 1] = (uint64_t)(v >> 64);
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

int q48_launch_gemm_i8(q48_ctx *c, int64_t *Y, const int64_t *W, const int64_t *X, int T,
                       int N, int K)
{
    const int S = q48_gemm_i8_splits(T, N, K, c->cu_count);
    const int steps = (K + MK - 1) / MK;
    const int spb = (steps + S - 1) / S;
    // short token counts count the digit sums inside the GEMM (W is read
    // once); long ones amortise a separate pass over W and X, which keeps
    // 32 v_dot4 per step out of the MFMA loop
    const bool fuse = T < FUSE_BELOW_T;
    const size_t corr = fuse ? 0 : 16 * ((size_t)N + (size_t)T);
    const size_t part = S > 1 ? 16 * (size_t)S * T * N : 0;
    uint64_t *cw = nullptr, *cx = nullptr, *P = nullptr;
    if (corr + part) {
        int rc = q48_ws_reserve(c, corr + part);
        if (rc)
            return rc;
        uint64_t *ws = (uint64_t *)c->ws;
        if (!fuse) {
            cw = ws;
            cx = cw + 2 * (size_t)N;
            ws = cx + 2 * (size_t)T;
        }
        if (S > 1)
            P = ws;
        if (!fuse) {
            hipLaunchKernelGGL(k_digit_corr, dim3((N + 3) / 4), dim3(256), 0, c->stream, cw, W,
                               N, K, 1);
            hipLaunchKernelGGL(k_digit_corr, dim3((T + 3) / 4), dim3(256), 0, c->stream, cx, X,
                               T, K, 0);
        }
    }
    const dim3 grid(((N + MN - 1) / MN) * ((T + MT - 1) / MT), 1, S);
    const bool vec = K % 2 == 0 && (((uintptr_t)W | (uintptr_t)X) & 15) == 0;
#define GEMM_I8_LAUNCH(V, F)                                                                 \
    hipLaunchKernelGGL((k_gemm_i8<V, F>), grid, dim3(256), 0, c->stream, Y, P, W, X, cw, cx, T, \
                       N, K, spb)
    if (vec && fuse)
        GEMM_I8_LAUNCH(true, true);
    else if (vec)
        GEMM_I8_LAUNCH(true, false);
    else if (fuse)
        GEMM_I8_LAUNCH(false, true);
    else
        GEMM_I8_LAUNCH(false, false);
#undef GEMM_I8_LAUNCH
    if (S > 1) {
        const size_t tn = (size_t)T * N;
        hipLaunchKernelGGL(k_gemm_i8_reduce, dim3((unsigned)((tn + 255) / 256)), dim3(256), 0,
                           c->stream, Y, P, cw, cx, T, N, S);
    }
    return (int)hipGetLastError();
}
