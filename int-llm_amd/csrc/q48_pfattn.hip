// q48_pfattn.hip — causal attention of a batched prefill on the int8 matrix
// cores: T query rows at positions p0 .. p0 + T - 1, row t over the cache rows
// 0 .. p0 + t, each row bit-identical to the reference's exact attention path
// at its position (llama_int.c:1502-1529 with softmax, 1060-1072).
//
// Scores.  s_j = fp_mul((sum_d q_d k_j,d) >> 48, scale): the int128 dot
//   product from the digit identity over d (q48_digits.hpp), 63
//   v_mfma_i32_16x16x64_i8 per 16 x 16 tile and 64 dims.
// Weights.  The softmax on the VALU: exact maximum, fp_safe_exp of the
//   wrapped difference, wrapping sum, fp_div when the sum is positive.
// Values.  o_d = sum_j fp_mul(p_j, v_j,d) truncates every product.  With
//   X_d = sum_j p_j v_j,d from the digit identity over j and Λ_d = sum_j t_j,d
//   the 24-bit limb term of trunc_low_acc, o_d = (X_d - 2^24 Λ_d) >> 48: the
//   MFMA digit products plus six full-rate VALU instructions per (row,
//   position, dim) instead of a 64 x 64 -> 128 product each.
//
// A block owns 16 consecutive query rows of one head.  k_pfa_prep first
// writes the layer's keys and values as digit planes once per KV head; the
// scores go to a workspace region of the block (16 rows x its position span)
// and are overwritten by the exponentials.
#include "q48_digits.hpp"

namespace {

constexpr int PF_ROWS = 16;   // query rows per block: one MFMA tile
constexpr int PF_STEP = 64;   // positions per value step: one MFMA depth

// Accumulation runs stay below 16320 positions: |digit-product sum| < 2^31.
constexpr int PF_MAX_POS = 16320;

__host__ __device__ inline int pf_round64(int x) { return (x + 63) & ~63; }

// positions the block of rows [16 tile, 16 tile + 16) reads, rounded up to 64
__host__ __device__ inline int pf_span(int tile, int p0, int T)
{
    const int end = PF_ROWS * (tile + 1) < T ? PF_ROWS * (tile + 1) : T;
    return pf_round64(p0 + end);
}

__device__ __forceinline__ int64_t row16_max64(int64_t v)
{
    int64_t o = (int64_t)q48_dpp64<Q48_DPP_XOR1>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_XOR2>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_HALF_MIRROR>((uint64_t)v);
    v = o > v ? o : v;
    o = (int64_t)q48_dpp64<Q48_DPP_MIRROR>((uint64_t)v);
    return o > v ? o : v;
}

__device__ __forceinline__ q48_u128 ld128(const uint64_t *p)
{
    return ((q48_u128)p[1] << 64) | p[0];
}

__device__ __forceinline__ void st128(uint64_t *p, q48_u128 v)
{
    p[0] = (uint64_t)v;
    p[1] = (uint64_t)(v >> 64);
}

// Digit planes of the layer's keys and values at positions [64 c, 64 c + 64)
// of KV head kh (grid (Ppad / 64, n_kv)); positions at or past P read as C
// (all digits zero):
//  KD[kh][a][j][HDP]   digit a of k_j,d (HDP: head_dim rounded up to 64, the
//                      pad dims zero digits)
//  VD[kh][a][d][Ppad]  digit a of v_j,d
//  CK[kh][j]           C sum_d k_j,d - hd C^2
//  VS[kh][c][d]        sum of v_j,d over the 64 positions of c
//  VL[kh][j][d]        low_limbs(v_j,d) (0 past P)
// (int128 values as two words, low first).
template <int HD>
__global__ __launch_bounds__(256) void k_pfa_prep(uint8_t *__restrict__ KD,
                                                 uint8_t *__restrict__ VD,
                                                 uint64_t *__restrict__ CK,
                                                 uint64_t *__restrict__ VS,
                                                 uint2 *__restrict__ VL,
                                                 const int64_t *__restrict__ kcache,
                                                 const int64_t *__restrict__ vcache, int layer,
                                                 int P, int Ppad, int n_kv, int max_seq)
{
    constexpr int HDP = HD < 64 ? 64 : HD;
    const int c = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, j0 = PF_STEP * c;
    const size_t kvd = (size_t)n_kv * HD;
    const int64_t *kb = kcache + (size_t)layer * max_seq * kvd + (size_t)kh * HD;
    const int64_t *vb = vcache + (size_t)layer * max_seq * kvd + (size_t)kh * HD;
    uint8_t *kd = KD + (size_t)kh * 8 * Ppad * HDP;
    uint8_t *vd = VD + (size_t)kh * 8 * HD * Ppad;
    uint2 *vl = VL + (size_t)kh * Ppad * HD;

    // keys: (position, 4 dims) per item
    for (int it = tid; it < PF_STEP * (HDP / 4); it += 256) {
        const int j = j0 + it / (HDP / 4), d = 4 * (it % (HDP / 4));
        uint64_t v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[e] = (j < P && d + e < HD) ? (uint64_t)kb[(size_t)j * kvd + d + e] : kDig;
        uint32_t w[8];
        digits4(v, w);
#pragma unroll
        for (int a = 0; a < 8; ++a)
            *reinterpret_cast<uint32_t *>(kd + ((size_t)a * Ppad + j) * HDP + d) = w[a];
    }
    // values: (dim, 4 positions) per item, the dims of a wave consecutive
    for (int it = tid; it < HD * (PF_STEP / 4); it += 256) {
        const int d = it % HD, j = j0 + 4 * (it / HD);
        uint64_t v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[e] = j + e < P ? (uint64_t)vb[(size_t)(j + e) * kvd + d] : kDig;
        uint32_t w[8];
        digits4(v, w);
#pragma unroll
        for (int a = 0; a < 8; ++a)
            *reinterpret_cast<uint32_t *>(vd + ((size_t)a * HD + d) * Ppad + j) = w[a];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            vl[(size_t)(j + e) * HD + d] = j + e < P ? low_limbs(v[e]) : make_uint2(0, 0);
    }
    if (tid < PF_STEP) {
        const int j = j0 + tid;
        q48_u128 s = 0;
        if (j < P) {
            for (int d = 0; d < HD; ++d)
                s += (q48_u128)(q48_i128)kb[(size_t)j * kvd + d];
            s = s * kDig - (q48_u128)kDig * kDig * (q48_u128)HD;
        }
        st128(CK + 2 * ((size_t)kh * Ppad + j), s);
    } else if (tid < PF_STEP + HD) {
        const int d = tid - PF_STEP;
        q48_u128 s = 0;
        for (int j = j0; j < j0 + PF_STEP; ++j)
            s += j < P ? (q48_u128)(q48_i128)vb[(size_t)j * kvd + d] : (q48_u128)kDig;
        st128(VS + 2 * (((size_t)kh * (Ppad / PF_STEP) + c) * HD + d), s);
    }
}

// Attention of 16 query rows of one head.  Blocks go round-robin to the 8
// XCDs; when n_kv divides 8, XCD x takes KV head x % n_kv only, so each L2
// holds the digit planes of one KV head.  Within an XCD the longest row
// blocks (the last rows) start first.
//  phase 1: scores by MFMA (wave w: position tiles w, w + 4, ...), written to
//           the block's workspace rows, and the row maxima;
//  phase 2: exponentials in place and the row sums;
//  phase 3: per 64 positions, the weights p (fp_div) as digits and limbs in
//           LDS, the values' limbs in LDS; X by MFMA (wave w: dims 16 w ..),
//           Λ on the VALU (wave w: rows 4 w ..);
//  then o = (X - 2^24 Λ) >> 48.
template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 128 ? 1 : 2))) void
k_pfa(int64_t *__restrict__ out,
                                            const int64_t *__restrict__ QKV,
                                            const uint8_t *__restrict__ KD,
                                            const uint8_t *__restrict__ VD,
                                            const uint64_t *__restrict__ CK,
                                            const uint64_t *__restrict__ VS,
                                            const uint2 *__restrict__ VL,
                                            int64_t *__restrict__ SCR,
                                            const int64_t *__restrict__ scale_p, int p0, int T,
                                            int n_heads, int n_kv, int Ppad, size_t per_head)
{
    constexpr int HDP = HD < 64 ? 64 : HD, KS = HDP / 64;
    constexpr int NDT = HD / 16, DTW = (NDT + 3) / 4;   // 16-dim tiles, per wave
    constexpr int DB = HD / 4, JG = 64 / DB, JPER = PF_STEP / JG;
    static_assert(DB * JG == 64 && HD % 16 == 0, "lane split");
    __shared__ __align__(16) uint8_t pd[8][PF_ROWS][PF_STEP];   // weight digits of a step
    __shared__ __align__(16) uint2 pl[PF_ROWS][PF_STEP];        // weight limbs of a step
    __shared__ __align__(16) uint2 vl[PF_STEP][HD];             // value limbs of a step
    __shared__ uint64_t lam[PF_ROWS][HD];
    __shared__ q48_u128 cq[PF_ROWS], cp[PF_ROWS], cv[HD];
    __shared__ int64_t mxs[4][PF_ROWS], sums[PF_ROWS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rl = lane & 15, kq = lane >> 4;
    const int G = n_heads / n_kv, nt = (T + PF_ROWS - 1) / PF_ROWS;
    int tile, h;
    if (8 % n_kv == 0) {
        const int x = (int)blockIdx.x & 7, item = ((int)blockIdx.x >> 3) * (8 / n_kv) + x / n_kv;
        if (item >= G * nt)
            return;   // uniform over the block
        tile = nt - 1 - item / G;
        h = (x % n_kv) * G + item % G;
    } else {
        if ((int)blockIdx.x >= n_heads * nt)
            return;
        tile = nt - 1 - (int)blockIdx.x / n_heads;
        h = (int)blockIdx.x % n_heads;
    }
    const int kh = h / G;
    const int t0 = PF_ROWS * tile, nrow = min(PF_ROWS, T - t0);
    const int J = pf_span(tile, p0, T);
    size_t off = 0;
    for (int i = 0; i < tile; ++i)
        off += (size_t)pf_span(i, p0, T);
    int64_t *sc = SCR + (size_t)h * per_head + (size_t)PF_ROWS * off;   // [16][J]
    const int64_t scale = *scale_p;

    // query digits: lane (row rl, dims 64 ks + 16 kq .. + 15), the A operand
    v4i A[KS][8];
    {
        const int64_t *q = QKV + (size_t)min(t0 + rl, T - 1) * ((size_t)(n_heads + 2 * n_kv) * HD) +
                           (size_t)h * HD;
        q48_u128 qs = 0;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 64 * ks + 16 * kq;
            uint64_t v[16];
            if (d0 < HD) {   // head_dim is a multiple of 16: all 16 dims real
                const ulonglong2 *q2 = reinterpret_cast<const ulonglong2 *>(q + d0);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const ulonglong2 u = q2[e];
                    v[2 * e] = u.x;
                    v[2 * e + 1] = u.y;
                }
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    qs += (q48_u128)(q48_i128)(int64_t)v[e];
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    v[e] = kDig;
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint64_t v4[4] = {v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
                uint32_t wd[8];
                digits4(v4, wd);
#pragma unroll
                for (int a = 0; a < 8; ++a)
                    A[ks][a][g] = (int)wd[a];
            }
        }
        qs += shfl_xor128(qs, 16);
        qs += shfl_xor128(qs, 32);
        if (w == 0 && kq == 0)
            cq[rl] = qs * kDig;
    }
    __syncthreads();

    // phase 1: lane holds position j0 + rl of rows 4 kq + i
    int64_t mx[4] = {INT64_MIN, INT64_MIN, INT64_MIN, INT64_MIN};
    {
        const uint8_t *kd = KD + (size_t)kh * 8 * Ppad * HDP;
        const uint64_t *ck = CK + 2 * (size_t)kh * Ppad;
        for (int jt = w; jt < J / 16; jt += 4) {
            const int j = 16 * jt + rl;
            v4i B[KS][8];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    B[ks][b] = *reinterpret_cast<const v4i *>(kd + ((size_t)b * Ppad + j) * HDP +
                                                              64 * ks + 16 * kq);
            v4i acc[14];
#pragma unroll
            for (int d = 0; d < 14; ++d)
                acc[d] = (v4i){0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int a = 0; a < 8; ++a)
#pragma unroll
                    for (int b = 0; b < 8; ++b)
                        if (a + b <= 13)
                            acc[a + b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                A[ks][a], B[ks][b], acc[a + b], 0, 0, 0);
            const q48_u128 ckj = ld128(ck + 2 * (size_t)j);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * kq + i;
                const q48_u128 tot = digits_total(acc, i) + cq[m] + ckj;
                const int64_t s = q48_mul((int64_t)(tot >> 48), scale);
                sc[(size_t)m * J + j] = s;
                if (m < nrow && j <= p0 + t0 + m)
                    mx[i] = s > mx[i] ? s : mx[i];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        mx[i] = row16_max64(mx[i]);
    if (rl == 0)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            mxs[w][4 * kq + i] = mx[i];
    __syncthreads();

    // phase 2: row r = tid / 16, positions tid % 16 + 16 k
    {
        const int r = tid >> 4, jj = tid & 15;
        int64_t sum = 0;
        if (r < nrow) {
            int64_t m = mxs[0][r];
#pragma unroll
            for (int u = 1; u < 4; ++u)
                m = mxs[u][r] > m ? mxs[u][r] : m;
            const int S = p0 + t0 + r + 1;
            int64_t *srow = sc + (size_t)r * J;
            auto ex = [&](int j) {
                const int64_t e = q48_safe_exp((int64_t)((uint64_t)srow[j] - (uint64_t)m));
                srow[j] = e;
                return e;
            };
            int j = jj;
            for (; j + 48 < S; j += 64) {
                const int64_t e0 = ex(j), e1 = ex(j + 16), e2 = ex(j + 32), e3 = ex(j + 48);
                sum = (int64_t)((uint64_t)sum + (uint64_t)e0 + (uint64_t)e1 + (uint64_t)e2 +
                                (uint64_t)e3);
            }
            for (; j < S; j += 16)
                sum = (int64_t)((uint64_t)sum + (uint64_t)ex(j));
        }
        sum = (int64_t)group_sum64<16>((uint64_t)sum);
        if (jj == 0)
            sums[r] = sum;
    }
    __syncthreads();

    // phase 3: per step of 64 positions the step's weights are in pd / pl and
    // its value limbs in vl.  Before the low-part loop each thread loads the
    // next step's exponentials and its wave's value digits of this step; after
    // the step's barrier the next value limbs go straight to LDS
    // (global_load_lds) while the next weights are divided.
    const int r3 = tid >> 4, q4 = tid & 15;
    const int S3 = p0 + t0 + r3 + 1;
    const bool rv = r3 < nrow;
    const int64_t den = sums[r3];
    const q48_divisor dvr = q48_divisor_of(den);
    const int db = lane / JG, jg = lane % JG;
    constexpr int FLUSH = 128 / JPER;   // steps between flushes of the 32-bit Λ sums (< 2^31)
    const uint8_t *vd = VD + (size_t)kh * 8 * HD * Ppad;
    const char *vlg = reinterpret_cast<const char *>(VL + (size_t)kh * Ppad * HD);
    q48_u128 psum = 0;
    uint64_t er[4] = {0, 0, 0, 0};
    auto load_e = [&](int j0) {
        if (rv) {
            const ulonglong2 *e2 =
                reinterpret_cast<const ulonglong2 *>(sc + (size_t)r3 * J + j0 + 4 * q4);
            const ulonglong2 u0 = e2[0], u1 = e2[1];
            er[0] = u0.x;
            er[1] = u0.y;
            er[2] = u1.x;
            er[3] = u1.y;
        }
    };
    // weights of row r3 at positions j0 + 4 q4 .. + 3 (0 past the row's position)
    auto weights = [&](int j0) {
        const int jb = j0 + 4 * q4;
        uint64_t p[4] = {0, 0, 0, 0};
        if (rv) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (jb + k < S3)
                    p[k] = (uint64_t)(den > 0 ? q48_div_by((int64_t)er[k], dvr) : (int64_t)er[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            psum += p[k];
        uint32_t wd[8];
        digits4(p, wd);
#pragma unroll
        for (int a = 0; a < 8; ++a)
            *reinterpret_cast<uint32_t *>(&pd[a][r3][4 * q4]) = wd[a];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            pl[r3][4 * q4 + k] = low_limbs(p[k]);
    };
    // value limbs of positions j0 .. j0 + 63: 512 HD contiguous bytes, 1 KiB
    // per wave and instruction
    auto load_vl = [&](int j0) {
        const char *src = vlg + (size_t)j0 * HD * sizeof(uint2) + 16 * tid;
        char *dst = reinterpret_cast<char *>(&vl[0][0]) + 1024 * w;
#pragma unroll
        for (int i = 0; i < HD / 8; ++i)
            __builtin_amdgcn_global_load_lds(src + 4096 * i, dst + 4096 * i, 16, 0, 0);
    };
    for (int i = tid; i < PF_ROWS * HD; i += 256)
        (&lam[0][0])[i] = 0;
    v4i accp[DTW][14];
#pragma unroll
    for (int u = 0; u < DTW; ++u)
#pragma unroll
        for (int d = 0; d < 14; ++d)
            accp[u][d] = (v4i){0, 0, 0, 0};
    uint32_t t32[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
            t32[i][cc] = 0;
    load_vl(0);
    load_e(0);
    weights(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int ns = J / PF_STEP;
    for (int st = 0; st < ns; ++st) {
        const int j0 = PF_STEP * st;
        if (st + 1 < ns)
            load_e(j0 + PF_STEP);
        v4i Bv[DTW][8];
#pragma unroll
        for (int u = 0; u < DTW; ++u)
            if (w + 4 * u < NDT)
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    Bv[u][b] = *reinterpret_cast<const v4i *>(
                        vd + ((size_t)b * HD + 16 * (w + 4 * u) + rl) * Ppad + j0 + 16 * kq);
        // Λ: rows 4 w .. 4 w + 3, dims 4 db .. 4 db + 3, positions j0 + jg + JG k
#pragma unroll 4
        for (int k = 0; k < JPER; ++k) {
            const int jl = jg + JG * k;
            uint2 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a[i] = pl[4 * w + i][jl];
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                b[cc] = vl[jl][4 * db + cc];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int cc = 0; cc < 4; ++cc)
                    t32[i][cc] = trunc_low_acc(a[i], b[cc], t32[i][cc]);
        }
        if ((st + 1) % FLUSH == 0 || st + 1 == ns) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    atomicAdd(reinterpret_cast<unsigned long long *>(&lam[4 * w + i][4 * db + cc]),
                              (unsigned long long)t32[i][cc]);
                    t32[i][cc] = 0;
                }
        }
        // X: the wave's 16-dim tiles
#pragma unroll
        for (int u = 0; u < DTW; ++u) {
            if (w + 4 * u < NDT) {
                v4i Ap[8];
#pragma unroll
                for (int a = 0; a < 8; ++a)
                    Ap[a] = *reinterpret_cast<const v4i *>(&pd[a][rl][16 * kq]);
#pragma unroll
                for (int a = 0; a < 8; ++a)
#pragma unroll
                    for (int b = 0; b < 8; ++b)
                        if (a + b <= 13)
                            accp[u][a + b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                Ap[a], Bv[u][b], accp[u][a + b], 0, 0, 0);
            }
        }
        __syncthreads();
        if (st + 1 < ns) {
            load_vl(j0 + PF_STEP);
            weights(j0 + PF_STEP);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }

    psum = q48_dpp128<Q48_DPP_XOR1>(psum) + psum;
    psum = q48_dpp128<Q48_DPP_XOR2>(psum) + psum;
    psum = q48_dpp128<Q48_DPP_HALF_MIRROR>(psum) + psum;
    psum = q48_dpp128<Q48_DPP_MIRROR>(psum) + psum;
    if (q4 == 0)
        cp[r3] = psum * kDig;
    if (tid < HD) {
        const uint64_t *vs = VS + 2 * ((size_t)kh * (Ppad / PF_STEP) * HD + tid);
        q48_u128 s = 0;
        for (int c = 0; c < J / PF_STEP; ++c)
            s += ld128(vs + 2 * (size_t)c * HD);
        cv[tid] = s * kDig - (q48_u128)kDig * kDig * (q48_u128)(uint64_t)J;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < DTW; ++u) {
        const int dt = w + 4 * u;
        if (dt < NDT) {
            const int d = 16 * dt + rl;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * kq + i;
                if (m < nrow) {
                    const q48_u128 X = digits_total(accp[u], i) + cp[m] + cv[d];
                    const q48_u128 o = X - ((q48_u128)lam[m][d] << 24);
                    out[(size_t)(t0 + m) * n_heads * HD + (size_t)h * HD + d] = (int64_t)(o >> 48);
                }
            }
        }
    }
}

} // namespace

bool q48_pf_attn_mfma_ok(int p0, int T, int hd)
{
    return (hd == 32 || hd == 64 || hd == 128) && T > 0 && p0 >= 0 && p0 + T <= PF_MAX_POS;
}

int q48_pf_attn_mfma_max_pos() { return PF_MAX_POS; }

int q48_launch_pf_attn_mfma(q48_ctx *c, int64_t *out, const int64_t *QKV, int64_t *kcache,
                            int64_t *vcache, int layer, int p0, int T, int n_heads, int n_kv,
                            int hd, int max_seq)
{
    const int P = p0 + T, Ppad = pf_round64(P), HDP = hd < 64 ? 64 : hd;
    const int nt = (T + PF_ROWS - 1) / PF_ROWS, G = n_heads / n_kv;
    size_t span = 0;
    for (int i = 0; i < nt; ++i)
        span += (size_t)pf_span(i, p0, T);
    const size_t per_head = PF_ROWS * span;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += (bytes + 255) & ~(size_t)255;
        return at;
    };
    const size_t o_kd = take((size_t)n_kv * 8 * Ppad * HDP);
    const size_t o_vd = take((size_t)n_kv * 8 * hd * Ppad);
    const size_t o_ck = take((size_t)n_kv * Ppad * 16);
    const size_t o_vs = take((size_t)n_kv * (Ppad / PF_STEP) * hd * 16);
    const size_t o_vl = take((size_t)n_kv * Ppad * hd * sizeof(uint2));
    const size_t o_sc = take((size_t)n_heads * per_head * sizeof(int64_t));
    int rc = q48_ws_reserve(c, o);
    if (rc)
        return rc;
    uint8_t *ws = (uint8_t *)c->ws;
    uint8_t *KD = ws + o_kd, *VD = ws + o_vd;
    uint64_t *CK = (uint64_t *)(ws + o_ck), *VS = (uint64_t *)(ws + o_vs);
    uint2 *VL = (uint2 *)(ws + o_vl);
    int64_t *SCR = (int64_t *)(ws + o_sc);
    const int64_t *scale_p = c->rope_sin + (size_t)c->rope_max_seq * (c->rope_head_dim / 2);
    const dim3 pgrid(Ppad / PF_STEP, n_kv);
    const unsigned grid = 8 % n_kv == 0
                              ? 8u * (unsigned)((G * nt + 8 / n_kv - 1) / (8 / n_kv))
                              : (unsigned)(n_heads * nt);
#define PFA_LAUNCH(HDV)                                                                       \
    do {                                                                                      \
        hipLaunchKernelGGL(k_pfa_prep<HDV>, pgrid, dim3(256), 0, c->stream, KD, VD, CK, VS,   \
                           VL, kcache, vcache, layer, P, Ppad, n_kv, max_seq);                \
        hipLaunchKernelGGL(k_pfa<HDV>, dim3(grid), dim3(256), 0, c->stream, out, QKV, KD, VD, \
                           CK, VS, VL, SCR, scale_p, p0, T, n_heads, n_kv, Ppad, per_head);   \
    } while (0)
    if (hd == 64)
        PFA_LAUNCH(64);
    else if (hd == 32)
        PFA_LAUNCH(32);
    else
        PFA_LAUNCH(128);
#undef PFA_LAUNCH
    return (int)hipGetLastError();
}
