// q48_attn.hpp — the exact decode attention of one query head as a device
// function (k_attn_v3's body), shared by the standalone attention kernel and
// the fused attention + output-projection kernel.  Included by the HIP
// sources of libintllm_hip only.
#pragma once

#include "q48_internal.h"

namespace {

// Sum an int64 (wrapping) across a block of NT threads; every thread gets it.
template <int NT>
__device__ __forceinline__ int64_t block_sum64(int64_t v, int64_t *red, bool reused = true)
{
    v = q48_wave_sum64(v);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (reused)   // red may still be read by a previous reduction
        __syncthreads();
    if (lane == 0)
        red[w] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i)
        t += (uint64_t)red[i];
    return (int64_t)t;
}

template <int NT>
__device__ __forceinline__ int64_t block_max64(int64_t v, int64_t *red, bool reused = true)
{
    v = q48_wave_max64(v);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (reused)
        __syncthreads();
    if (lane == 0)
        red[w] = v;
    __syncthreads();
    int64_t t = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i)
        t = red[i] > t ? red[i] : t;
    return t;
}

constexpr int ATT_LDS_MAX = 4096;   // positions whose scores fit in LDS (32 KiB)

// Attention v3 of query head h, run by threads 0..NT-1 of the block (NT =
// 256 or 512; threads past NT - 1 must not call it): RoPE of q_h and the new
// k, KV store at pos (by the first query head of each KV head), scores, max,
// fp_safe_exp, sum, fp_div, V (llama_int.c:997-1008, 1060-1072, 1392-1395,
// 1414-1416, 1502-1529).
//  - the K rows of the first two score passes are issued before RoPE, and
//    each later pass is issued one pass ahead (two register buffers), only
//    where it exists; a pass or V batch with no position below S is neither
//    scored nor used;
//  - the first V batches are issued before the softmax, later ones one
//    batch ahead where they exist, so the V pass rarely waits;
//  - the score scale fp_inv_sqrt(fp_from_int(hd)) is read, not recomputed
//    (k_rope_init stores it after the sine table).
// Loads past the last position are clamped to it (in bounds, unused).  Rows at pos
// are read from the cache and replaced by the block's own rotated k and v.
// HD = 32, 64 or 128; at most SMAX positions (scores in LDS).  COH: the
// output goes out with agent-coherent (write-through) stores, for a consumer
// on other compute units in the same kernel.  PRE (batched prefill): q_h is
// already rotated and the key and value at pos are already in the cache
// (k_new, v_new, cos_t, sin_t unused); the rest is the same arithmetic.
// CIN: q, k_new and v_new are read with agent-coherent loads (written earlier
// in the same kernel by other compute units, e.g. the persistent decode step).
// ROT (decode over the cache): like PRE (q_h rotated, k and v at pos already
// stored by the projection's epilogue), and q and the K rows of the first
// two passes (rows up to 2 NT / 8 - 1, clamped to max_seq - 1: in bounds
// whatever the position) go out before the device-resident position is
// read, so that its round trip overlaps theirs.
template <int HD, int SMAX, bool COH, bool PRE = false, bool CIN = false, int NT = 256,
          bool ROT = false>
__device__ __forceinline__ void attn_v3_head(
    int64_t *__restrict__ out, const int64_t *__restrict__ q, int64_t *__restrict__ kcache,
    int64_t *__restrict__ vcache, const int64_t *__restrict__ k_new,
    const int64_t *__restrict__ v_new, const int64_t *__restrict__ cos_t,
    const int64_t *__restrict__ sin_t, const int64_t *__restrict__ scale_p, int layer,
    const int *__restrict__ d_pos, int pos, int n_heads, int n_kv, int max_seq, int h)
{
    static_assert(NT == 256 || NT == 512, "attention block size");
    constexpr int DPL = HD / 8, DP2 = DPL / 2, SL = NT / HD, NG = NT / 8, VB = 8;
    __shared__ int64_t qs[HD], ks[HD], vs[HD];
    __shared__ int64_t red[NT / 64], red2[NT / 64];
    __shared__ int64_t part[NT];
    __shared__ int64_t sc[SMAX];
    if (!ROT) {
        if (d_pos)
            pos = *d_pos;
        if (pos < 0 || pos >= max_seq)
            return;   // uniform over the block: no barrier is skipped by part of it
    }
    const int tid = threadIdx.x;
    const int group = n_heads / n_kv, kh = h / group;
    const size_t kvd = (size_t)n_kv * HD;
    const size_t base = (size_t)layer * max_seq;
    int S = pos + 1;
    const int half = HD / 2;
    const int g = tid >> 3, l8 = tid & 7;
    const int64_t scale = *scale_p;

    const int64_t *kb0 = kcache + base * kvd + (size_t)kh * HD + l8 * DPL;
    auto krow = [&](int t) {
        return reinterpret_cast<const ulonglong2 *>(kb0 + (size_t)min(t, S - 1) * kvd);
    };
    ulonglong2 ka[DP2], kb[DP2];
    if constexpr (ROT) {
        const int j = min(tid, HD - 1);
        const int64_t qv = q[(size_t)h * HD + j];
        const auto *r0 = reinterpret_cast<const ulonglong2 *>(kb0 + (size_t)min(g, max_seq - 1) * kvd);
        const auto *r1 =
            reinterpret_cast<const ulonglong2 *>(kb0 + (size_t)min(g + NG, max_seq - 1) * kvd);
#pragma unroll
        for (int d = 0; d < DP2; ++d)
            ka[d] = r0[d];
#pragma unroll
        for (int d = 0; d < DP2; ++d)
            kb[d] = r1[d];
        // a scalar load (constant address space): no vector-memory wait,
        // which would cover the K rows, is needed for it
        typedef const __attribute__((address_space(4))) int cint;
        if (d_pos)
            pos = *(cint *)d_pos;
        if (pos < 0 || pos >= max_seq)
            return;   // uniform over the block: no barrier is skipped by part of it
        S = pos + 1;
        qs[j] = qv;
        __syncthreads();
    } else if constexpr (PRE) {
        const int j = min(tid, HD - 1);
        const int64_t qv = q[(size_t)h * HD + j];
        const int64_t kv = kcache[(base + pos) * kvd + (size_t)kh * HD + j];
        const int64_t vv = vcache[(base + pos) * kvd + (size_t)kh * HD + j];
#pragma unroll
        for (int d = 0; d < DP2; ++d)
            ka[d] = krow(g)[d];
#pragma unroll
        for (int d = 0; d < DP2; ++d)
            kb[d] = krow(g + NG)[d];
        qs[j] = qv;
        ks[j] = kv;
        vs[j] = vv;
        __syncthreads();
    } else {
        // the RoPE inputs and the new v first (loads retire in issue order: the
        // RoPE then waits for them alone), every thread loading (clamped index)
        const int64_t *qh = q + (size_t)h * HD, *kn = k_new + (size_t)kh * HD;
        const int i = min(tid, half - 1), j = min(tid, HD - 1);
        auto ld = [](const int64_t *p) {
            if constexpr (CIN)
                return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                return *p;
        };
        int64_t c = cos_t[(size_t)pos * half + i];
        int64_t sn = sin_t[(size_t)pos * half + i];
        int64_t q0 = ld(qh + i), q1 = ld(qh + i + half);
        int64_t k0 = ld(kn + i), k1 = ld(kn + i + half);
        int64_t vn = ld(v_new + (size_t)kh * HD + j);
        __builtin_amdgcn_sched_barrier(0);

        // K rows of passes 0 and 1: lane l8 of group g holds dims [l8 DPL, +DPL)
#pragma unroll
        for (int d = 0; d < DP2; ++d)
            ka[d] = krow(g)[d];
#pragma unroll
        for (int d = 0; d < DP2; ++d)
            kb[d] = krow(g + NG)[d];
        __builtin_amdgcn_sched_barrier(0);
        // first use of the RoPE inputs here, after the K loads are out (else the
        // compiler extends them to 128 bits, and waits for them, earlier)
        asm volatile("" : "+v"(c), "+v"(sn), "+v"(q0), "+v"(q1), "+v"(k0), "+v"(k1), "+v"(vn));

        // RoPE of q_h and the new k (rope_apply, llama_int.c:997-1008, 1392-1395);
        // threads past half repeat the last pair (same values, same slots): no
        // branch, so the loads above are not sunk into one
        qs[i] = (int64_t)((uint64_t)q48_mul(q0, c) - (uint64_t)q48_mul(q1, sn));
        qs[i + half] = (int64_t)((uint64_t)q48_mul(q1, c) + (uint64_t)q48_mul(q0, sn));
        ks[i] = (int64_t)((uint64_t)q48_mul(k0, c) - (uint64_t)q48_mul(k1, sn));
        ks[i + half] = (int64_t)((uint64_t)q48_mul(k1, c) + (uint64_t)q48_mul(k0, sn));
        vs[j] = vn;
        __syncthreads();
        if (h % group == 0 && tid < HD) {
            kcache[(base + pos) * kvd + (size_t)kh * HD + tid] = ks[tid];
            vcache[(base + pos) * kvd + (size_t)kh * HD + tid] = vs[tid];
        }
    }

    // scores s_t = fp_mul((sum_d q_d k_t,d) >> 48, scale), llama_int.c:1502-1512
    const int64_t *qd = qs + l8 * DPL, *kd = ks + l8 * DPL;
    int64_t mx = INT64_MIN;
    auto score = [&](const ulonglong2 (&kr)[DP2], int t) {
        const bool own = !ROT && t == pos;
        q48_u128 dot = 0;
#pragma unroll
        for (int d = 0; d < DP2; ++d) {
            const int64_t a0 = own ? kd[2 * d] : (int64_t)kr[d].x;
            const int64_t a1 = own ? kd[2 * d + 1] : (int64_t)kr[d].y;
            dot += (q48_u128)q48_smul128(qd[2 * d], a0);
            dot += (q48_u128)q48_smul128(qd[2 * d + 1], a1);
        }
        dot = q48_sum8_u128(dot);
        if (t < S && l8 == 0) {
            const int64_t s = q48_mul((int64_t)((q48_i128)dot >> 48), scale);
            sc[t] = s;
            mx = s > mx ? s : mx;
        }
    };
    for (int t0 = 0; t0 < S; t0 += 2 * NG) {
        // the next passes' rows, where there is a next pass (a block-uniform
        // test: unneeded reloads would hold the compute unit's load return
        // path, and the wave, until they landed)
        score(ka, t0 + g);
        if (t0 + 2 * NG < S) {
#pragma unroll
            for (int d = 0; d < DP2; ++d)
                ka[d] = krow(t0 + 2 * NG + g)[d];
        }
        if (t0 + NG < S)
            score(kb, t0 + NG + g);
        if (t0 + 3 * NG < S) {
#pragma unroll
            for (int d = 0; d < DP2; ++d)
                kb[d] = krow(t0 + 3 * NG + g)[d];
        }
    }

    // V batches 0 and 1 go out before the softmax: thread (d, sl) takes
    // positions sl + SL i, VB of them per batch
    const int d = tid % HD, sl = tid / HD;
    const int64_t *vcol = vcache + base * kvd + (size_t)kh * HD + d;
    auto vld = [&](int i) { return vcol[(size_t)min(sl + SL * i, S - 1) * kvd]; };
    int64_t va[VB], vb[VB];
#pragma unroll
    for (int u = 0; u < VB; ++u)
        va[u] = vld(u);
#pragma unroll
    for (int u = 0; u < VB; ++u)
        vb[u] = vld(VB + u);

    // softmax, llama_int.c:1060-1072
    // each reduction has its own slots, used once: no barrier before the
    // slot writes (the one after them also orders the score stores)
    mx = block_max64<NT>(mx, red, false);
    int64_t sum = 0;
    for (int t = tid; t < S; t += NT) {
        const int64_t e = q48_safe_exp((int64_t)((uint64_t)sc[t] - (uint64_t)mx));
        sc[t] = e;
        sum = (int64_t)((uint64_t)sum + (uint64_t)e);
    }
    sum = block_sum64<NT>(sum, red2, false);
    // the weights are never negative (exponentials over a positive sum, or
    // the exponentials themselves); checked, and the values take the product
    // for non-negative weights (q48_pv_mac) unless one is
    int neg = 0;
    const q48_divisor dv = q48_divisor_of(sum);
    for (int t = tid; t < S; t += NT) {
        if (sum > 0)
            sc[t] = q48_div_by(sc[t], dv);
        neg |= sc[t] < 0;
    }
    neg = __syncthreads_or(neg);

    // o[d] = sum_t fp_mul(p_t, v_t[d]), llama_int.c:1514-1529; one copy of
    // the loop per product form, chosen once for the block
    auto values = [&](auto nonneg) -> uint64_t {
        uint64_t acc = 0;
        q48_pv_acc pa = {0, 0};
        auto vmac = [&](const int64_t(&vv)[VB], int i0) {
#pragma unroll
            for (int u = 0; u < VB; ++u) {
                const int t = sl + SL * (i0 + u);
                if (t < S) {
                    const int64_t v = !ROT && t == pos ? vs[d] : vv[u];
                    if constexpr (decltype(nonneg)::value)
                        q48_pv_mac(pa, sc[t], v);
                    else
                        acc += (uint64_t)q48_mul(sc[t], v);
                }
            }
        };
        for (int i0 = 0; sl + SL * i0 < S; i0 += 2 * VB) {
            // the next batches where some position of them exists (as above)
            vmac(va, i0);
            if (SL * (i0 + 2 * VB) < S) {
#pragma unroll
                for (int u = 0; u < VB; ++u)
                    va[u] = vld(i0 + 2 * VB + u);
            }
            if (SL * (i0 + VB) < S)
                vmac(vb, i0 + VB);
            if (SL * (i0 + 3 * VB) < S) {
#pragma unroll
                for (int u = 0; u < VB; ++u)
                    vb[u] = vld(i0 + 3 * VB + u);
            }
        }
        return acc + (uint64_t)q48_pv_total(pa);
    };
    const uint64_t acc = neg ? values(std::false_type{}) : values(std::true_type{});
    part[tid] = (int64_t)acc;
    __syncthreads();
    if (sl == 0) {
        uint64_t o = 0;
#pragma unroll
        for (int s2 = 0; s2 < SL; ++s2)
            o += (uint64_t)part[s2 * HD + d];
        if (COH)
            __hip_atomic_store(&out[(size_t)h * HD + d], (int64_t)o, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        else
            out[(size_t)h * HD + d] = (int64_t)o;
    }
}

} // namespace
