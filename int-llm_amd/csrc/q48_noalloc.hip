// q48_noalloc.hip — the allocation-free entry point of libintllm_hip:
// q48_attn_decode_rope_noalloc, for callers that cannot allocate device
// memory (code under graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  It is q48_attn_decode_rope with the split attention's
// workspace taken from a fixed device array instead of the context's
// workspace, which q48_attn_decode_rope grows with hipMalloc on demand.
#include "../../include/intllm_hip.h"
#include "q48_internal.h"

#include <mutex>

namespace {

int launch_rc(int e) { return e == (int)hipSuccess ? Q48_OK : Q48_EHIP; }

constexpr int kMaxHeadDim = 256;

} // namespace

// ---- the allocation-free entry point's scratch ------------------------------
// The device memory of q48_attn_decode_rope_noalloc: the three-launch split
// attention's scores, chunk maxima and chunk sums (where the one-launch
// k_attn_g does not serve) in the first q48_scratch_bytes() bytes, then
// k_attn_g's exchange region: epoch-tagged exchange words, per-KV-head
// epochs and the error word.  One copy per device (a file-scope device
// array), zero at load; the exchange region is zeroed once per device here,
// and again only by q48_attn_status after a timeout or by q48_attg_account
// before the epochs could wrap.  Host code never uses the array's name as a
// device address: q48_scratch_init looks its address up once per device.
constexpr size_t Q48_SCRATCH_BYTES = (size_t)4 << 20;   // the stated maximum: 4 MiB
static __device__ __align__(256) int64_t scratch[Q48_SCRATCH_BYTES / sizeof(int64_t)];

size_t q48_scratch_bytes() { return Q48_SCRATCH_BYTES - q48_attn_sync_bytes(); }

// k_attn_g launches on each device's scratch exchange region (every context
// on the device shares the array)
uint64_t *q48_scratch_attg_count(int device)
{
    static uint64_t count[64];
    return device >= 0 && device < 64 ? &count[device] : nullptr;
}

int q48_scratch_init(q48_ctx *c)
{
    static std::mutex mu;
    static int64_t *addr[64];      // per device
    if (c->device < 0 || c->device >= 64)
        return Q48_EINVAL;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[c->device]) {
        // the calling thread has this context's device current
        int64_t *p = nullptr;
        if (hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
            return Q48_EHIP;
        // the barrier region starts at zero (the array is zero at load; this
        // makes it explicit, once per device)
        unsigned *sy = reinterpret_cast<unsigned *>(reinterpret_cast<char *>(p) +
                                                    q48_scratch_bytes());
        if (q48_launch_zero(c, sy, q48_attn_sync_bytes()) != (int)hipSuccess ||
            hipStreamSynchronize(c->stream) != hipSuccess)
            return Q48_EHIP;
        addr[c->device] = p;
    }
    c->scratch = addr[c->device];
    c->scratch_sync = reinterpret_cast<unsigned *>(
        reinterpret_cast<char *>(c->scratch) + q48_scratch_bytes());
    return Q48_OK;
}

extern "C" {

int q48_attn_decode_rope_noalloc(q48_ctx *c, int64_t *out, const int64_t *q, int64_t *kcache,
                                 int64_t *vcache, const int64_t *k_new, const int64_t *v_new,
                                 int layer, int pos, int n_heads, int n_kv, int head_dim,
                                 int max_seq)
{
    if (!c || !out || !q || !kcache || !vcache || !k_new || !v_new)
        return Q48_EINVAL;
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || head_dim <= 0 ||
        head_dim > kMaxHeadDim || 256 % head_dim || head_dim % 8 || layer < 0 || max_seq <= 0)
        return Q48_EINVAL;
    if (!c->rope_cos || head_dim != c->rope_head_dim || max_seq > c->rope_max_seq)
        return Q48_ESTATE;
    if (pos < 0 || pos >= max_seq)
        return Q48_ERANGE;
    if (!c->scratch)
        return Q48_ESTATE;
    const int *dp = c->step_mode ? c->d_step + 1 : nullptr;
    int rc = q48_launch_attn_v2(c, out, q, kcache, vcache, k_new, v_new, layer, dp, pos, n_heads,
                                n_kv, head_dim, max_seq, 1, nullptr, 0, c->scratch,
                                q48_scratch_bytes(), c->scratch_sync);
    if (rc == Q48_ERANGE)
        return Q48_ETOOBIG;   // the workspace it needs exceeds the scratch
    return launch_rc(rc);
}

size_t q48_attn_noalloc_max_bytes(void) { return q48_scratch_bytes(); }

} // extern "C"
