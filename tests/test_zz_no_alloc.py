"""The allocation-free entry point q48_attn_decode_rope_noalloc, through the
C ABI, against q48_attn_decode_rope (the entry point it is a variant of):
the same output and the same KV-cache writes on two calls in a row, the
second with a smaller input, and a clear error for a workspace larger than
its fixed scratch."""
import ctypes as C

import numpy as np
import pytest

import intllm
import spec

pytestmark = pytest.mark.gpu

ONE = 1 << 48
P = C.c_void_p


def say(*a):
    print("[case]", *a, flush=True)


def _lib():
    lib = intllm.hip_lib()
    f = lib.q48_attn_decode_rope_noalloc
    f.argtypes = [P, P, P, P, P, P, P] + [C.c_int] * 6
    f.restype = C.c_int
    lib.q48_attn_noalloc_max_bytes.restype = C.c_size_t
    return lib


def _device_free_bytes() -> int:
    """hipMemGetInfo's free bytes on the current device (the HIP runtime is
    loaded with libintllm_hip, whose symbols are global)."""
    hip = C.CDLL(None)
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def _case(ctx, lib, rng, nh, nkv, hd, max_seq, pos, layer=1, noalloc_first=False):
    kvd = nkv * hd
    kc = (rng.standard_normal(2 * max_seq * kvd) * ONE).astype(np.int64)
    vc = (rng.standard_normal(2 * max_seq * kvd) * ONE).astype(np.int64)
    q = (rng.standard_normal(nh * hd) * 3 * ONE).astype(np.int64)
    kn = (rng.standard_normal(kvd) * ONE).astype(np.int64)
    vn = (rng.standard_normal(kvd) * ONE).astype(np.int64)
    dq, dkn, dvn = ctx.to_device(q), ctx.to_device(kn), ctx.to_device(vn)
    dk1, dv1, do1 = ctx.to_device(kc), ctx.to_device(vc), ctx.buffer(nh * hd)
    dk2, dv2, do2 = ctx.to_device(kc), ctx.to_device(vc), ctx.buffer(nh * hd)

    def allocating():
        ctx.attn_decode_rope(do1.ptr, dq.ptr, dk1.ptr, dv1.ptr, dkn.ptr, dvn.ptr, layer, pos, nh,
                             nkv, hd, max_seq)

    def noalloc():
        say("noalloc attention", nh, nkv, hd, "max_seq", max_seq, "pos", pos)
        ctx.sync()
        before = _device_free_bytes()
        rc = lib.q48_attn_decode_rope_noalloc(ctx.h, do2.ptr, dq.ptr, dk2.ptr, dv2.ptr, dkn.ptr,
                                              dvn.ptr, layer, pos, nh, nkv, hd, max_seq)
        assert rc == 0, intllm.strerror(rc)
        ctx.sync()
        # no device memory was taken (on a fresh context a fall-back to the
        # context's workspace would allocate it now)
        assert _device_free_bytes() == before

    # the existing entry point on one copy of the cache, the allocation-free
    # one on another
    if noalloc_first:
        noalloc()
        allocating()
    else:
        allocating()
        noalloc()
    ctx.sync()
    assert ctx.attn_status() == 0
    want, got = do1.download(), do2.download()
    assert np.array_equal(got, want)
    assert np.array_equal(dk2.download(), dk1.download())
    assert np.array_equal(dv2.download(), dv1.download())
    for b in (dq, dkn, dvn, dk1, dv1, do1, dk2, dv2, do2):
        b.free()


def test_noalloc_attention_equals_allocating_entry(ctx):
    lib = _lib()
    rng = np.random.default_rng(2025)
    ctx.rope_init(64, 4096, 10000)
    # split attention (chunks over many blocks), the scratch holding its
    # chunk maxima, chunk sums and barrier words; then a smaller call that
    # reuses the same scratch
    _case(ctx, lib, rng, 32, 4, 64, 4096, 2100)
    _case(ctx, lib, rng, 8, 2, 64, 1024, 700)
    # below the split position: one block per head, no scratch
    _case(ctx, lib, rng, 8, 2, 64, 1024, lib.q48_attn_split_min() - 56)


def test_noalloc_first_on_fresh_context(ctx):
    """On a context that has never allocated a workspace, the allocation-free
    entry point runs first (device free memory unchanged across the call),
    then the allocating one: the same outputs and cache writes."""
    lib = _lib()
    rng = np.random.default_rng(77)
    # the kernels' code is loaded on the device before the measured calls
    ctx.rope_init(64, 4096, 10000)
    _case(ctx, lib, rng, 32, 4, 64, 4096, 1500)
    _case(ctx, lib, rng, 8, 2, 64, 1024, 700)
    with intllm.Context(0) as fresh:
        fresh.rope_init(64, 4096, 10000)
        _case(fresh, lib, rng, 32, 4, 64, 4096, 2100, noalloc_first=True)
        fresh.rope_init(64, 1024, 10000)
        _case(fresh, lib, rng, 8, 2, 64, 1024, 700, noalloc_first=True)


def test_noalloc_split_fallback_rejects_oversize(ctx):
    """A cache of at most 4096 positions (no workspace for the single-block
    kernels) with the one-launch kernel off: the three-launch split attention
    needs 128 heads x 4096 scores, more than the scratch holds, and its own
    workspace check refuses the call (Q48_ETOOBIG) before anything runs."""
    lib = _lib()
    cap = lib.q48_attn_noalloc_max_bytes()
    nh, nkv, hd, max_seq = 128, 16, 64, 4096
    assert nh * max_seq * 8 > cap
    ctx.rope_init(hd, max_seq, 10000)
    ctx.set_attn_one_launch(False)
    try:
        bufs = [ctx.buffer(n) for n in (nh * hd, nh * hd, max_seq * nkv * hd,
                                        max_seq * nkv * hd, nkv * hd, nkv * hd)]
        rc = lib.q48_attn_decode_rope_noalloc(ctx.h, *[b.ptr for b in bufs], 0, 1000, nh, nkv,
                                              hd, max_seq)
        assert rc == intllm.Q48_ETOOBIG
        # below the split position the same call needs no workspace
        rc = lib.q48_attn_decode_rope_noalloc(ctx.h, *[b.ptr for b in bufs], 0,
                                              lib.q48_attn_split_min() - 56, nh, nkv, hd, max_seq)
        assert rc == 0, intllm.strerror(rc)
        ctx.sync()
        for b in bufs:
            b.free()
    finally:
        ctx.set_attn_one_launch(True)


def test_noalloc_attention_rejects_oversize(ctx):
    """A cache longer than 4096 positions: the single-block kernel keeps its
    32 heads x 16384 scores in the workspace, more than the scratch holds,
    so the call is refused (Q48_ETOOBIG) before anything is launched."""
    lib = _lib()
    cap = lib.q48_attn_noalloc_max_bytes()
    assert 0 < cap <= 4 * 1024 * 1024   # the stated maximum: a 4 MiB array
    nh, nkv, hd, max_seq = 32, 4, 64, 16384
    assert nh * max_seq * 8 > cap
    ctx.rope_init(hd, max_seq, 10000)
    ctx.set_attn_one_launch(False)
    try:
        bufs = [ctx.buffer(n) for n in (nh * hd, nh * hd, max_seq * nkv * hd,
                                        max_seq * nkv * hd, nkv * hd, nkv * hd)]
        rc = lib.q48_attn_decode_rope_noalloc(ctx.h, *[b.ptr for b in bufs], 0, 1000, nh, nkv,
                                              hd, max_seq)
        assert rc == intllm.Q48_ETOOBIG
        for b in bufs:
            b.free()
    finally:
        ctx.set_attn_one_launch(True)
