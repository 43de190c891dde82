"""The decode layer's first half with RoPE and the KV store in the q|k|v
projection (q48_norm_gemv_rope_kv, its bfloat16 form) and attention from the
cache (q48_attn_decode_cached), against the oracle's composition of the
reference steps: rmsnorm + matmul_vec (llama_int.c:1014-1058), rope_apply on
the q and k heads (llama_int.c:997-1008, 1392-1395), the KV store at pos
(llama_int.c:1414-1416) and attention (llama_int.c:1060-1072, 1502-1529).
Bit-exact."""
import numpy as np
import pytest

import intllm
import oracle_lib as O
import spec
from test_gpu_ops import _bf16_matrix, _bf16_values, _rms

pytestmark = pytest.mark.gpu

ONE = 1 << 48


def say(*a):
    print("[rope_kv]", *a, flush=True)


def _oracle_case(oracle, rng, nh, nkv, hd, K, max_seq, pos, W, x, nw, kc, vc, layer):
    """Expected qkv rows (q, k rotated), caches after the store, attention."""
    M = (nh + 2 * nkv) * hd
    kvd = nkv * hd
    qkv = O.gemv(W, _rms(oracle, x, nw), M, K)
    cos_t = np.empty(max_seq * hd // 2, dtype=np.int64)
    sin_t = np.empty(max_seq * hd // 2, dtype=np.int64)
    oracle.q48o_rope_tables(cos_t.ctypes.data, sin_t.ctypes.data, hd, max_seq, 10000)
    q = qkv[:nh * hd].copy()
    k = qkv[nh * hd:nh * hd + kvd].copy()
    v = qkv[nh * hd + kvd:].copy()
    for h in range(nh):
        oracle.q48o_rope_apply(cos_t.ctypes.data, sin_t.ctypes.data, hd // 2,
                               q[h * hd:].ctypes.data, pos)
    for h in range(nkv):
        oracle.q48o_rope_apply(cos_t.ctypes.data, sin_t.ctypes.data, hd // 2,
                               k[h * hd:].ctypes.data, pos)
    out = np.empty(nh * hd, dtype=np.int64)
    # stores k and v at pos into kc, vc
    oracle.q48o_attn_decode(out.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                            k.ctypes.data, v.ctypes.data, layer, pos, nh, nkv, hd, max_seq)
    return np.concatenate([q, k, v]), out


@pytest.mark.parametrize("nh,nkv,hd,K,max_seq,positions", [
    # TinyLlama heads (the v5 pipeline with 16 tiles per wave)
    (32, 4, 64, 2048, 600, [0, 1, 37, 63, 64, 127, 128, 129, 191, 192, 255, 256, 257, 300,
                            383, 447, 511]),
    (8, 2, 32, 256, 200, [0, 5, 199]),
    (16, 4, 128, 1024, 300, [0, 130, 299]),
    # K off the unrolled pipeline (the batched-loop kernel)
    (8, 2, 64, 7680, 100, [3, 99]),
])
def test_rope_kv_projection_and_cached_attention(ctx, oracle, nh, nkv, hd, K, max_seq,
                                                 positions):
    rng = np.random.default_rng(nh * 131 + hd + K)
    M = (nh + 2 * nkv) * hd
    kvd = nkv * hd
    layers = 2
    W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
    kc = (rng.standard_normal(layers * max_seq * kvd) * ONE).astype(np.int64)
    vc = (rng.standard_normal(layers * max_seq * kvd) * ONE).astype(np.int64)
    ctx.rope_init(hd, max_seq, 10000)
    dW, dkc, dvc = ctx.to_device(W), ctx.to_device(kc), ctx.to_device(vc)
    dqkv, do, do2 = ctx.buffer(M), ctx.buffer(nh * hd), ctx.buffer(nh * hd)
    ds = ctx.buffer(intllm.stats_words(K) + 2)
    for pos in positions:
        x = (rng.standard_normal(K) * 3 * ONE).astype(np.int64)
        nw = (rng.standard_normal(K) * ONE).astype(np.int64)
        want_qkv, want_out = _oracle_case(oracle, rng, nh, nkv, hd, K, max_seq, pos, W, x, nw,
                                          kc, vc, 1)
        dx, dnw = ctx.to_device(x), ctx.to_device(nw)
        ctx.rms_stats(ds.ptr, dx.ptr, K)
        say("norm_gemv_rope_kv", nh, nkv, hd, "K", K, "max_seq", max_seq, "pos", pos)
        ctx.norm_gemv_rope_kv(dqkv.ptr, dW.ptr, dx.ptr, dnw.ptr, ds.ptr, dkc.ptr, dvc.ptr, 1,
                              pos, nh, nkv, hd, max_seq, K)
        assert np.array_equal(dqkv.download(), want_qkv), ("qkv", pos)
        assert np.array_equal(dkc.download(), kc), ("k cache", pos)
        assert np.array_equal(dvc.download(), vc), ("v cache", pos)
        say("attn_decode_cached", "pos", pos)
        ctx.attn_decode_cached(do.ptr, dqkv.ptr, dkc.ptr, dvc.ptr, 1, pos, nh, nkv, hd, max_seq)
        assert np.array_equal(do.download(), want_out), ("attention", pos)
        # the idle compute units reading another buffer meanwhile: same bits
        ctx.attn_decode_cached(do2.ptr, dqkv.ptr, dkc.ptr, dvc.ptr, 1, pos, nh, nkv, hd,
                               max_seq, dvc.ptr, (vc.size * 8) // 16 * 16)
        assert np.array_equal(do2.download(), want_out), ("attention, prefetch", pos)
        assert np.array_equal(dkc.download(), kc) and np.array_equal(dvc.download(), vc)
        dx.free()
        dnw.free()
    for b in (dW, dkc, dvc, dqkv, do, do2, ds):
        b.free()


@pytest.mark.parametrize("mode", ["window", "mixed"])
@pytest.mark.parametrize("nh,nkv,hd,K", [(32, 4, 64, 2048), (16, 4, 128, 1024)])
def test_rope_kv_projection_bf16_equals_int64(ctx, oracle, nh, nkv, hd, K, mode):
    """The bfloat16 form gives the int64 form's bits on the expanded weights:
    qkv rows and both caches."""
    rng = np.random.default_rng(nh + hd + K + len(mode))
    M = (nh + 2 * nkv) * hd
    kvd = nkv * hd
    max_seq, pos = 64, 41
    bits = _bf16_matrix(rng, M, K, mode)
    W = _bf16_values(oracle, np.arange(1 << 16, dtype=np.uint16))[bits]
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    nw = (rng.standard_normal(K) * ONE).astype(np.int64)
    kc = (rng.standard_normal(max_seq * kvd) * ONE).astype(np.int64)
    ctx.rope_init(hd, max_seq, 10000)
    dW, dWb = ctx.to_device(W), ctx.buffer((M * K + 3) // 4)
    dWb.upload(np.concatenate([bits, np.zeros((-M * K) % 4, np.uint16)]).view(np.int64))
    dx, dnw = ctx.to_device(x), ctx.to_device(nw)
    ds = ctx.buffer(intllm.stats_words(K) + 2)
    ctx.rms_stats(ds.ptr, dx.ptr, K)
    ka, va, kb, vb = (ctx.to_device(kc) for _ in range(4))
    ya, yb = ctx.buffer(M), ctx.buffer(M)
    say("norm_gemv_rope_kv bf16", nh, nkv, hd, K, mode)
    ctx.norm_gemv_rope_kv(ya.ptr, dW.ptr, dx.ptr, dnw.ptr, ds.ptr, ka.ptr, va.ptr, 0, pos, nh,
                          nkv, hd, max_seq, K)
    ctx.norm_gemv_rope_kv_bf16(yb.ptr, dWb.ptr, dx.ptr, dnw.ptr, ds.ptr, kb.ptr, vb.ptr, 0, pos,
                               nh, nkv, hd, max_seq, K)
    assert np.array_equal(ya.download(), yb.download())
    assert np.array_equal(ka.download(), kb.download())
    assert np.array_equal(va.download(), vb.download())
    for b in (dW, dWb, dx, dnw, ds, ka, va, kb, vb, ya, yb):
        b.free()


def test_rope_kv_errors(ctx):
    """Out-of-range positions, unsupported head sizes and caches past the
    single-block attention's reach are refused before any launch."""
    nh, nkv, hd, K, max_seq = 8, 2, 64, 512, 32
    M = (nh + 2 * nkv) * hd
    ctx.rope_init(hd, max_seq, 10000)
    dW, dx, dnw = ctx.buffer(M * K), ctx.buffer(K), ctx.buffer(K)
    ds, dq = ctx.buffer(intllm.stats_words(K) + 2), ctx.buffer(M)
    dkc, dvc, do = ctx.buffer(max_seq * nkv * hd), ctx.buffer(max_seq * nkv * hd), ctx.buffer(M)
    args = (dq.ptr, dW.ptr, dx.ptr, dnw.ptr, ds.ptr, dkc.ptr, dvc.ptr, 0)
    for pos, want in ((max_seq, intllm.Q48_ERANGE), (-1, intllm.Q48_ERANGE)):
        with pytest.raises(intllm.Q48Error) as e:
            ctx.norm_gemv_rope_kv(*args, pos, nh, nkv, hd, max_seq, K)
        assert e.value.code == want
        with pytest.raises(intllm.Q48Error) as e:
            ctx.attn_decode_cached(do.ptr, dq.ptr, dkc.ptr, dvc.ptr, 0, pos, nh, nkv, hd, max_seq)
        assert e.value.code == want
    with pytest.raises(intllm.Q48Error) as e:   # head_dim 16: not a supported head size
        ctx.norm_gemv_rope_kv(*args, 0, nh, nkv, 16, max_seq, K)
    assert e.value.code == intllm.Q48_EINVAL
    with pytest.raises(intllm.Q48Error) as e:   # RoPE tables for another head_dim
        ctx.norm_gemv_rope_kv(*args, 0, nh // 2, nkv // 2, 128, max_seq, K)
    assert e.value.code == intllm.Q48_ESTATE
    with pytest.raises(intllm.Q48Error) as e:   # scores of > 4096 positions do not fit LDS
        ctx.attn_decode_cached(do.ptr, dq.ptr, dkc.ptr, dvc.ptr, 0, 0, nh, nkv, hd, 4097)
    assert e.value.code == intllm.Q48_EINVAL
    for b in (dW, dx, dnw, ds, dq, dkc, dvc, do):
        b.free()
