"""Batched-prefill attention (q48_attn_prefill) against the oracle's decode
attention (llama_int.c:1502-1529, 1060-1072) run row by row: row t of a
prefill is the reference's attention of that row's rotated q at position
p0 + t over the cache rows 0 .. p0 + t.  Both kernels: the int8 matrix-core
kernel (k_pfa, the default) and the VALU kernel (one block per head and row,
up to 4096 cache rows).  Bit-exact.

Cases cover head_dim 32/64/128, row counts that are not a multiple of the
16-row block, p0 > 0, KV-head counts that do and do not divide 8 (the XCD
mapping), full-range int64 operands (every digit of the identity, the top
byte signed) and the largest cache the matrix-core kernel takes with every
key and value INT64_MIN (the digit-product accumulators' bound).
"""
import numpy as np
import pytest

import spec

pytestmark = pytest.mark.gpu
ONE = spec.ONE
I64_MIN = np.iinfo(np.int64).min


def say(*a):
    print("[case]", *a, flush=True)


def full_range(rng, n):
    return rng.integers(np.iinfo(np.int64).min, np.iinfo(np.int64).max, size=n,
                        dtype=np.int64, endpoint=True)


CASES = [
    # nh, nkv, hd, p0, T, max_seq, values
    (32, 4, 64, 0, 300, 320, "normal"),
    (8, 2, 32, 37, 45, 96, "normal"),
    (6, 3, 128, 5, 70, 80, "normal"),
    (4, 1, 64, 0, 17, 17, "full"),
    (16, 16, 32, 100, 33, 140, "full"),
    (2, 1, 64, 16300, 20, 16320, "min"),
]


def make_case(nh, nkv, hd, p0, T, max_seq, values, L=2):
    rng = np.random.default_rng(nh * 1000 + hd * 10 + T)
    kvd = nkv * hd
    row = (nh + 2 * nkv) * hd
    if values == "normal":
        kc = (rng.standard_normal(L * max_seq * kvd) * ONE).astype(np.int64)
        vc = (rng.standard_normal(L * max_seq * kvd) * ONE).astype(np.int64)
        qkv = (rng.standard_normal(T * row) * 3 * ONE).astype(np.int64)
    elif values == "full":
        kc = full_range(rng, L * max_seq * kvd)
        vc = full_range(rng, L * max_seq * kvd)
        qkv = full_range(rng, T * row)
    else:
        kc = np.full(L * max_seq * kvd, I64_MIN, dtype=np.int64)
        vc = np.full(L * max_seq * kvd, I64_MIN, dtype=np.int64)
        qkv = full_range(rng, T * row)
    return kc, vc, qkv


def oracle_rows(oracle, kc, vc, qkv, layer, p0, T, nh, nkv, hd, max_seq):
    kvd = nkv * hd
    row = (nh + 2 * nkv) * hd
    out = np.empty((T, nh * hd), dtype=np.int64)
    kcc, vcc = kc.copy(), vc.copy()
    base = layer * max_seq * kvd
    for t in range(T):
        pos = p0 + t
        q = np.ascontiguousarray(qkv[t * row:t * row + nh * hd])
        kn = np.ascontiguousarray(kcc[base + pos * kvd:base + (pos + 1) * kvd])
        vn = np.ascontiguousarray(vcc[base + pos * kvd:base + (pos + 1) * kvd])
        o = np.empty(nh * hd, dtype=np.int64)
        oracle.q48o_attn_decode(o.ctypes.data, q.ctypes.data, kcc.ctypes.data, vcc.ctypes.data,
                                kn.ctypes.data, vn.ctypes.data, layer, pos, nh, nkv, hd, max_seq)
        out[t] = o
    assert np.array_equal(kcc, kc) and np.array_equal(vcc, vc)
    return out


@pytest.mark.parametrize("nh,nkv,hd,p0,T,max_seq,values", CASES)
def test_prefill_attention_vs_oracle(ctx, oracle, nh, nkv, hd, p0, T, max_seq, values):
    layer = 1
    kc, vc, qkv = make_case(nh, nkv, hd, p0, T, max_seq, values)
    want = oracle_rows(oracle, kc, vc, qkv, layer, p0, T, nh, nkv, hd, max_seq)
    ctx.rope_init(hd, max_seq, 10000)
    dk, dv, dq = ctx.to_device(kc), ctx.to_device(vc), ctx.to_device(qkv)
    do = ctx.buffer(T * nh * hd)
    try:
        kernels = (True, False) if p0 + T <= 4096 else (True,)
        for mfma in kernels:
            say("prefill attention", nh, nkv, hd, "p0", p0, "T", T, values, "mfma", mfma)
            ctx.set_pf_attn_mfma(mfma)
            ctx.attn_prefill(do.ptr, dq.ptr, dk.ptr, dv.ptr, layer, p0, T, nh, nkv, hd, max_seq)
            got = do.download().reshape(T, nh * hd)
            bad = [t for t in range(T) if not np.array_equal(got[t], want[t])]
            assert not bad, (mfma, len(bad), bad[:5])
            assert np.array_equal(dk.download(), kc) and np.array_equal(dv.download(), vc)
    finally:
        ctx.set_pf_attn_mfma(True)
        for b in (dk, dv, dq, do):
            b.free()


def test_prefill_attention_limits(ctx):
    """Past 4096 cache rows the VALU kernel refuses (ERANGE); past 16320 both do."""
    import intllm
    nh, nkv, hd, max_seq = 2, 1, 64, 16384
    ctx.rope_init(hd, max_seq, 10000)
    d = ctx.buffer(8)
    try:
        for mfma, p0, T in ((False, 4090, 10), (True, 16300, 30)):
            ctx.set_pf_attn_mfma(mfma)
            with pytest.raises(intllm.Q48Error) as e:
                ctx.attn_prefill(d.ptr, d.ptr, d.ptr, d.ptr, 0, p0, T, nh, nkv, hd, max_seq)
            assert e.value.code == intllm.Q48_ERANGE, (mfma, p0, T)
    finally:
        ctx.set_pf_attn_mfma(True)
        d.free()
