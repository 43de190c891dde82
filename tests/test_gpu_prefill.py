"""Batched prefill (q48h_prefill): the prompt's T tokens as row ops and
q48_gemm projections instead of T llama_forward calls
(llama_int.c:3081-3092).  The bar is the per-token path's bits: every
logits row equals the reference's per-step hash (tests/golden/*_generate.json)
or the sequential q48h_forward's row, and the KV cache equals the one that T
forward calls leave, word for word."""
import ctypes as C
import os

import numpy as np
import pytest

import intllm
import spec
from conftest import golden

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def threads():
    return max(1, min(16, os.cpu_count() or 1))


def kv_rows(ctx, m, cfg, npos):
    """The first npos cached positions of every layer: (keys, values)."""
    dim, nl, nkv, hd, ms = cfg[0], cfg[4], cfg[2], cfg[3], cfg[7]
    kvd = nkv * hd
    out = []
    for p in m.kv_pointers():
        a = np.empty((nl, npos, kvd), dtype=np.int64)
        for l in range(nl):
            intllm.check("q48_memcpy_d2h", intllm.hip_lib().q48_memcpy_d2h(
                ctx.h, a[l].ctypes.data, C.c_void_p(p + 8 * l * ms * kvd), npos * kvd * 8))
        out.append(a)
    return out


def sequential(m, tokens, p0, vocab):
    rows = []
    for i, tok in enumerate(tokens):
        _, lg = m.forward(tok, p0 + i, vocab, choose=False)
        rows.append(lg)
    return np.stack(rows)


def test_tiny_prefill_equals_reference_steps(ctx):
    """The 16-token prompt in one pass: the 16 logits hashes and the first
    generated token of the reference's generate, and the KV cache of the
    per-token path."""
    g = golden("tiny_generate.json")
    cfg = g["config"]
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    try:
        m.synth(g["seed"], threads())
        P = len(g["prompt"])
        say("tiny prefill T", P)
        nxt, lg = m.prefill(g["prompt"], 0, cfg[6])
        assert [intllm.fnv(r) for r in lg] == g["step_fnv"][:P]
        assert nxt == g["tokens"][P]
        kb = kv_rows(ctx, m, cfg, P)
        m.kv_reset()
        sequential(m, g["prompt"], 0, cfg[6])
        ks = kv_rows(ctx, m, cfg, P)
        assert all(np.array_equal(a, b) for a, b in zip(kb, ks))
    finally:
        m.free()


def test_tiny_prefill_in_chunks(ctx):
    """The prompt as chunks of 5, 1 (the per-token route) and 10 tokens at
    p0 = 0, 5, 6: each chunk's rows are the reference's steps."""
    g = golden("tiny_generate.json")
    cfg = g["config"]
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    try:
        m.synth(g["seed"], threads())
        hs = []
        for a, b in ((0, 5), (5, 6), (6, 16)):
            say("tiny prefill chunk", a, b)
            _, lg = m.prefill(g["prompt"][a:b], a, cfg[6], choose=False)
            hs += [intllm.fnv(r) for r in lg]
        assert hs == g["step_fnv"][:16]
    finally:
        m.free()


@pytest.mark.parametrize("chunks", [((0, 1100), (1100, 1500)), ((0, 300), (300, 333))])
def test_tiny_long_prefill_equals_sequential(ctx, chunks):
    """Random prompts of 1100 (the GEMM's digit-correction route, attention
    spans past one LDS tile of keys) and 300 tokens, each followed by a
    second chunk at p0 > 0: logits rows and KV cache against the per-token
    forward on the same weights."""
    cfg = list(spec.TINY)
    n = chunks[-1][1]
    toks = [int(t) for t in np.random.default_rng(n).integers(0, cfg[6], size=n)]
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    try:
        m.synth(7, threads())
        got = []
        for a, b in chunks:
            say("tiny batched prefill", a, b)
            _, lg = m.prefill(toks[a:b], a, cfg[6], choose=False)
            got.append(lg)
        got = np.concatenate(got)
        kb = kv_rows(ctx, m, cfg, n)
        m.kv_reset()
        say("tiny sequential forward", n)
        want = sequential(m, toks, 0, cfg[6])
        ks = kv_rows(ctx, m, cfg, n)
        bad = [i for i in range(n) if not np.array_equal(got[i], want[i])]
        assert not bad, (len(bad), bad[:5])
        assert all(np.array_equal(a, b) for a, b in zip(kb, ks))
    finally:
        m.free()


def test_prefill_planes_follow_weight_uploads(ctx):
    """The prefill's prepared weight planes (made at the first prefill of 128
    tokens or more; the tiny config's gate|up, 1376 rows, takes the planes
    kernel) are made again after q48h_upload: a 200-token prefill after one
    layer's gate and up weights change equals the per-token forward on the
    new weights, and one with the planes turned off equals it too."""
    cfg = list(spec.TINY)
    n = 200
    toks = [int(t) for t in np.random.default_rng(21).integers(0, cfg[6], size=n)]
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    try:
        m.synth(9, threads())
        say("tiny prefill 200 (prepares the planes)")
        m.prefill(toks, 0, cfg[6], choose=False)
        rng = np.random.default_rng(22)
        for nm in ("model.layers.1.mlp.gate_proj.weight", "model.layers.1.mlp.up_proj.weight"):
            w = (rng.integers(-(1 << 40), 1 << 40, size=cfg[5] * cfg[0], dtype=np.int64)
                 >> 24) << 24
            m.upload(nm, w)
        m.kv_reset()
        say("tiny prefill 200 after the upload")
        _, got = m.prefill(toks, 0, cfg[6], choose=False)
        m.kv_reset()
        m.set_gemm_planes(False)
        _, off = m.prefill(toks, 0, cfg[6], choose=False)
        m.set_gemm_planes(True)
        m.kv_reset()
        say("tiny sequential forward 200")
        want = sequential(m, toks, 0, cfg[6])
        bad = [i for i in range(n) if not np.array_equal(got[i], want[i])]
        assert not bad, (len(bad), bad[:5])
        assert np.array_equal(off, want)
    finally:
        m.free()


def test_generate_batched_and_per_token_prefill_agree(ctx):
    """generate() with the batched prompt (default) and with per-token
    forward calls: both the reference's tokens and step hashes."""
    g = golden("tiny_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        m.synth(g["seed"], threads())
        for on in (True, False, True):
            say("generate batched_prefill", on)
            m.set_batched_prefill(on)
            toks, hs, _ = m.generate(g["prompt"], g["max_new"])
            assert toks == g["tokens"]
            assert ["%016x" % h for h in hs] == g["step_fnv"]
            toks, _, _ = m.generate(g["prompt"], g["max_new"], hashes=False)
            assert toks == g["tokens"]
    finally:
        m.free()


def test_prefill_range_errors(ctx):
    cfg = list(spec.TINY)
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    try:
        for toks, p0, code in (([1, 2, 3], cfg[7] - 2, intllm.Q48_ERANGE),
                               ([1, cfg[6], 3], 0, intllm.Q48_ERANGE),
                               ([1, -1], 0, intllm.Q48_ERANGE),
                               ([1, 2], -1, intllm.Q48_ERANGE),
                               ([], 0, intllm.Q48_EINVAL)):
            with pytest.raises(intllm.Q48Error) as e:
                m.prefill(toks, p0, cfg[6])
            assert e.value.code == code, (toks, p0)
    finally:
        m.free()


def test_tinyllama_prefill_equals_reference_and_sequential(ctx):
    """Config 3: the 32-token golden prompt in one pass against the
    reference's hashes and first token, then 480 more random tokens in one
    pass at p0 = 32 against the per-token forward (hashes of every row and
    the KV cache).  The 480-token pass runs its projections through the
    weights' prepared digit planes (the default) and again splitting W in
    each GEMM."""
    g = golden("tinyllama_generate.json")
    cfg = g["config"]
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    try:
        say("tinyllama synth (8.8 GB)")
        m.synth(g["seed"], threads())
        P = len(g["prompt"])
        say("tinyllama prefill T", P)
        nxt, lg = m.prefill(g["prompt"], 0, cfg[6])
        assert [intllm.fnv(r) for r in lg] == g["step_fnv"][:P]
        assert nxt == g["tokens"][P]
        more = [int(t) for t in np.random.default_rng(5).integers(0, cfg[6], size=480)]
        say("tinyllama prefill T 480 at 32")
        _, lg = m.prefill(more, P, cfg[6], choose=False)
        got = [intllm.fnv(r) for r in lg]
        kb = kv_rows(ctx, m, cfg, P + 480)
        m.kv_reset()
        m.set_gemm_planes(False)
        say("tinyllama prefill T 32 + 480, W split per GEMM")
        m.prefill(g["prompt"], 0, cfg[6], choose=False)
        _, lg = m.prefill(more, P, cfg[6], choose=False)
        assert [intllm.fnv(r) for r in lg] == got
        m.set_gemm_planes(True)
        m.kv_reset()
        say("tinyllama sequential forward 512")
        want = []
        for i, tok in enumerate(g["prompt"] + more):
            _, r = m.forward(tok, i, cfg[6], choose=False)
            if i >= P:
                want.append(intllm.fnv(r))
        ks = kv_rows(ctx, m, cfg, P + 480)
        assert got == want
        assert all(np.array_equal(a, b) for a, b in zip(kb, ks))
    finally:
        m.free()
