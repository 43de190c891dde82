"""Device sampling (q48_sample / q48_sample_step, sample_token of
llama_int.c:2958-3039) against the reference's own draws recorded in
tests/golden/sample.json and against the oracle (oracle/q48_oracle.c
q48o_sample, itself pinned to those draws by tests/test_oracle_ops.py).

Bit-exact bar: the token and the xoroshiro128+ state after the draw."""
import ctypes as C
import os

import numpy as np
import pytest

import intllm
import oracle_lib as O
import spec
from conftest import golden

pytestmark = pytest.mark.gpu
ONE = spec.ONE


def say(*a):
    print("[case]", *a, flush=True)


def threads():
    return max(1, min(16, os.cpu_count() or 1))


class Sampler:
    """Device logits buffer + rng state for one context."""

    def __init__(self, ctx, cap):
        self.ctx = ctx
        self.lg = ctx.buffer(cap)
        self.rng = ctx.buffer(2)

    def __call__(self, x, T, k, p, state):
        x = np.ascontiguousarray(x, dtype=np.int64)
        self.lg.upload(x)
        self.rng.upload(np.array(state, dtype=np.uint64).view(np.int64))
        tok = self.ctx.sample(self.lg.ptr, x.size, T, k, p, self.rng.ptr)
        st = self.rng.download(2).view(np.uint64)
        return tok, [int(st[0]), int(st[1])]

    def free(self):
        self.lg.free()
        self.rng.free()


def test_rng_seed_matches_reference(ctx):
    """q48_rng_seed (host) against the reference's rng_seed states."""
    for seed, v in golden("sample.json")["rng"].items():
        assert ["%016x" % w for w in intllm.rng_seed(int(seed))] == v["state"]


def test_sample_matches_reference_draws(ctx):
    """All 1176 recorded sample_token calls: four logit kinds (spread, runs
    of ties, one dominant logit, magnitudes that wrap the temperature
    division and the softmax sums), temperatures on both sides of the 0.01
    greedy floor, top-k off / 1 / 2 / 10 / 50 / n - 1, top-p off / 0.05 /
    0.5 / 0.9 / 0.999 / 1.0, on 512 and 32000 logits."""
    cases = golden("sample.json")["cases"]
    s = Sampler(ctx, 32000)
    try:
        say("sample_token, recorded cases", len(cases))
        bad = []
        for c in cases:
            x = spec.sample_logits(c["kind"], c["seed"], c["n"])
            st = [int(v, 16) for v in c["rng_in"]]
            tok, st2 = s(x, c["T"], c["top_k"], c["top_p"], st)
            if tok != c["token"] or ["%016x" % v for v in st2] != c["rng_out"]:
                bad.append((c, tok))
        assert not bad, bad[:3]
    finally:
        s.free()


@pytest.mark.parametrize("n", [1, 2, 3, 63, 1000, 1025, 32000, 50257])
def test_sample_random_equals_oracle(ctx, n):
    """Random logits and parameters at vocabulary sizes around the block and
    chunk boundaries (and GPT-2's 50257), against the oracle."""
    rng = np.random.default_rng(n)
    s = Sampler(ctx, n)
    try:
        say("sample vs oracle, n", n)
        for it in range(24):
            scale = int(rng.choice([1, 4, 40, 4000]))
            x = rng.integers(-scale * ONE, scale * ONE, size=n, dtype=np.int64)
            if it % 4 == 1:
                x = x[rng.integers(0, n, size=n)] // (ONE // 4) * (ONE // 4)   # ties
            T = int(rng.choice([ONE // 100, ONE // 3, ONE, 2 * ONE, ONE // 100 - 1]))
            k = int(rng.choice([0, 1, 3, max(1, n // 2), max(1, n - 1), n, n + 5]))
            p = int(rng.choice([ONE, 0, ONE // 10, ONE // 2, ONE * 95 // 100, 1]))
            st = O.rng_seed(int(rng.integers(0, 2**63)))
            want = O.sample(x, T, k, p, st)
            got = s(x, T, k, p, st)
            assert got == want, (n, it, T, k, p)
    finally:
        s.free()


def test_generate_sampled_matches_reference(ctx):
    """generate() with sampling on the tiny model (llama_int.c:3067-3135):
    the C host's loop, token choice on the device, equals the reference's
    streams for four (temperature, top-k, top-p, seed) settings."""
    g = golden("sample.json")["generate_tiny"]
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        m.synth(g["seed"], threads())
        for r in g["runs"]:
            say("generate sampled", r["T"], r["top_k"], r["top_p"], r["seed"])
            m.set_sampling(r["T"], r["top_k"], r["top_p"], r["seed"])
            toks, _, _ = m.generate(g["prompt"], g["max_new"])
            assert toks == r["tokens"], r
    finally:
        m.free()


def test_graph_decode_sampled_matches_reference(ctx):
    """The same streams with the decode steps replayed from a captured graph
    (q48_sample_step: token choice and rng state on the device): prefill
    with the host forward, then q48h_decode_graph."""
    g = golden("sample.json")["generate_tiny"]
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        m.synth(g["seed"], threads())
        P = len(g["prompt"])
        for r in g["runs"]:
            say("graph decode sampled", r["T"], r["top_k"], r["top_p"], r["seed"])
            m.set_sampling(r["T"], r["top_k"], r["top_p"], r["seed"])
            m.kv_reset()
            nxt = None
            for pos, tok in enumerate(g["prompt"]):
                nxt, _ = m.forward(tok, pos, spec.TINY[6], logits=False, choose=pos == P - 1)
            want = r["tokens"][P:]
            assert nxt == want[0]
            # decode_graph stops after EOS; the reference does not append it
            n = g["max_new"] - 1
            _, steps, _ = m.decode_graph(nxt, P, n)
            # the token chosen at the prompt's end is kept even if it is EOS
            # (llama_int.c:3087-3090); decode stops before an EOS (3111)
            dec = list(steps)
            if 2 in dec:
                dec = dec[:dec.index(2)]
            assert [nxt] + dec == want, r
    finally:
        m.free()


def test_tinyllama_sampled_generate_and_graph_match_reference(ctx):
    """Config 3 (TinyLlama-1.1B shape) with temperature 0.8, top-k 40,
    top-p 0.9: the reference's 16 sampled tokens, through the host generate
    loop and through graph-replayed decode steps."""
    g = golden("sample_tinyllama.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tinyllama synth (8.8 GB)")
        m.synth(g["seed"], threads())
        say("tinyllama generate sampled")
        m.set_sampling(g["T"], g["top_k"], g["top_p"], g["rng_seed"])
        toks, _, _ = m.generate(g["prompt"], g["max_new"], hashes=False)
        assert toks == g["tokens"]
        say("tinyllama graph decode sampled")
        m.set_sampling(g["T"], g["top_k"], g["top_p"], g["rng_seed"])
        m.kv_reset()
        P = len(g["prompt"])
        nxt = None
        for pos, tok in enumerate(g["prompt"]):
            nxt, _ = m.forward(tok, pos, g["config"][6], logits=False, choose=pos == P - 1)
        _, steps, _ = m.decode_graph(nxt, P, g["max_new"] - 1)
        dec = list(steps)
        if 2 in dec:
            dec = dec[:dec.index(2)]
        assert [nxt] + dec == g["tokens"][P:]
    finally:
        m.free()
