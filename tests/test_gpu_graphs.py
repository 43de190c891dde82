"""Graph-replayed decode across setting changes, workspace growth and
attention time-outs, through the C host over libintllm_hip.

The model keeps one captured decode step per combination of settings, for
its lifetime; these tests switch settings back and forth, grow the context's
workspace between replays, and force the one-launch split attention to give
up, and check every replayed step against the reference's recorded logits
hashes (tests/golden/tiny_generate.json) or the eager per-token forward."""
import os

import pytest

import intllm
import spec
from conftest import golden

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def threads():
    return max(1, min(16, os.cpu_count() or 1))


def _tiny(ctx, max_seq=None):
    g = golden("tiny_generate.json")
    cfg = list(g["config"])
    if max_seq is not None:
        cfg[7] = max_seq
    m = intllm.HostModel(ctx, intllm.Config(*cfg))
    m.synth(g["seed"], threads())
    return g, m


def test_graph_cache_across_settings(ctx):
    """Greedy (hashed and not), sampled and fused-mode runs interleaved: every
    combination replays its own cached graph, more combinations than the cache
    holds force evictions, and every greedy run gives the reference's hashes."""
    g, m = _tiny(ctx)
    try:
        P, V = len(g["prompt"]), g["config"][6]
        ref = g["step_fnv"]
        say("tiny prefill")
        tok0, _ = m.prefill(g["prompt"], 0, V, logits=False)
        assert tok0 == g["tokens"][P]
        n = 12
        say("greedy hashed")
        _, t1, h1, _ = m.decode_graph_hashed(tok0, P, n)
        assert h1 == ref[P:P + n]
        assert t1 == g["tokens"][P + 1:P + 1 + n]
        samp = spec.SAMPLE_GEN[0]
        say("sampled", samp)
        m.set_sampling(*samp)
        _, s1, _ = m.decode_graph(tok0, P, n)
        say("greedy again")
        m.set_sampling(0)
        _, t2, h2, _ = m.decode_graph_hashed(tok0, P, n)
        assert (t2, h2) == (t1, h1)
        _, t3, _ = m.decode_graph(tok0, P, n)
        assert t3 == t1
        say("sampled again, same seed")
        m.set_sampling(*samp)
        _, s2, _ = m.decode_graph(tok0, P, n)
        assert s2 == s1
        m.set_sampling(0)
        # 4 fused modes x RoPE placement x hashed or not: 16 combinations, more
        # than the 8 cached graphs, each replayed twice
        for rep in range(2):
            for mode in (3, 2, 1, 0):
                for rope in (True, False):
                    say("fused", mode, "rope in gemv", rope, "rep", rep)
                    m.set_fused(mode)
                    m.set_rope_gemv(rope)
                    _, t, h, _ = m.decode_graph_hashed(tok0, P, n)
                    assert (t, h) == (t1, h1), (mode, rope, rep)
                    _, t, _ = m.decode_graph(tok0, P, n)
                    assert t == t1, (mode, rope, rep)
        m.set_fused(3)
        m.set_rope_gemv(True)
        say("context switch between replays: one-launch attention off and on")
        ctx.set_attn_one_launch(False)
        _, t, h, _ = m.decode_graph_hashed(tok0, P, n)
        ctx.set_attn_one_launch(True)
        assert (t, h) == (t1, h1)
    finally:
        m.free()


def test_graph_replay_after_workspace_growth(ctx):
    """A cache longer than 4096 positions: attention takes the context
    workspace inside the captured step.  A batched prefill then grows that
    workspace (the old one is kept while a graph may use it) and the cached
    graph replays again: the reference's hashes, and the eager forward's."""
    g, m = _tiny(ctx, max_seq=8192)
    try:
        P, V = len(g["prompt"]), g["config"][6]
        ref = g["step_fnv"]
        tok0, _ = m.prefill(g["prompt"], 0, V, logits=False)
        n = 10
        say("graph decode, max_seq 8192")
        _, t1, h1, _ = m.decode_graph_hashed(tok0, P, n)
        assert h1 == ref[P:P + n]
        say("eager decode")
        t0_, he, _ = m.decode_from(tok0, P, n)
        assert ["%016x" % h for h in he] == h1
        say("prefill of 1500 tokens at positions 200.. (grows the workspace)")
        tk = spec.prompt(spec.SEED_TINY + 7, 1500, V)
        m.prefill(tk, 200, V, logits=False)
        say("graph decode again")
        _, t2, h2, _ = m.decode_graph_hashed(tok0, P, n)
        assert (t2, h2) == (t1, h1)
        _, t3, _ = m.decode_graph(tok0, P, n)
        assert t3 == t1
    finally:
        m.free()


def test_attention_timeout_reported_then_clean(ctx):
    """The one-launch split attention told to give up at once (a host
    setting: every block still exits normally): the graph decode, the eager
    decode and the single forward report Q48_ETIMEOUT instead of returning
    wrong logits; with the default bound restored the next runs equal the
    eager forward computed before."""
    g, m = _tiny(ctx)
    try:
        V = g["config"][6]
        pos0 = 700   # past the split position: k_attn_g
        assert pos0 >= intllm.hip_lib().q48_attn_split_min()
        say("kv fill", pos0)
        m.kv_fill_synth(spec.SEED_KV, pos0, threads())
        n = 6
        _, want, _ = m.decode_from(1, pos0, n)
        ctx.set_attn_wait(0)
        try:
            for what, run in (("graph", lambda: m.decode_graph_hashed(1, pos0, n)),
                              ("graph, not hashed", lambda: m.decode_graph(1, pos0, n)),
                              ("eager", lambda: m.decode_from(1, pos0, n)),
                              ("forward", lambda: m.forward(1, pos0, V))):
                say("give-up run:", what)
                with pytest.raises(intllm.Q48Error) as e:
                    run()
                assert e.value.code == intllm.Q48_ETIMEOUT, what
        finally:
            ctx.set_attn_wait(-1)
        assert ctx.attn_status() == 0   # the error was read and cleared
        say("default bound")
        _, _, h, _ = m.decode_graph_hashed(1, pos0, n)
        assert h == ["%016x" % v for v in want]
        _, h2, _ = m.decode_from(1, pos0, n)
        assert h2 == want
    finally:
        m.free()
