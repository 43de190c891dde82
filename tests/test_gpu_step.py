"""The one-launch decode step (q48_step_fused, k_step_fused): every step's
logits hash and token against the reference's own generate on the
TinyLlama-1.1B-shape synthetic model (tests/golden/tinyllama_generate.json,
recorded from llama_int.c's llama_forward), for int64 and bfloat16-resident
weights, stepped one launch at a time and replayed from a captured graph."""
import os

import pytest

import intllm
import oracle_lib as O
import spec
from conftest import golden

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def threads():
    return max(1, min(16, os.cpu_count() or 1))


def _prefill(m, prompt):
    nxt = None
    for pos, tok in enumerate(prompt):
        nxt, _ = m.forward(tok, pos, spec.TINYLLAMA[6], logits=False)
    return nxt


@pytest.mark.parametrize("bf16", [pytest.param(False, id="int64"), pytest.param(True, id="bf16")])
def test_onelaunch_steps_match_reference(ctx, bf16):
    g = golden("tinyllama_generate.json")
    prompt, ref, fnv = g["prompt"], g["tokens"], g["step_fnv"]
    P = len(prompt)
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tinyllama synth", "bf16" if bf16 else "int64")
        m.synth(g["seed"], threads())
        if bf16:
            m.set_bf16(True)
        assert not m.onelaunch_active(P)   # opt-in
        m.set_onelaunch(True)
        assert m.onelaunch_active(P)
        tok = _prefill(m, prompt)
        assert tok == ref[P]
        # one launch per call (the first step of decode_graph runs eagerly):
        # the logits of every step against the reference's hash
        n1 = 12
        for i in range(n1):
            pos = P + i
            say("one-launch step", pos)
            _, steps, _ = m.decode_graph(tok, pos, 1)
            assert O.fnv(m.read_logits()) == fnv[pos], f"logits at pos {pos}"
            assert steps[0] == ref[pos + 1]
            tok = steps[0]
        # then replays of the captured one-launch step
        say("one-launch graph replay")
        n2 = 48 if not bf16 else 24
        _, steps, _ = m.decode_graph(tok, P + n1, n2)
        assert steps == ref[P + n1 + 1:P + n1 + 1 + n2]
        assert O.fnv(m.read_logits()) == fnv[P + n1 + n2 - 1]
    finally:
        m.free()


def test_onelaunch_off_and_on_agree_across_recapture(ctx):
    """The same decode through the fused launches (one-launch off) and through
    the one-launch step, switching between them on one model: each switch
    recaptures the step graph and the stream continues the reference's."""
    g = golden("tinyllama_generate.json")
    prompt, ref = g["prompt"], g["tokens"]
    P = len(prompt)
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tinyllama synth")
        m.synth(g["seed"], threads())
        tok = _prefill(m, prompt)
        pos = P
        for on in (False, True, False, True):
            m.set_onelaunch(on)
            assert m.onelaunch_active(pos) == on
            say("decode_graph onelaunch", on, "at", pos)
            _, steps, _ = m.decode_graph(tok, pos, 8)
            assert steps == ref[pos + 1:pos + 9]
            tok, pos = steps[-1], pos + 8
    finally:
        m.free()


def test_onelaunch_not_used_where_not_served(ctx):
    """Off by default; when on, shapes other than dim 2048 / ffn 5632 /
    head_dim 64, sampling, the other fused modes and positions from 512 on
    take the fused launches."""
    m = intllm.HostModel(ctx, intllm.Config(*spec.TINY))
    try:
        m.set_onelaunch(True)
        assert not m.onelaunch_active(0)
    finally:
        m.free()
    g = golden("tinyllama_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        assert not m.onelaunch_active(0)
        m.set_onelaunch(True)
        assert m.onelaunch_active(0) and m.onelaunch_active(511)
        assert not m.onelaunch_active(512)
        m.set_fused(2)
        assert not m.onelaunch_active(0)
        m.set_fused(3)
        m.set_sampling(int(0.8 * (1 << 48)), 40, int(0.9 * (1 << 48)), 1)
        assert not m.onelaunch_active(0)
    finally:
        m.free()
