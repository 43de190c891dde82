"""generate()'s stop branches against the reference (tests/golden/
generate_stops.json, written by the reference's own generate on the
config-1 model): EOS chosen in decode (not appended, llama_int.c:3111),
EOS as the prompt's final choice (appended, :3087-3090), the cache
reaching max_seq (llama_forward returns NULL, :2817-2820; decode breaks,
:3106) and a prompt longer than max_seq (the prefill fails).

Each case runs through the C host's generate (batched and per-token
prefill), the graph-replayed decode with every step's logits hashed, and
the reference-side binding (the reference's generate with llama_forward
on the device)."""
import os

import pytest

import intllm
from conftest import golden
from test_refbind import REFBIND_SO, RefModel, _lib

pytestmark = pytest.mark.gpu

CASES = [c["name"] for c in golden("generate_stops.json")["cases"]]


def say(*a):
    print("[case]", *a, flush=True)


def case(name):
    g = golden("generate_stops.json")
    return g["seed"], next(c for c in g["cases"] if c["name"] == name)


@pytest.mark.parametrize("batched", [True, False], ids=["batched_prefill", "token_prefill"])
@pytest.mark.parametrize("name", CASES)
def test_host_generate_stops(ctx, name, batched):
    seed, c = case(name)
    m = intllm.HostModel(ctx, intllm.Config(*c["config"]))
    try:
        say("stops host generate", name, "batched" if batched else "per-token")
        m.synth(seed, 4)
        m.set_batched_prefill(batched)
        if c["total"] < 0:
            # the prefill runs past max_seq: generate fails, as the
            # reference's returns -1 (Q48_ERANGE here)
            with pytest.raises(intllm.Q48Error) as e:
                m.generate(c["prompt"], c["max_new"])
            assert e.value.code == intllm.Q48_ERANGE
            return
        toks, hs, st = m.generate(c["prompt"], c["max_new"])
        assert len(toks) == c["total"]
        assert toks == c["tokens"]
        assert ["%016x" % h for h in hs] == c["step_fnv"]
        assert st.decode_tokens == c["total"] - len(c["prompt"]) - 1
    finally:
        m.free()


@pytest.mark.parametrize("name", [n for n in CASES if n != "prompt_past_max_seq"])
def test_graph_decode_stops(ctx, name):
    """The prompt by forward calls, then the decode replayed from a graph
    with every step's logits recorded on the device: the chosen tokens and
    the logits hashes of every step up to the stop."""
    seed, c = case(name)
    P = len(c["prompt"])
    m = intllm.HostModel(ctx, intllm.Config(*c["config"]))
    try:
        say("stops graph decode", name)
        m.synth(seed, 4)
        for pos, tok in enumerate(c["prompt"]):
            nxt, _ = m.forward(tok, pos, c["config"][6], logits=False)
        assert nxt == c["tokens"][P]
        decode_hashes = c["step_fnv"][P:]
        k, allt, hs, st = m.decode_graph_hashed(nxt, P, c["max_new"] - 1)
        ran = len(decode_hashes)
        assert len(k) == ran and st.decode_tokens == ran
        assert hs[:ran] == decode_hashes
        want = c["tokens"][P + 1:]
        if name == "eos_in_decode":
            assert k == want + [2]        # the step that chose EOS counts
        else:
            assert k == want
        if name == "max_seq":             # clipped at max_seq: no step past it
            assert len(allt) == c["config"][7] - P
        # the eager per-step loop agrees
        m.kv_reset()
        for pos, tok in enumerate(c["prompt"]):
            m.forward(tok, pos, c["config"][6], logits=False)
        toks2, hs2, _ = m.decode_from(nxt, P, c["max_new"] - 1)
        assert toks2 == k
        assert ["%016x" % h for h in hs2] == decode_hashes
    finally:
        m.free()


@pytest.mark.skipif(not REFBIND_SO.exists(), reason="refbind library not built")
@pytest.mark.parametrize("name", CASES)
def test_refbind_generate_stops(name):
    """The reference's own generate(), llama_forward on the device."""
    seed, c = case(name)
    lib = _lib()
    rm = RefModel(lib, c["config"], seed)
    try:
        say("stops refbind generate", name)
        assert lib.lq48_attach(rm.m, 0) == 0
        total, toks, hs = rm.generate(c["prompt"], c["max_new"])
        assert total == c["total"]
        if total >= 0:
            assert toks == c["tokens"]
            assert hs == c["step_fnv"]
        lib.lq48_detach()
    finally:
        rm.free()
