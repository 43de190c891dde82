"""End-to-end GPU parity: the C host's generate loop over libintllm_hip
against the token streams and per-step logits hashes recorded from the
reference's own llama_forward / generate (tests/golden/*_generate.json,
longctx_decode.json)."""
import ctypes as C
import os
import tempfile

import numpy as np
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


def test_tiny_generate_bit_exact(ctx):
    g = golden("tiny_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tiny synth")
        m.synth(g["seed"], threads())
        say("tiny generate")
        toks, hs, _ = m.generate(g["prompt"], g["max_new"])
        assert toks == g["tokens"]
        assert ["%016x" % h for h in hs] == g["step_fnv"]
        # determinism: a second run (kv reset inside generate) is identical
        toks2, hs2, _ = m.generate(g["prompt"], g["max_new"])
        assert toks2 == toks and hs2 == hs
    finally:
        m.free()


def test_tiny_forward_logits_equal_oracle(ctx):
    g = golden("tiny_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    om = O.Model(spec.TINY, g["seed"])
    try:
        m.synth(g["seed"], threads())
        for pos, tok in enumerate(g["prompt"][:6]):
            say("tiny forward pos", pos)
            nxt, lg = m.forward(tok, pos, spec.TINY[6])
            rc, want = om.forward(tok, pos)
            assert rc == 0 and np.array_equal(lg, want), pos
            assert nxt == int(np.argmax(want))
    finally:
        m.free()
        om.free()


def test_forward_range_errors(ctx):
    m = intllm.HostModel(ctx, intllm.Config(*spec.TINY))
    try:
        for tok, pos in ((spec.TINY[6], 0), (-1, 0), (3, spec.TINY[7])):
            with pytest.raises(intllm.Q48Error) as e:
                m.forward(tok, pos, spec.TINY[6])
            assert e.value.code == intllm.Q48_ERANGE
    finally:
        m.free()


def test_mgw_roundtrip_bit_exact(ctx):
    """A .mgw written in mgw_export's layout loads through mgw_load's checks
    and generates the reference token stream."""
    g = golden("tiny_generate.json")
    cfg = intllm.Config(*g["config"])
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.mgw")
        say("mgw write")
        intllm.check("q48h_mgw_write_synth", intllm.host_lib().q48h_mgw_write_synth(
            path.encode(), C.byref(cfg), g["seed"], threads()))
        say("mgw load")
        m = intllm.HostModel(ctx, mgw=path)
        try:
            toks, hs, _ = m.generate(g["prompt"], g["max_new"])
            assert toks == g["tokens"]
            assert ["%016x" % h for h in hs] == g["step_fnv"]
        finally:
            m.free()
        # a truncated file is rejected, not read past its end
        with open(path, "rb") as f:
            data = f.read()
        bad = os.path.join(d, "bad.mgw")
        with open(bad, "wb") as f:
            f.write(data[: len(data) // 2])
        with pytest.raises(intllm.Q48Error):
            intllm.HostModel(ctx, mgw=bad)


def test_tinyllama_generate_bit_exact(ctx):
    """Config 3: TinyLlama-1.1B shape, 32-token prompt, 128 greedy tokens."""
    g = golden("tinyllama_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tinyllama synth (8.8 GB)")
        m.synth(g["seed"], threads())
        say("tinyllama generate")
        toks, hs, st = m.generate(g["prompt"], g["max_new"])
        assert toks == g["tokens"]
        assert ["%016x" % h for h in hs] == g["step_fnv"]
        print(f"decode {1e3 * st.decode_s / max(1, st.decode_tokens):.3f} ms/tok", flush=True)
    finally:
        m.free()


def test_long_context_decode_bit_exact(ctx):
    """Config 5: KV pre-filled to 2048 positions, 256 greedy decode steps."""
    g = golden("longctx_decode.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("longctx synth + kv fill")
        m.synth(g["seed"], threads())
        m.kv_fill_synth(g["kv_seed"], g["prefill"], threads())
        say("longctx decode")
        toks, hs, st = m.decode_from(g["start_token"], g["prefill"], spec.LONG_STEPS)
        assert toks == g["tokens"]
        assert ["%016x" % h for h in hs] == g["step_fnv"]
    finally:
        m.free()


def test_long_context_graph_decode_bit_exact(ctx):
    """Config 5 through a graph captured at position 2048 (split attention),
    then a short-context graph decode on the same model: the step graph is
    recaptured whenever attention changes kernels, and both streams match
    the reference's, tokens and every replayed step's logits hash (all 256
    config-5 steps)."""
    g = golden("longctx_decode.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("longctx synth + kv fill")
        m.synth(g["seed"], threads())
        m.kv_fill_synth(g["kv_seed"], g["prefill"], threads())
        say("longctx graph decode, all", g["steps"], "steps hashed")
        _, toks, hs, _ = m.decode_graph_hashed(g["start_token"], g["prefill"], g["steps"])
        assert toks == g["tokens"]
        assert hs == g["step_fnv"]
        # back to the start of the cache: the graph drops back to one-block attention
        gt = golden("tinyllama_generate.json")
        assert gt["seed"] == g["seed"]
        for pos, tok in enumerate(gt["prompt"]):
            nxt, _ = m.forward(tok, pos, spec.TINYLLAMA[6], logits=False)
        say("short graph decode after long")
        P = len(gt["prompt"])
        _, toks2, hs2, _ = m.decode_graph_hashed(nxt, P, 8)
        ref = gt["tokens"][P:]
        assert [nxt] + toks2[:7] == ref[:8]
        assert hs2 == gt["step_fnv"][P:P + 8]
    finally:
        m.free()


@pytest.mark.parametrize("kernel", [pytest.param(intllm.GEMM_VALU, id="valu"),
                                    pytest.param(intllm.GEMM_I8, id="i8")])
@pytest.mark.parametrize("T", spec.GEMM_TOKENS)
def test_gemm_config4_vs_reference(ctx, T, kernel):
    g = golden("gemm.json")["shapes"]
    for (N, K) in spec.GEMV_SHAPES:
        W = O.synth(spec.gemv_w_name(N, K), N, K, spec.SEED_GEMV, spec.SIGMA_W, 1)
        X = O.synth(spec.gemm_x_name(T, K), T, K, spec.SEED_GEMV, spec.SIGMA_ACT, 0)
        dW, dX, dY = ctx.to_device(W), ctx.to_device(X), ctx.buffer(T * N)
        say("gemm config4", T, N, K, "kernel", kernel)
        ctx.gemm(dY.ptr, dW.ptr, dX.ptr, T, N, K, kernel)
        assert O.fnv(dY.download()) == g[f"{T}x{N}x{K}"]["fnv"], (T, N, K)
        for b in (dW, dX, dY):
            b.free()


@pytest.mark.parametrize("mode", [0, 1, 2, "noprefetch"])
def test_tiny_generate_other_paths_bit_exact(ctx, mode):
    """One library op per reference step (0), the per-block-statistics
    fusion (1), the producer-statistics fusion (2) and the default path
    without the W_o prefetch give the same stream as the default path
    (partial sums finished by the consumer, prefetch on)."""
    g = golden("tiny_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        m.synth(g["seed"], threads())
        if mode == "noprefetch":
            m.set_prefetch(False)
        else:
            m.set_fused(mode)
        say("tiny generate mode", mode)
        toks, hs, _ = m.generate(g["prompt"], g["max_new"])
        assert toks == g["tokens"]
        assert ["%016x" % h for h in hs] == g["step_fnv"]
    finally:
        m.free()


def test_graph_decode_across_split_position(ctx, oracle):
    """A graph-replayed run that crosses q48_attn_split_min() (256), where
    attention changes kernels (one block per head below it, split attention
    from it on): the run is replayed from two captured graphs and equals the
    eager per-token decode and the oracle's decode."""
    g = golden("tiny_generate.json")
    cfg = intllm.Config(*g["config"])
    split = intllm.hip_lib().q48_attn_split_min()
    start, n, tok0 = split - 12, 24, 7
    m = intllm.HostModel(ctx, cfg)
    try:
        m.synth(g["seed"], threads())
        m.kv_fill_synth(spec.SEED_KV, start, threads())
        say("graph decode across", split)
        _, steps, _ = m.decode_graph(tok0, start, n)
        say("eager decode across", split)
        eager, _, _ = m.decode_from(tok0, start, n, hashes=False)
    finally:
        m.free()
    ocfg = O.Config(*g["config"])
    om = oracle.q48o_model_synth(C.byref(ocfg), g["seed"], threads())
    try:
        oracle.q48o_kv_fill_synth(om, spec.SEED_KV, start, threads())
        out = (C.c_int * n)()
        k = oracle.q48o_decode_from(om, tok0, start, n, out, None)
        ref = list(out[:k])
    finally:
        oracle.q48o_model_free(om)
    assert eager[:k] == ref
    assert steps[:k] == ref


def test_tiny_graph_decode_replays(ctx):
    """Graph-replayed decode: several launches of the captured step, with
    eager work and host synchronisation between the calls, each continuing
    the token stream exactly where the eager generate has it."""
    g = golden("tiny_generate.json")
    prompt, ref = g["prompt"], g["tokens"]
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        m.synth(g["seed"], threads())
        for pos, tok in enumerate(prompt):          # eager prefill
            nxt, _ = m.forward(tok, pos, spec.TINY[6], logits=False)
        assert nxt == ref[len(prompt)]
        tok, pos, got = nxt, len(prompt), [nxt]
        for chunk in (5, 9, 10):
            say("graph decode chunk", chunk, "from pos", pos)
            _, steps, hs, _ = m.decode_graph_hashed(tok, pos, chunk)
            assert hs == g["step_fnv"][pos:pos + chunk]
            got += steps
            tok, pos = steps[-1], pos + chunk
            ctx.sync()
            # eager work between replays: a forward whose result must also agree
            _, lg = m.forward(tok, pos, spec.TINY[6])
            got_next = int(np.argmax(lg))
            _, steps1, _ = m.decode_graph(tok, pos, 1)
            assert steps1[0] == got_next
        n = min(len(got), len(ref) - len(prompt))
        assert got[:n] == ref[len(prompt):len(prompt) + n]
    finally:
        m.free()


def test_tinyllama_graph_decode_bit_exact(ctx):
    g = golden("tinyllama_generate.json")
    prompt, ref = g["prompt"], g["tokens"]
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tinyllama synth")
        m.synth(g["seed"], threads())
        for pos, tok in enumerate(prompt):
            nxt, _ = m.forward(tok, pos, spec.TINYLLAMA[6], logits=False)
        say("tinyllama graph decode, every step hashed")
        P = len(prompt)
        toks, steps, hs, st = m.decode_graph_hashed(nxt, P, g["max_new"] - 1)
        assert [nxt] + toks[:len(ref) - P - 1] == ref[P:]
        assert hs == g["step_fnv"][P:]
        print(f"graph decode {1e3 * st.decode_s / max(1, st.decode_tokens):.3f} ms/tok", flush=True)
    finally:
        m.free()


def test_tinyllama_bf16_weights_bit_exact(ctx):
    """Config 3 with the projection matrices and lm_head read as bfloat16 bits
    (2 bytes per weight): the same 128-token stream and per-step logits
    hashes as the reference, eager and graph-replayed."""
    g = golden("tinyllama_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        say("tinyllama synth, bf16 pack")
        m.synth(g["seed"], threads())
        m.set_bf16(True)
        say("tinyllama bf16 generate")
        toks, hs, _ = m.generate(g["prompt"], g["max_new"])
        assert toks == g["tokens"]
        assert ["%016x" % h for h in hs] == g["step_fnv"]
        prompt, ref = g["prompt"], g["tokens"]
        for pos, tok in enumerate(prompt):
            nxt, _ = m.forward(tok, pos, spec.TINYLLAMA[6], logits=False)
        say("tinyllama bf16 graph decode, every step hashed")
        P = len(prompt)
        toks2, _, hs2, _ = m.decode_graph_hashed(nxt, P, 32)
        assert [nxt] + toks2[:31] == ref[P:P + 32]
        assert hs2 == g["step_fnv"][P:P + 32]
    finally:
        m.free()


def test_bf16_weights_refused_when_not_applicable(ctx):
    """The tiny model (dim 256) has no bfloat16 GEMV shape, and weights that
    are not bfloat16 values cannot be packed: both refuse, and the model
    keeps decoding with its int64 weights."""
    g = golden("tiny_generate.json")
    m = intllm.HostModel(ctx, intllm.Config(*g["config"]))
    try:
        m.synth(g["seed"], threads())
        with pytest.raises(intllm.Q48Error):
            m.set_bf16(True)
        toks, _, _ = m.generate(g["prompt"], g["max_new"])
        assert toks == g["tokens"]
    finally:
        m.free()
    cfg = intllm.config(intllm.TINY, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024,
                        vocab=512, n_layers=1)
    m = intllm.HostModel(ctx, cfg)
    try:
        m.synth(3, threads())
        m.set_bf16(True)      # synthetic weights are bfloat16 values
        m.set_bf16(False)
        wo = np.full(512 * 512, 0x123456789, dtype=np.int64)
        m.upload("model.layers.0.self_attn.o_proj.weight", wo)
        with pytest.raises(intllm.Q48Error):
            m.set_bf16(True)
    finally:
        m.free()
