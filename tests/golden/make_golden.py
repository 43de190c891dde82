#!/usr/bin/env python3
"""Write the golden vectors under tests/golden/ from the REAL reference.

Runs only in the build container, where /root/reference exists: it loads
oracle/_ref/libq48_ref.so (built by `make -C oracle ref` from the
reference's own llama_int.c / fp_determinism.c, see oracle/ref_harness.c)
and records what the reference computes on the synthetic inputs of
int-llm_amd/host/q48_synth.h.  The JSON files it writes are data (inputs,
seeds and outputs or their FNV-1a-64 hashes); the GPU box never runs this.

    python tests/golden/make_golden.py fp gemv ops tiny      # seconds
    python tests/golden/make_golden.py tinyllama longctx gemm  # minutes
"""
from __future__ import annotations

import ctypes as C
import json
import os
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
GOLD = Path(__file__).resolve().parent
REF_SO = ROOT / "oracle" / "_ref" / "libq48_ref.so"
REF_DET = ROOT / "oracle" / "_ref" / "fp_determinism"

sys.path.insert(0, str(ROOT / "tests"))
import spec  # noqa: E402  (shared fixture definitions)

FNV_OFF = 1469598103934665603


class RefCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in
                ("dim", "n_heads", "n_kv_heads", "head_dim", "n_layers", "ffn",
                 "vocab", "max_seq", "rope_theta")]


def ref():
    if not REF_SO.exists():
        subprocess.check_call(["make", "-C", str(ROOT / "oracle"), "ref"])
    lib = C.CDLL(str(REF_SO))
    P, I, U = C.c_void_p, C.c_int, C.c_uint64
    sig = {
        "q48r_gemv": ([P, P, P, I, I], None),
        "q48r_rmsnorm": ([P, P, P, I], None),
        "q48r_softmax": ([P, I], None),
        "q48r_rope_tables": ([P, P, I, I, I], None),
        "q48r_rope_apply": ([P, P, I, I, P, I], None),
        "q48r_model_synth": ([C.POINTER(RefCfg), U, I], P),
        "q48r_model_free": ([P], None),
        "q48r_kv_fill_synth": ([P, U, I, I], None),
        "q48r_kv_reset": ([P], None),
        "q48r_layer_forward": ([P, I, I, P], None),
        "q48r_forward": ([P, I, I, P], I),
        "q48r_generate": ([P, P, I, I, P, P, P], I),
        "q48r_generate_tokens": ([P, P, I, I, P], I),
        "q48r_decode_from": ([P, I, I, I, P, P], I),
        "q48s_fill": ([P, C.c_int64, C.c_int64, U, C.c_int64, I, I], None),
        "q48s_tensor_seed": ([U, C.c_char_p], U),
        "q48s_tokens": ([P, I, U, I, I], None),
        "q48s_fnv_i64": ([U, P, C.c_size_t], U),
        "q48r_bf16_to_q48": ([C.c_uint16], C.c_int64),
        "q48r_f16_to_q48": ([C.c_uint16], C.c_int64),
        "q48r_rng_seed": ([U, P], None),
        "q48r_rng_next": ([P], U),
        "q48r_sample": ([P, I, C.c_int64, I, C.c_int64, P], I),
        "q48r_generate_sampled": ([P, P, I, I, P, C.c_int64, I, C.c_int64, U], I),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = args, res
    for name in ("q48r_fp_mul", "q48r_fp_div"):
        f = getattr(lib, name)
        f.argtypes, f.restype = [C.c_int64, C.c_int64], C.c_int64
    for name in ("q48r_fp_inv_sqrt", "q48r_fp_exp", "q48r_fp_safe_exp", "q48r_fp_log",
                 "q48r_fp_sqrt", "q48r_fp_sigmoid", "q48r_fp_silu"):
        f = getattr(lib, name)
        f.argtypes, f.restype = [C.c_int64], C.c_int64
    lib.q48r_fp_sincos.argtypes = [C.c_int64, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
    lib.q48r_fp_consts.argtypes = [C.POINTER(C.c_int64)] * 3
    return lib


def fnv(arr: np.ndarray) -> str:
    a = np.ascontiguousarray(arr, dtype=np.int64)
    return "%016x" % R.q48s_fnv_i64(FNV_OFF, a.ctypes.data, a.size)


def synth(name: str, rows: int, cols: int, seed: int, sigma: int, bf16: int) -> np.ndarray:
    a = np.empty(rows * cols, dtype=np.int64)
    R.q48s_fill(a.ctypes.data, rows, cols, R.q48s_tensor_seed(seed, name.encode()),
                sigma, bf16, os.cpu_count() or 4)
    return a


def write(name: str, obj) -> None:
    (GOLD / name).write_text(json.dumps(obj, indent=1) + "\n")
    print("wrote", name, flush=True)


# ---------------------------------------------------------------------------

def gen_fp():
    out = subprocess.run([str(REF_DET)], capture_output=True, text=True, check=True).stdout
    kv = dict(line.split("=", 1) for line in out.splitlines() if "=" in line)
    subs = {k[4:]: v for k, v in kv.items() if k.startswith("sub:")}
    pi, gain = C.c_int64(), C.c_int64()
    ang = (C.c_int64 * 48)()
    R.q48r_fp_consts(C.byref(pi), C.byref(gain), ang)
    golden = (Path("/root/reference/tests/determinism_golden.txt").read_text().split()[0])
    # per-function vectors on the inputs of spec.fp_inputs (edge values too)
    x, y = spec.fp_inputs()
    vec = {}
    vec["mul"] = fnv(np.array([R.q48r_fp_mul(int(a), int(b)) for a, b in zip(x, y)]))
    vec["div"] = fnv(np.array([R.q48r_fp_div(int(a), int(b)) if b != 0 else 0
                               for a, b in zip(x, y)]))
    pos = np.array([spec.pos_of(int(a)) for a in x], dtype=np.int64)
    for nm in ("inv_sqrt", "sqrt", "log"):
        f = getattr(R, "q48r_fp_" + nm)
        vec[nm] = fnv(np.array([f(int(a)) for a in pos]))
    e = np.array([spec.exp_arg(int(a)) for a in x], dtype=np.int64)
    vec["exp"] = fnv(np.array([R.q48r_fp_exp(int(a)) for a in e]))
    vec["safe_exp"] = fnv(np.array([R.q48r_fp_safe_exp(int(a)) for a in e]))
    c, s = C.c_int64(), C.c_int64()
    cs, ss = [], []
    for a in x:
        R.q48r_fp_sincos(int(a), C.byref(c), C.byref(s))
        cs.append(c.value)
        ss.append(s.value)
    vec["cos"], vec["sin"] = fnv(np.array(cs)), fnv(np.array(ss))
    vec["sigmoid"] = fnv(np.array([R.q48r_fp_sigmoid(int(a)) for a in x]))
    vec["silu"] = fnv(np.array([R.q48r_fp_silu(int(a)) for a in x]))
    write("fp.json", {
        "source": "fp_determinism.c (compiled from /root/reference) and fp_math.h via oracle/ref_harness.c",
        "determinism_golden": golden,
        "determinism_hash": kv["DETERMINISM_HASH"],
        "grid_inputs": int(kv["grid_inputs"]),
        "sub_hashes": subs,
        "consts": {"pi": pi.value, "gain": gain.value, "angles": list(ang)},
        "vectors": {"inputs": "spec.fp_inputs()", "fnv": vec},
    })


def ref_gemv(W, x, M, K):
    y = np.empty(M, dtype=np.int64)
    R.q48r_gemv(y.ctypes.data, W.ctypes.data, x.ctypes.data, M, K)
    return y


def gen_gemv():
    shapes = {}
    for (M, K) in spec.GEMV_SHAPES:
        W, x = spec.gemv_inputs_ref(synth, M, K)
        t = time.time()
        y = ref_gemv(W, x, M, K)
        shapes[f"{M}x{K}"] = {"fnv": fnv(y), "head": [int(v) for v in y[:4]],
                              "ref_cpu_s": round(time.time() - t, 4)}
    edges = []
    for (M, K, W, x) in spec.gemv_edge_cases():
        y = ref_gemv(W, x, M, K)
        edges.append({"M": M, "K": K, "W": [int(v) for v in W], "x": [int(v) for v in x],
                      "y": [int(v) for v in y]})
    write("gemv.json", {
        "source": "matmul_vec (llama_int.c:1014-1046) via oracle/ref_harness.c",
        "inputs": "spec.gemv_inputs: W sigma 0.02 bf16-rounded, x sigma 1 raw Q16.48",
        "shapes": shapes, "edges": edges})


def gen_ops():
    out = {"source": "rmsnorm / rope_init / rope_apply / softmax / transformer_layer_forward "
                     "(llama_int.c) via oracle/ref_harness.c"}
    # rmsnorm
    rms = {}
    for dim in (256, 2048, 688, 7):
        x, w = spec.rmsnorm_inputs(synth, dim)
        o = np.empty(dim, dtype=np.int64)
        R.q48r_rmsnorm(o.ctypes.data, x.ctypes.data, w.ctypes.data, dim)
        rms[str(dim)] = fnv(o)
    out["rmsnorm"] = rms
    # rope tables
    rope = {}
    for (hd, ms, th) in spec.ROPE_TABLES:
        n = ms * (hd // 2)
        c = np.empty(n, dtype=np.int64)
        s = np.empty(n, dtype=np.int64)
        R.q48r_rope_tables(c.ctypes.data, s.ctypes.data, hd, ms, th)
        rope[f"{hd}x{ms}x{th}"] = {"cos": fnv(c), "sin": fnv(s),
                                  "cos_head": [int(v) for v in c[:8]],
                                  "sin_head": [int(v) for v in s[:8]]}
        if (hd, ms) == (32, 64):
            # rope_apply on one vector at every position
            v0 = synth("rope.vec", 1, hd, spec.SEED_OPS, spec.SIGMA_ACT, 0)
            res = []
            for pos in range(ms):
                v = v0.copy()
                R.q48r_rope_apply(c.ctypes.data, s.ctypes.data, hd // 2, ms, v.ctypes.data, pos)
                res.append(fnv(v))
            rope[f"{hd}x{ms}x{th}"]["apply"] = res
    out["rope"] = rope
    # softmax
    sm = {}
    for n in (1, 5, 64, 2049):
        x = spec.softmax_inputs(synth, n)
        R.q48r_softmax(x.ctypes.data, n)
        sm[str(n)] = fnv(x)
    out["softmax"] = sm
    write("ops.json", out)


def model(cfg: RefCfg, seed: int):
    return R.q48r_model_synth(C.byref(cfg), seed, os.cpu_count() or 4)


def gen_layer():
    """One transformer layer (attention + SwiGLU) at several positions."""
    cfg = RefCfg(*spec.TINY)
    m = model(cfg, spec.SEED_TINY)
    res = []
    h = synth("layer.hidden", 1, cfg.dim, spec.SEED_OPS, spec.SIGMA_W, 1)
    for pos in range(40):
        R.q48r_layer_forward(m, 0, pos, h.ctypes.data)
        res.append(fnv(h))
    R.q48r_model_free(m)
    write("layer.json", {"source": "transformer_layer_forward (llama_int.c:1326-1569)",
                         "config": list(spec.TINY), "seed": spec.SEED_TINY,
                         "hidden_fnv_per_pos": res})


def run_generate(cfg_t, seed, prompt, max_new):
    cfg = RefCfg(*cfg_t)
    t = time.time()
    m = model(cfg, seed)
    t_synth = time.time() - t
    cap = len(prompt) + max_new + 1
    p = (C.c_int * len(prompt))(*prompt)
    out = (C.c_int * cap)()
    hs = (C.c_uint64 * cap)()
    n = C.c_int()
    t = time.time()
    total = R.q48r_generate(m, p, len(prompt), max_new, out, hs, C.byref(n))
    t_gen = time.time() - t
    toks = list(out[:total])
    # the reference's own generate() must give the same stream
    out2 = (C.c_int * cap)()
    same = None
    if cfg.n_layers <= 2:
        total2 = R.q48r_generate_tokens(m, p, len(prompt), max_new, out2)
        same = list(out2[:total2]) == toks
    R.q48r_model_free(m)
    return toks, ["%016x" % v for v in hs[:n.value]], same, t_synth, t_gen


def gen_tiny():
    prompt = spec.prompt(spec.SEED_TINY, 16, spec.TINY[6])
    toks, hs, same, ts, tg = run_generate(spec.TINY, spec.SEED_TINY, prompt, 32)
    assert same, "generate() and the hashed loop disagree"
    write("tiny_generate.json", {
        "source": "generate (llama_int.c:3067-3135) via oracle/ref_harness.c",
        "config": list(spec.TINY), "seed": spec.SEED_TINY, "prompt": prompt,
        "max_new": 32, "tokens": toks, "step_fnv": hs})


def gen_stops():
    """generate()'s stop branches on the config-1 model (llama_int.c:3067-3135):
    a decode that chooses EOS (id 2; not appended, :3111), a prompt whose
    final choice is EOS (appended anyway, :3087-3090, and decoding goes on
    from it), a run that reaches max_seq (llama_forward returns NULL,
    :2817-2820, and decode breaks, :3106) and a prompt longer than max_seq
    (the prefill fails: generate returns -1).  Prompts are searched with
    the reference itself over prompt seeds SEED_TINY + i."""
    vocab = spec.TINY[6]
    cases = []

    def run(cfg_t, prompt, max_new):
        toks, hs, same, _, _ = run_generate(cfg_t, spec.SEED_TINY, prompt, max_new)
        assert same, "generate() and the hashed loop disagree"
        return toks, hs

    cfg = RefCfg(*spec.TINY)
    m = model(cfg, spec.SEED_TINY)
    cap = 64
    out = (C.c_int * cap)()
    hs = (C.c_uint64 * cap)()
    n = C.c_int()
    eos_decode = eos_prompt = None
    for i in range(1, 20000):
        if eos_decode is not None and eos_prompt is not None:
            break
        prompt = spec.prompt(spec.SEED_TINY + i, 16, vocab)
        p = (C.c_int * 16)(*prompt)
        if eos_prompt is None:
            total = R.q48r_generate(m, p, 16, 1, out, hs, C.byref(n))
            if total == 17 and out[16] == 2:
                eos_prompt = i
        if eos_decode is None:
            total = R.q48r_generate(m, p, 16, 32, out, hs, C.byref(n))
            if 17 < total < 48:
                eos_decode = i
    R.q48r_model_free(m)
    assert eos_decode is not None and eos_prompt is not None
    for name, i, max_new in (("eos_in_decode", eos_decode, 32),
                             ("eos_as_prompt_choice", eos_prompt, 32)):
        prompt = spec.prompt(spec.SEED_TINY + i, 16, vocab)
        toks, h = run(spec.TINY, prompt, max_new)
        cases.append({"name": name, "config": list(spec.TINY), "prompt_seed": spec.SEED_TINY + i,
                      "prompt": prompt, "max_new": max_new, "total": len(toks),
                      "tokens": toks, "step_fnv": h})
    short = list(spec.TINY)
    short[7] = 24                       # max_position_embeddings
    prompt = spec.prompt(spec.SEED_TINY, 16, vocab)
    toks, h = run(tuple(short), prompt, 32)
    cases.append({"name": "max_seq", "config": list(short), "prompt_seed": spec.SEED_TINY,
                  "prompt": prompt, "max_new": 32, "total": len(toks), "tokens": toks,
                  "step_fnv": h})
    short[7] = 12
    cfg = RefCfg(*short)
    m = model(cfg, spec.SEED_TINY)
    p = (C.c_int * 16)(*prompt)
    total = R.q48r_generate_tokens(m, p, 16, 32, out)
    R.q48r_model_free(m)
    cases.append({"name": "prompt_past_max_seq", "config": list(short),
                  "prompt_seed": spec.SEED_TINY, "prompt": prompt, "max_new": 32,
                  "total": total})
    write("generate_stops.json", {
        "source": "generate (llama_int.c:3067-3135) via oracle/ref_harness.c; "
                  "weights seed SEED_TINY", "seed": spec.SEED_TINY, "cases": cases})


def gen_bf16():
    """bfloat16_to_q1648 (safetensors.h:115-152) of all 65536 bit patterns,
    as the reference computes it: the values of the normal range follow
    from the formula; the exponent-255 clamp, shifts of 64 bits or more
    and left-shift wrap are the reference's conventions."""
    vals = np.array([R.q48r_bf16_to_q48(b) for b in range(65536)], dtype=np.int64)
    np.savez_compressed(GOLD / "bf16_to_q48.npz", v=vals)
    write("bf16_to_q48.json", {
        "source": "bfloat16_to_q1648 (safetensors.h:115-152) via oracle/ref_harness.c",
        "file": "bf16_to_q48.npz", "n": 65536, "fnv": fnv(vals)})


def gen_f16():
    """float16_to_q1648 (safetensors.h:74-111) of all 65536 bit patterns, as
    the reference computes them (subnormals, the exponent-31 clamp and the
    wrapping shift at exponent 30 included)."""
    vals = np.array([R.q48r_f16_to_q48(b) for b in range(65536)], dtype=np.int64)
    np.savez_compressed(GOLD / "f16_to_q48.npz", v=vals)
    write("f16_to_q48.json", {
        "source": "float16_to_q1648 (safetensors.h:74-111) via oracle/ref_harness.c",
        "file": "f16_to_q48.npz", "n": 65536, "fnv": fnv(vals)})


def gen_tinyllama():
    prompt = spec.prompt(spec.SEED_TL, 32, spec.TINYLLAMA[6])
    toks, hs, _, ts, tg = run_generate(spec.TINYLLAMA, spec.SEED_TL, prompt, 128)
    write("tinyllama_generate.json", {
        "source": "generate (llama_int.c:3067-3135) via oracle/ref_harness.c",
        "config": list(spec.TINYLLAMA), "seed": spec.SEED_TL, "prompt": prompt,
        "max_new": 128, "tokens": toks, "step_fnv": hs,
        "ref_cpu_s": {"synth": round(ts, 1), "generate": round(tg, 1),
                      "forward_calls": len(hs)}})


def gen_longctx():
    cfg = RefCfg(*spec.LONGCTX)
    t = time.time()
    m = model(cfg, spec.SEED_TL)
    R.q48r_kv_fill_synth(m, spec.SEED_KV, spec.LONG_PREFILL, os.cpu_count() or 4)
    ts = time.time() - t
    n = spec.LONG_STEPS
    out = (C.c_int * n)()
    hs = (C.c_uint64 * n)()
    t = time.time()
    steps = R.q48r_decode_from(m, spec.LONG_TOKEN, spec.LONG_PREFILL, n, out, hs)
    tg = time.time() - t
    R.q48r_model_free(m)
    write("longctx_decode.json", {
        "source": "llama_forward (llama_int.c:2807-2886) + argmax over a pre-filled "
                  "kv_cache_t via oracle/ref_harness.c",
        "config": list(spec.LONGCTX), "seed": spec.SEED_TL, "kv_seed": spec.SEED_KV,
        "prefill": spec.LONG_PREFILL, "start_token": spec.LONG_TOKEN, "steps": steps,
        "tokens": list(out[:steps]), "step_fnv": ["%016x" % v for v in hs[:steps]],
        "ref_cpu_s": {"setup": round(ts, 1), "decode": round(tg, 1)}})


def gen_gemm():
    res = {}
    for (N, K) in spec.GEMV_SHAPES:
        W = synth(spec.gemv_w_name(N, K), N, K, spec.SEED_GEMV, spec.SIGMA_W, 1)
        for T in spec.GEMM_TOKENS:
            X = synth(spec.gemm_x_name(T, K), T, K, spec.SEED_GEMV, spec.SIGMA_ACT, 0)
            Y = np.empty((T, N), dtype=np.int64)
            t = time.time()

            def rows(t0, t1):
                for t_ in range(t0, t1):
                    R.q48r_gemv(Y[t_].ctypes.data, W.ctypes.data, X[t_ * K:].ctypes.data, N, K)

            nt = os.cpu_count() or 4
            with ThreadPoolExecutor(nt) as ex:
                list(ex.map(lambda i: rows(T * i // nt, T * (i + 1) // nt), range(nt)))
            res[f"{T}x{N}x{K}"] = {"fnv": fnv(Y), "ref_cpu_s_{}threads".format(nt):
                                   round(time.time() - t, 2)}
            print(T, N, K, res[f"{T}x{N}x{K}"], flush=True)
    write("gemm.json", {"source": "matmul_vec per token (llama_int.c:1014-1046, "
                                  "sequential prefill 3081-3092) via oracle/ref_harness.c",
                        "inputs": "W as gemv.json, X[T][K] sigma 1 raw Q16.48",
                        "shapes": res})


def sample_cases():
    """The sampling grid: every parameter combination on 512 logits of each
    kind, and a subset on 32000 (the TinyLlama vocabulary)."""
    cases = []
    for kind in spec.SAMPLE_KINDS:
        for ti, T in enumerate(spec.SAMPLE_TEMPS):
            for ki, k in enumerate(spec.SAMPLE_TOPK):
                for pi, p in enumerate(spec.SAMPLE_TOPP):
                    seed = 1000 * ti + 100 * ki + 10 * pi + spec.SAMPLE_KINDS.index(kind)
                    cases.append((kind, seed, 512, T, 511 if k is None else k, p))
                    if kind in ("gauss", "ties") and ti in (3, 5) and ki in (0, 4) and pi in (0, 3, 4):
                        cases.append((kind, seed, 32000, T, 31999 if k is None else k, p))
    return cases


def gen_sample():
    # rng_seed / rng_next streams
    rng = {}
    for seed in (0, 1, 42, 0x9E3779B97F4A7C15, 2**64 - 1):
        s = (C.c_uint64 * 2)()
        R.q48r_rng_seed(seed, s)
        st = ["%016x" % s[0], "%016x" % s[1]]
        rng[str(seed)] = {"state": st, "next": ["%016x" % R.q48r_rng_next(s) for _ in range(8)]}
    out = []
    t = time.time()
    for (kind, seed, n, T, k, p) in sample_cases():
        x = spec.sample_logits(kind, seed, n)
        s = (C.c_uint64 * 2)()
        R.q48r_rng_seed(seed * 7919 + 1, s)
        s_in = [s[0], s[1]]
        tok = R.q48r_sample(x.ctypes.data, n, T, k, p, s)
        out.append({"kind": kind, "seed": seed, "n": n, "T": T, "top_k": k, "top_p": p,
                    "rng_in": ["%016x" % v for v in s_in], "token": tok,
                    "rng_out": ["%016x" % s[0], "%016x" % s[1]]})
    print(f"  {len(out)} sample_token cases in {time.time() - t:.1f}s", flush=True)
    # generate() with sampling, tiny model
    gens = []
    prompt = spec.prompt(spec.SEED_TINY, 16, spec.TINY[6])
    cfg = RefCfg(*spec.TINY)
    m = model(cfg, spec.SEED_TINY)
    for (T, k, p, seed) in spec.SAMPLE_GEN:
        cap = len(prompt) + 32 + 1
        pr = (C.c_int * len(prompt))(*prompt)
        o = (C.c_int * cap)()
        total = R.q48r_generate_sampled(m, pr, len(prompt), 32, o, T, k, p, seed)
        gens.append({"T": T, "top_k": k, "top_p": p, "seed": seed, "tokens": list(o[:total])})
    R.q48r_model_free(m)
    write("sample.json", {
        "source": "rng_seed / rng_next / sample_token / generate(sp) "
                  "(llama_int.c:2909-2929, 2958-3039, 3067-3135) via oracle/ref_harness.c",
        "logits": "tests/spec.py sample_logits(kind, seed, n); rng_in = rng_seed(seed * 7919 + 1)",
        "rng": rng, "cases": out,
        "generate_tiny": {"config": list(spec.TINY), "seed": spec.SEED_TINY,
                          "prompt": prompt, "max_new": 32, "runs": gens}})


def gen_sample_tl():
    """generate() with sampling on the TinyLlama-shape model (config 3):
    32-token prompt, 16 sampled tokens."""
    prompt = spec.prompt(spec.SEED_TL, 32, spec.TINYLLAMA[6])
    cfg = RefCfg(*spec.TINYLLAMA)
    m = model(cfg, spec.SEED_TL)
    T, k, p, seed = spec.SAMPLE_GEN_TL
    cap = len(prompt) + 16 + 1
    pr = (C.c_int * len(prompt))(*prompt)
    o = (C.c_int * cap)()
    t = time.time()
    total = R.q48r_generate_sampled(m, pr, len(prompt), 16, o, T, k, p, seed)
    tg = time.time() - t
    R.q48r_model_free(m)
    write("sample_tinyllama.json", {
        "source": "generate(sp) (llama_int.c:3067-3135, sample_token 2958-3039) via "
                  "oracle/ref_harness.c",
        "config": list(spec.TINYLLAMA), "seed": spec.SEED_TL, "prompt": prompt, "max_new": 16,
        "T": T, "top_k": k, "top_p": p, "rng_seed": seed, "tokens": list(o[:total]),
        "ref_cpu_s": round(tg, 1)})


R = None

if __name__ == "__main__":
    R = ref()
    jobs = sys.argv[1:] or ["fp", "gemv", "ops", "layer", "tiny"]
    for j in jobs:
        t = time.time()
        globals()["gen_" + j]()
        print(f"{j}: {time.time() - t:.1f}s", flush=True)
