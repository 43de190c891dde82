#!/usr/bin/env python3
"""bench.py — TinyLlama-shape Q16.48 decode on one MI355X.

One "step" is one greedy decode token of the TinyLlama-1.1B-shape model
(22 layers, d=2048, 32/4 heads, ffn 5632, vocab
32000, all int64 Q16.48) at batch 1, through the C host (libq48host) and
libintllm_hip: embed, 22 x (RMSNorm, q|k|v GEMV, RoPE, exact attention,
o GEMV, residual, RMSNorm, gate|up GEMV, SwiGLU, down GEMV, residual),
final RMSNorm, lm_head GEMV, argmax.  Weights are synthetic random-init
(q48_synth.h), resident in HBM before timing starts.

Printed (one JSON line): decode tok/s, the roofline of the dominant kernel
(q48_gemv, HBM-bound: algorithmic bytes / HIP-event launch time), the
config-2 GEMV shapes' GB/s over rotating buffers (> MALL), the CPU
baseline (the reference's own llama_forward, compiled from its sources,
single-threaded, on this host) and whether the decoded tokens equal the
reference's token stream.

    python bench.py [--gpus 1] [--steps 64] [--warmup 8] [--cpu-seconds 15]
"""
from __future__ import annotations

import argparse
import ctypes as C
import hashlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "int-llm_amd"))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the roofline sweep, from rocprofv3 --pmc FETCH_SIZE
# and WRITE_SIZE runs scaled by the counters' reading for a copy kernel of known
# size (profiles/k_gemv_decode_tinyllama.md).  The figure holds for the GEMV
# sources it was measured on: TRAFFIC_SOURCES hash to TRAFFIC_SHA256 (the first
# 16 hex digits of the sha256 of their code, in this order, with comments and
# whitespace removed); with any other code the bench line reports traffic null
# until the counters are re-run.
TRAFFIC = 93623763
TRAFFIC_SOURCES = ("int-llm_amd/csrc/q48_gemv.hip", "int-llm_amd/csrc/q48_gemv_tiles.hpp")
TRAFFIC_SHA256 = "098d50a3e7231121"
REF_CPU_MS_PER_TOK = 501.4   # reference decode, Zen 4, 1 thread
# int8 GEMM: MI355X dense int8 MFMA peak; one Q16.48 MAC is 63 int8 products
# (digit pairs a + b <= 13), 2 ops each
I8_PEAK_OPS = 5.0e15
I8_OPS_PER_MAC = 126
# VALU GEMM: one Q16.48 MAC is four v_mad_u64_u32 (32 x 32 -> 64-bit limb
# products); their rate on MI355X, measured with 16 independent chains per
# lane and 16 waves per compute unit: 17.2e12 lane-ops/s (28 per clock per CU)
VALU_MAD_PEAK = 17.2e12
VALU_MADS_PER_MAC = 4


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def threads():
    return max(1, min(16, os.cpu_count() or 1))


def gemv_shapes(ctx, spec, intllm, reps: int):
    """GB/s of q48_gemv per config-2 shape, rotating over distinct weight
    buffers totalling > 2 GiB so the 256 MB MALL cannot serve them; launches
    back to back between two HIP events on the library's stream."""
    out = {}
    gold = json.loads((ROOT / "tests" / "golden" / "gemv.json").read_text())["shapes"]
    pool_bytes = 2_600_000_000
    pool = ctx.buffer(pool_bytes // 8)
    for (M, K) in spec.GEMV_SHAPES + spec.GEMV_FUSED:
        W, x = spec.gemv_inputs_ref(intllm.synth, M, K) if (M, K) in spec.GEMV_SHAPES else (
            intllm.synth(spec.gemv_w_name(M, K), M, K, spec.SEED_GEMV, spec.SIGMA_W, 1),
            intllm.synth(spec.gemv_x_name(K), 1, K, spec.SEED_GEMV, spec.SIGMA_ACT, 0))
        per = M * K + 64
        nbuf = max(1, min(64, (pool.n - 4096) // per))
        pool.upload(W)
        for b in range(1, nbuf):
            intllm.check("d2d", intllm.hip_lib().q48_memcpy_d2d(ctx.h, pool.at(b * per), pool.ptr, M * K * 8))
        dx = ctx.to_device(x)
        dy = ctx.buffer(M)
        for b in range(nbuf):   # warm-up
            ctx.gemv(dy.ptr, pool.at(b * per), dx.ptr, M, K)
        ctx.sync()
        n = max(reps, nbuf)
        ctx.timer_start()
        for i in range(n):
            ctx.gemv(dy.ptr, pool.at((i % nbuf) * per), dx.ptr, M, K)
        ms = ctx.timer_stop()
        # result check against the committed golden vector for the real shapes
        ok = None
        if f"{M}x{K}" in gold:
            ok = intllm.fnv(dy.download()) == gold[f"{M}x{K}"]["fnv"]
        us = 1e3 * ms / n
        out[f"{M}x{K}"] = {"us": round(us, 2),
                           "GB_s": round(8.0 * (M * K + K + M) / (us * 1e-6) / 1e9, 1),
                           "buffers": nbuf, "bit_exact": ok}
        dx.free()
        dy.free()
        log("gemv", M, K, out[f"{M}x{K}"])
    pool.free()
    return out


def sources_sha256() -> str:
    """sha256 (16 hex digits) of the TRAFFIC_SOURCES' code: // and /* */
    comments and all whitespace removed, so comment edits keep the hash."""
    import re
    h = hashlib.sha256()
    for f in TRAFFIC_SOURCES:
        src = (ROOT / f).read_text()
        src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
        src = re.sub(r"//[^\n]*", " ", src)
        h.update(re.sub(r"\s+", "", src).encode())
    return h.hexdigest()[:16]


def traffic_bytes():
    """The PMC-measured HBM bytes per GEMV launch, or None when the GEMV
    sources differ from the ones the counters were read on."""
    return TRAFFIC if sources_sha256() == TRAFFIC_SHA256 else None


def gemm_prefill(ctx, spec, intllm, reps: int):
    """Config 4: q48_gemm at T in {128, 512, 2048} tokens on the config-2
    shapes, with each kernel: int8 digits on the matrix cores ("i8": the one
    q48_gemm picks by shape; "i8_fused": digit split inside the k loop;
    "i8_planes": digit planes split once per call, read by DMA) and 32-bit
    limbs on the vector ALUs ("valu").  Each output is hashed against the golden vector of
    the reference's per-token matmul_vec; times are whole q48_gemm calls
    (the redo pass for blocks outside the digit window and the split-K
    reduction included) between two HIP events on the library's stream."""
    gold = json.loads((ROOT / "tests" / "golden" / "gemm.json").read_text())["shapes"]
    out = {}
    for (N, K) in spec.GEMV_SHAPES:
        dW = ctx.to_device(intllm.synth(spec.gemv_w_name(N, K), N, K, spec.SEED_GEMV,
                                        spec.SIGMA_W, 1, threads()))
        for T in spec.GEMM_TOKENS:
            dX = ctx.to_device(intllm.synth(spec.gemm_x_name(T, K), T, K, spec.SEED_GEMV,
                                            spec.SIGMA_ACT, 0, threads()))
            dY = ctx.buffer(T * N)
            key = f"{T}x{N}x{K}"
            macs = T * N * K
            rec = {}
            for name, kern, n in (("i8", intllm.GEMM_I8, reps),
                                  ("i8_fused", intllm.GEMM_I8_FUSED, reps),
                                  ("i8_planes", intllm.GEMM_I8_PLANES, reps),
                                  ("valu", intllm.GEMM_VALU, 1)):
                ctx.gemm(dY.ptr, dW.ptr, dX.ptr, T, N, K, kern)
                rec[f"{name}_bit_exact"] = intllm.fnv(dY.download()) == gold[key]["fnv"]
                ctx.timer_start()
                for _ in range(n):
                    ctx.gemm(dY.ptr, dW.ptr, dX.ptr, T, N, K, kern)
                us = 1e3 * ctx.timer_stop() / n
                rec[f"{name}_us"] = round(us, 1)
                rec[f"{name}_TMAC_s"] = round(macs / (us * 1e-6) / 1e12, 3)
            rec["i8_frac"] = round(I8_OPS_PER_MAC * macs / (rec["i8_us"] * 1e-6) / I8_PEAK_OPS, 4)
            rec["valu_frac"] = round(VALU_MADS_PER_MAC * macs / (rec["valu_us"] * 1e-6)
                                     / VALU_MAD_PEAK, 4)
            rec["speedup_i8_vs_valu"] = round(rec["valu_us"] / rec["i8_us"], 1)
            out[key] = rec
            log("gemm", key, rec)
            dX.free()
            dY.free()
        dW.free()
    return {"workload": "config 4: Q16.48 GEMM, T tokens x config-2 (N, K), W N(0,0.02) "
                        "bf16-exact, X N(0,1) raw Q16.48",
            "i8_peak_ops": I8_PEAK_OPS, "i8_ops_per_mac": I8_OPS_PER_MAC,
            "i8_frac_basis": "63 int8 digit products (126 ops) per Q16.48 MAC, the full "
                             "digit expansion; for these bfloat16-exact weights the kernel "
                             "runs 28-35 of them (zero digit planes skipped), so i8_frac "
                             "is the rate on the algorithmic count, not MFMA occupancy",
            "valu_mad_peak": VALU_MAD_PEAK, "valu_mads_per_mac": VALU_MADS_PER_MAC,
            "shapes": out}


def _cpu_flags():
    model, flags = "", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and not model:
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return model, flags


# x86-64 micro-architecture levels (the flags /proc/cpuinfo shows for them)
ISA_V3 = {"avx", "avx2", "bmi1", "bmi2", "f16c", "fma", "abm", "movbe", "xsave"}
ISA_V4 = ISA_V3 | {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}


def cpu_baseline(spec, intllm, seconds: float, prompt, n_prompt: int = 16):
    """Single-threaded CPU run of the same model: the reference's own
    llama_forward (oracle/_ref, compiled from llama_int.c with the
    reference's -O3 -fwrapv at the highest x86-64 level this CPU supports,
    standing in for its -march=native), else the oracle port.  Bounded
    sample: generate()'s loop over the first n_prompt prompt tokens
    (prefill, one forward per token) and then greedy decode steps until
    `seconds` of CPU time is spent; plus matmul_vec per config-2 shape.
    KPIs as the reference prints them (llama_int.c:271-285)."""
    import numpy as np
    model_name, flags = _cpu_flags()
    kind, isa = "reference", "x86-64"
    lib = None
    for lvl, need, so in (("x86-64-v4", ISA_V4, "libq48_ref_v4.so"),
                          ("x86-64-v3", ISA_V3, "libq48_ref_v3.so"),
                          ("x86-64", set(), "libq48_ref.so")):
        path = ROOT / "oracle" / "_ref" / so
        if need <= flags and path.exists():
            lib, isa = C.CDLL(str(path)), lvl
            break
    if lib is not None:
        mk, fwd, free = lib.q48r_model_synth, lib.q48r_forward, lib.q48r_model_free
        gemv = lib.q48r_gemv
    else:
        import oracle_lib as O
        lib = O.load()
        kind = "port"
        mk, fwd, free = lib.q48o_model_synth, lib.q48o_forward, lib.q48o_model_free
        gemv = lib.q48o_gemv
    mk.restype = C.c_void_p
    mk.argtypes = [C.c_void_p, C.c_uint64, C.c_int]
    fwd.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    fwd.restype = C.c_int
    free.argtypes = [C.c_void_p]
    gemv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
    gemv.restype = None
    import oracle_lib as O
    cfg = O.Config(*spec.TINYLLAMA)
    # the reference's setup prints to stdout: keep the JSON line alone there
    sys.stdout.flush()
    saved = os.dup(1)
    devnull = os.open(os.devnull, os.O_WRONLY)
    os.dup2(devnull, 1)
    try:
        m = mk(C.byref(cfg), spec.SEED_TL, threads())
    finally:
        os.dup2(saved, 1)
        os.close(saved)
        os.close(devnull)
    logits = np.empty(cfg.vocab, dtype=np.int64)
    t_all = time.perf_counter()
    t_pf = t_dc = 0.0
    n_pf = n_dc = 0
    tok = None
    for pos in range(n_prompt):                        # prefill (llama_int.c:3081-3092)
        t = time.perf_counter()
        assert fwd(m, prompt[pos], pos, logits.ctypes.data) == 0
        t_pf += time.perf_counter() - t
        n_pf += 1
    tok = int(np.argmax(logits))                       # the first maximum, as argmax
    pos = n_prompt
    while time.perf_counter() - t_all < seconds or n_dc < 2:   # decode (:3103-3113)
        t = time.perf_counter()
        assert fwd(m, tok, pos, logits.ctypes.data) == 0
        tok = int(np.argmax(logits))
        t_dc += time.perf_counter() - t
        n_dc += 1
        pos += 1
    free(m)
    # matmul_vec (llama_int.c:1014-1046) per config-2 shape, best of 3
    shapes = {}
    for (M, K) in spec.GEMV_SHAPES:
        W, x = spec.gemv_inputs_ref(intllm.synth, M, K)
        y = np.empty(M, dtype=np.int64)
        best = None
        for _ in range(3):
            t = time.perf_counter()
            gemv(y.ctypes.data, W.ctypes.data, x.ctypes.data, M, K)
            dt = time.perf_counter() - t
            best = dt if best is None else min(best, dt)
        shapes[f"{M}x{K}"] = {"us": round(1e6 * best, 1),
                              "GB_s": round(8.0 * (M * K + K + M) / best / 1e9, 2)}
        del W
    dec_ms = 1e3 * t_dc / n_dc
    return {"value": round(1e3 / dec_ms, 4), "unit": "tok/s", "cores": 1, "kind": kind,
            "isa": isa, "cflags": f"-O3 -fwrapv -march={isa} (reference Makefile:38 uses "
                                  "-O3 -march=native -fwrapv)",
            "cpu_model": model_name, "nproc": os.cpu_count(),
            "prefill_ms_per_tok": round(1e3 * t_pf / n_pf, 2),
            "decode_ms_per_tok": round(dec_ms, 2),
            "tok_per_sec": round((n_pf + n_dc) / (t_pf + t_dc), 4),
            "prefill_tokens": n_pf, "decode_tokens": n_dc,
            "matmul_vec_1core": shapes,
            "sample": f"generate()'s loop on the TinyLlama-shape model: {n_pf} prompt tokens "
                      f"(positions 0..{n_pf - 1}), then {n_dc} greedy decode steps; 1 thread"}


def refbind_decode(spec, intllm, gold, new_tokens: int):
    """The drop-in itself: the reference's own generate()
    (llama_int.c:3067-3135) with its llama_forward routed to libintllm_hip
    (int-llm_amd/refbind: the unmodified llama_int.c compiled with the
    binding), on the TinyLlama-shape model written as a .mgw and loaded by
    the reference's own mgw_load.  Each forward is one graph replay of the
    fused launches plus the synchronous logits copy llama_forward's
    contract needs.  Decode tok/s = K / (t(generate with K + 1 new tokens)
    - t(generate with 1 new token)), the same prompt both times, without
    hashing; a third, untimed run hashes every logits vector on the host
    (FNV-1a over 256 KB, about 0.25 ms each) for the parity check."""
    import tempfile
    so = ROOT / "int-llm_amd" / "refbind" / "_out" / "libllama_int_q48.so"
    if not so.exists():
        return {"skipped": "refbind library not built (its build needs the reference sources)"}
    lib = C.CDLL(str(so))
    lib.lq48_model_load_mgw.restype = C.c_void_p
    lib.lq48_model_load_mgw.argtypes = [C.c_char_p]
    lib.lq48_model_free.argtypes = [C.c_void_p]
    lib.lq48_attach.argtypes = [C.c_void_p, C.c_int]
    lib.lq48_generate.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                  C.c_void_p, C.c_int, C.POINTER(C.c_int)]
    cfg = intllm.Config(*gold["config"])
    prompt = gold["prompt"]
    out = {}
    # the reference prints its progress to stdout: keep the JSON line alone there
    sys.stdout.flush()
    saved = os.dup(1)
    devnull = os.open(os.devnull, os.O_WRONLY)
    os.dup2(devnull, 1)
    try:
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "tinyllama.mgw")
            t = time.perf_counter()
            assert intllm.host_lib().q48h_mgw_write_synth(path.encode(), C.byref(cfg),
                                                          gold["seed"], threads()) == 0
            m = lib.lq48_model_load_mgw(path.encode())
            assert m
            os.unlink(path)
            assert lib.lq48_attach(m, 0) == 0
            out["setup_s"] = round(time.perf_counter() - t, 2)
            p = (C.c_int * len(prompt))(*prompt)

            def gen(k, hashed=False):
                buf = (C.c_int * (len(prompt) + k))()
                hs = (C.c_uint64 * (len(prompt) + k))()
                n = C.c_int()
                t0 = time.perf_counter()
                total = lib.lq48_generate(m, p, len(prompt), k, buf, hs,
                                          len(hs) if hashed else 0, C.byref(n))
                dt = time.perf_counter() - t0
                return (dt, list(buf[:max(total, 0)]),
                        ["%016x" % h for h in hs[:min(n.value, len(hs))]] if hashed else [])

            gen(2)                                  # warm: captures both graphs' first kind
            t1, _, _ = gen(1)
            t2, toks, _ = gen(1 + new_tokens)
            _, toks_h, hs = gen(1 + new_tokens, hashed=True)
            lib.lq48_detach()
            lib.lq48_model_free(m)
    finally:
        os.dup2(saved, 1)
        os.close(saved)
        os.close(devnull)
    n = len(toks)
    ms = 1e3 * (t2 - t1) / new_tokens
    out.update({"workload": "config 3: the reference's generate() and mgw_load with "
                            "llama_forward on the device (refbind), greedy",
                "tok_s": round(1e3 / ms, 2), "ms_per_tok": round(ms, 4),
                "new_tokens_timed": new_tokens,
                "tokens_match_reference": toks == gold["tokens"][:n] and toks_h == toks,
                "step_hashes_match_reference": hs == gold["step_fnv"][:len(hs)]})
    log(f"refbind generate decode {ms:.3f} ms/tok")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    ap.add_argument("--long-steps", type=int, default=32,
                    help="config-5 (2048-position cache) decode steps timed; 0 skips")
    ap.add_argument("--gemv-reps", type=int, default=8,
                    help="decode-token GEMV sequences timed back to back for the roofline")
    ap.add_argument("--gemm-reps", type=int, default=5,
                    help="int8 GEMM calls timed per config-4 shape; 0 skips config 4")
    ap.add_argument("--no-sample", action="store_true",
                    help="skip the sampled-decode measurement")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the batched-prefill measurement")
    ap.add_argument("--prefill-reps", type=int, default=3)
    ap.add_argument("--no-bf16", action="store_true",
                    help="skip the bfloat16-resident-weights decode measurement")
    ap.add_argument("--no-refbind", action="store_true",
                    help="skip the reference-side binding's generate() measurement")
    ap.add_argument("--gemm-only", action="store_true",
                    help="run only the config-4 GEMM measurement (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the Q16.48 decode path is "
              "single-GPU)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import intllm
    import spec

    if args.gemm_only:
        ctx = intllm.Context(0)
        print(json.dumps({"gemm": gemm_prefill(ctx, spec, intllm, max(1, args.gemm_reps))}),
              flush=True)
        ctx.close()
        return

    gold = json.loads((ROOT / "tests" / "golden" / "tinyllama_generate.json").read_text())
    gold_long = json.loads((ROOT / "tests" / "golden" / "longctx_decode.json").read_text())
    ctx = intllm.Context(0)
    # config 3's weights with config 5's cache length (4096 positions): the
    # short-context decode does not depend on the cache length, and the same
    # model then serves the long-context measurement
    cfg = intllm.Config(*spec.LONGCTX)
    log("synthesising TinyLlama-shape weights (8.8 GB) and uploading")
    t = time.time()
    m = intllm.HostModel(ctx, cfg)
    m.synth(spec.SEED_TL, threads())
    if os.environ.get("INTLLM_FUSE"):
        m.set_fused(int(os.environ["INTLLM_FUSE"]))
    log(f"model ready in {time.time() - t:.1f}s")

    prompt = gold["prompt"]
    # every replayed decode step records its logits on the device and they
    # are hashed (FNV-1a 64, as the reference's logits) against the golden
    # per-step hashes: positions p of the golden run have step_fnv[p]
    hashes = {"compared": 0, "matched": 0, "first_mismatch": None}

    def check_hashes(label, p0, hs, ref):
        for i, h in enumerate(hs):
            if p0 + i < len(ref):
                hashes["compared"] += 1
                if h == ref[p0 + i]:
                    hashes["matched"] += 1
                elif hashes["first_mismatch"] is None:
                    hashes["first_mismatch"] = f"{label} position {p0 + i}"

    # prefill (untimed): the prompt, one forward per token as generate() does
    nxt = None
    for pos, tok in enumerate(prompt):
        nxt, _ = m.forward(tok, pos, cfg.vocab, logits=False)
    toks = [nxt]
    pos = len(prompt)
    # warm-up decode steps (also captures the decode-step graph)
    _, steps, hs, _ = m.decode_graph_hashed(toks[-1], pos, args.warmup)
    check_hashes("int64 warm-up", pos, hs, gold["step_fnv"])
    toks += steps
    pos += args.warmup
    ctx.sync()
    # timed: K greedy decode steps replayed from the graph (argmax and the
    # logits record on the device), from the first step's launch to the K
    # tokens back on the host; the host hashes the records afterwards
    t0 = time.perf_counter()
    _, steps, hs, st = m.decode_graph_hashed(toks[-1], pos, args.steps)
    wall = time.perf_counter() - t0
    check_hashes("int64 timed", pos, hs, gold["step_fnv"])
    toks += steps
    pos += args.steps
    ms = 1e3 * st.decode_s / args.steps
    log(f"decode {ms:.3f} ms/tok (call incl. hashing {1e3 * wall / args.steps:.3f})")

    p0 = len(prompt) + args.warmup
    # roofline of the dominant kernel (q48_gemv): the GEMV launches of one
    # decode token, in decode order on the model's own weights, timed back to
    # back with two HIP events on the library's stream (no per-launch events,
    # which would add their own gaps); average launch = elapsed / launches
    m.gemv_sweep(1)                                   # warm
    ctx.timer_start()
    launches, gbytes = m.gemv_sweep(args.gemv_reps)
    gemv_ms = ctx.timer_stop()
    avg_us = 1e3 * gemv_ms / launches
    bytes_per_launch = gbytes / launches
    achieved = bytes_per_launch / (avg_us * 1e-6) / 1e9

    # the same greedy stream continued with bfloat16-resident weights (2 B
    # per weight, expanded exactly in the kernels; same bits): the tokens
    # join the parity check below
    bf16 = None
    if not args.no_bf16:
        m.set_bf16(True)
        _, steps, hs, _ = m.decode_graph_hashed(toks[-1], pos, args.warmup)
        check_hashes("bf16 warm-up", pos, hs, gold["step_fnv"])
        toks += steps
        pos += args.warmup
        ctx.sync()
        b0 = pos
        _, steps, hs, bst = m.decode_graph_hashed(toks[-1], pos, args.steps)
        check_hashes("bf16 timed", pos, hs, gold["step_fnv"])
        bms = 1e3 * bst.decode_s / args.steps
        toks += steps
        pos += args.steps
        m.gemv_sweep(1)
        ctx.timer_start()
        bl, bgb = m.gemv_sweep(args.gemv_reps)
        bus = 1e3 * ctx.timer_stop() / bl
        bach = bgb / bl / (bus * 1e-6) / 1e9
        m.set_bf16(False)
        log(f"bf16-resident decode {bms:.3f} ms/tok")
        bf16 = {"workload": "config 3 with bfloat16-resident weights (2.07 GB read per token)",
                "tok_s": round(1e3 / bms, 2), "ms_per_tok": round(bms, 4),
                "positions": [b0, b0 + args.steps],
                "gemv_avg_launch_us": round(bus, 3), "gemv_achieved_GBs": round(bach, 1),
                "gemv_frac": round(bach / HBM_PEAK_GBS, 4)}

    # sampled decode (row f4): the same graph-replayed steps with
    # sample_token on the device (T 0.8, top-k 40, top-p 0.9) instead of
    # argmax; the tokens are not the greedy stream, so they stay out of the
    # parity check (tests/test_gpu_sample.py pins them)
    sampled = None
    if not args.no_sample:
        T, k, p_, seed = spec.SAMPLE_GEN_TL
        m.set_sampling(T, k, p_, seed)
        st_tok, _, _ = m.decode_graph(toks[-1], pos, args.warmup)
        ctx.sync()
        s0 = pos + args.warmup
        t0 = time.perf_counter()
        m.decode_graph(st_tok[-1] if st_tok else toks[-1], s0, args.steps)
        ctx.sync()
        sms = 1e3 * (time.perf_counter() - t0) / args.steps
        m.set_sampling(0)
        log(f"sampled decode {sms:.3f} ms/tok")
        sampled = {"workload": "config 3 decode, int64 weights, sample_token on the device "
                               "(temperature 0.8, top-k 40, top-p 0.9)",
                   "tok_s": round(1e3 / sms, 2), "ms_per_tok": round(sms, 4),
                   "positions": [s0, s0 + args.steps]}

    # batched prefill: prompts of T tokens through q48h_prefill (row ops and
    # q48_gemm projections; lm_head of the last row only), against the
    # per-token forward that the reference's generate runs for a prompt.
    # The golden prompt's first token joins the parity check.
    pf = None
    if not args.no_prefill:
        m.kv_reset()
        pf_next, _ = m.prefill(prompt, 0, cfg.vocab, logits=False)
        pf = {"workload": "config 3 prompt of T tokens at positions 0..T-1, int64 "
                               "weights, batched (q48h_prefill)",
                   "golden_prompt_next_token_matches": pf_next == gold["tokens"][len(prompt)],
                   "T": {}}
        rng = np.random.default_rng(11)
        for T in (32, 128, 512, 2048):
            tk = [int(v) for v in rng.integers(0, cfg.vocab, size=T)]
            m.prefill(tk, 0, cfg.vocab, logits=False)         # warm (buffers)
            ctx.sync()
            t0 = time.perf_counter()
            for _ in range(args.prefill_reps):
                m.prefill(tk, 0, cfg.vocab, logits=False)
            pms = 1e3 * (time.perf_counter() - t0) / args.prefill_reps
            pf["T"][str(T)] = {"ms": round(pms, 3), "tok_s": round(1e3 * T / pms, 1)}
            log(f"batched prefill T={T}: {pms:.2f} ms ({1e3 * T / pms:.0f} tok/s)")
            if T >= 512:
                # the same prefill with attention on the VALU kernel
                ctx.set_pf_attn_mfma(False)
                m.prefill(tk, 0, cfg.vocab, logits=False)
                ctx.sync()
                t0 = time.perf_counter()
                m.prefill(tk, 0, cfg.vocab, logits=False)
                vms = 1e3 * (time.perf_counter() - t0)
                ctx.set_pf_attn_mfma(True)
                pf["T"][str(T)]["valu_attention_ms"] = round(vms, 3)
                log(f"batched prefill T={T}, VALU attention: {vms:.2f} ms")
        # the per-token route over the golden prompt (what generate did
        # before batching): forward calls without logits copies
        m.set_batched_prefill(False)
        t0 = time.perf_counter()
        for pos, tok in enumerate(prompt):
            m.forward(tok, pos, cfg.vocab, logits=False, choose=pos == len(prompt) - 1)
        seq_ms = 1e3 * (time.perf_counter() - t0)
        m.set_batched_prefill(True)
        pf["per_token_forward"] = {"T": len(prompt), "ms": round(seq_ms, 3),
                                        "tok_s": round(1e3 * len(prompt) / seq_ms, 1)}

    # token stream vs the reference's (golden), over the tokens both have
    ref_new = gold["tokens"][len(prompt):]
    n_cmp = min(len(ref_new), len(toks))
    parity = {"tokens_compared": n_cmp, "tokens_match_reference": toks[:n_cmp] == ref_new[:n_cmp]}
    if pf is not None:
        parity["prefill_next_token_matches_reference"] = \
            pf["golden_prompt_next_token_matches"]

    # a one-launch split attention (positions from q48_attn_split_min()) that gave up reports
    # Q48_ETIMEOUT instead of logits: the leg is recorded as failed and the
    # parity check fails, rather than the run ending without a line
    timeouts = []

    def guarded(label, fn, *a):
        try:
            return fn(*a)
        except intllm.Q48Error as e:
            if e.code != intllm.Q48_ETIMEOUT:
                raise
            timeouts.append(label)
            log(f"{label}: split attention timed out")
            return None

    # config 5: the cache pre-filled to 2048 positions, then greedy decode
    # steps replayed from the graph (the golden stream covers 256 of them)
    longctx = None
    if args.long_steps > 0:
        prefill = gold_long["prefill"]
        m.kv_fill_synth(gold_long["kv_seed"], prefill, threads())
        tok0 = gold_long["start_token"]
        long_fnv = [None] * prefill + gold_long["step_fnv"]
        # the first steps warm (they are also checked against the reference)
        r1 = guarded("config-5 warm-up", m.decode_graph_hashed, tok0, prefill, args.warmup)
        r2 = None
        if r1 is not None:
            _, lw, hs, _ = r1
            check_hashes("config-5 warm-up", prefill, hs, long_fnv)
            ctx.sync()
            r2 = guarded("config-5 timed", m.decode_graph_hashed, lw[-1], prefill + args.warmup,
                         args.long_steps)
    if args.long_steps > 0 and r2 is None:
        longctx = {"attention_timeout": timeouts, "tokens_match_reference": False}
    elif args.long_steps > 0:
        _, lt, hs, lst = r2
        check_hashes("config-5 timed", prefill + args.warmup, hs, long_fnv)
        lms = 1e3 * lst.decode_s / args.long_steps
        ltoks = [tok0] + lw + lt
        ref = [tok0] + gold_long["tokens"]
        n = min(len(ref), len(ltoks))
        log(f"long-context decode {lms:.3f} ms/tok")
        kv_bytes = 2 * 22 * 4 * 64 * 8 * (prefill + args.warmup + args.long_steps // 2)
        longctx = {"workload": "config 5: TinyLlama-1.1B shape, int64 KV cache pre-filled to "
                               f"{prefill} positions (N(0,1) bf16-exact), greedy decode",
                   "tok_s": round(1e3 / lms, 2), "ms_per_tok": round(lms, 4),
                   "positions": [prefill + args.warmup, prefill + args.warmup + args.long_steps],
                   "kv_bytes_per_token": kv_bytes,
                   "tokens_compared": n, "tokens_match_reference": ltoks[:n] == ref[:n]}
    m.free()
    refbind = None if args.no_refbind else refbind_decode(spec, intllm, gold, args.steps)
    if refbind and "tok_s" in refbind:
        refbind["fraction_of_host_path"] = round(refbind["tok_s"] / (1e3 / ms), 4)
        parity["refbind_tokens_match_reference"] = (refbind["tokens_match_reference"] and
                                                    refbind["step_hashes_match_reference"])
    parity["step_logits_hashes_compared"] = hashes["compared"]
    parity["step_logits_hashes_matched"] = hashes["matched"]
    if hashes["first_mismatch"]:
        parity["first_hash_mismatch"] = hashes["first_mismatch"]
    parity["attention_timeouts"] = timeouts
    parity["all_match"] = (parity["tokens_match_reference"] and not timeouts and
                           hashes["matched"] == hashes["compared"] and
                           (longctx is None or longctx["tokens_match_reference"]) and
                           parity.get("prefill_next_token_matches_reference", True) and
                           parity.get("refbind_tokens_match_reference", True))

    shapes = None if args.no_shapes else gemv_shapes(ctx, spec, intllm, reps=64)
    gemm = gemm_prefill(ctx, spec, intllm, args.gemm_reps) if args.gemm_reps > 0 else None
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline(spec, intllm, args.cpu_seconds, prompt)

    value = 1e3 / ms
    line = {
        "metric": "TinyLlama-shape Q16.48 decode tok/s",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / (1e3 / REF_CPU_MS_PER_TOK), 1),
        "vs_baseline_source": "published llama_int CPU decode, 501.4 ms/tok, TinyLlama-1.1B on a "
                              "Ryzen 7 7700, 1 thread (validation/cpu/X86_64_AMD_ZEN4/results/"
                              "2026-07-30-x86-amd-zen4-tinyllama.txt:31)",
        "vs_cpu_same_run": (round(value / cpu["value"], 1) if cpu else None),
        "dtype": "int64",
        "data": "synthetic: random-init N(0,0.02) bf16-exact Q16.48 weights, seeded 32-token prompt",
        "config": {"workload": "config 3: TinyLlama-1.1B-shape greedy decode, batch 1, "
                               "int64 Q16.48 weights resident in HBM (8.28 GB read per token)",
                   "layers": 22, "dim": 2048, "heads": 32, "kv_heads": 4, "ffn": 5632,
                   "vocab": 32000, "prompt_tokens": len(prompt), "positions": [p0, p0 + args.steps]},
        "roofline": {"bound": "hbm",
                     "kernel": "k_gemv_r1 / k_gemv_v5 / k_gemv_p6 (q48_gemv family: the 89 "
                               "fused GEMV launches of a decode token, back to back)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(),
                     "traffic_sources_sha256": sources_sha256(),
                     "avg_launch_us": round(avg_us, 3),
                     "algorithmic_bytes_per_launch": round(bytes_per_launch),
                     "launches_timed": launches},
        "cpu_baseline": cpu,
        "gemv_shapes": shapes,
        "gemm_prefill": gemm,
        "long_context": longctx,
        "bf16_resident": bf16,
        "sampled_decode": sampled,
        "batched_prefill": pf,
        "refbind_generate": refbind,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
