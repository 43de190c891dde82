"""The reference-side binding (int-llm_amd/refbind/llama_int_q48.c): the
unmodified llama_int.c compiled in one unit with the code that routes its
llama_forward to libintllm_hip.

CPU: the library was built against the reference's own types and links
libintllm_hip; with nothing attached, llama_forward is still the
reference's CPU forward (the routing macro changes nothing else), and
the reference's mgw_load reads a .mgw the host wrote.
GPU: the reference's own generate() (llama_int.c:3067-3135), with
llama_forward running on the device, gives the golden tokens and every
step's logits hash.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest

import intllm
import oracle_lib as O
import spec
from conftest import golden

ROOT = Path(__file__).resolve().parents[1]
REFBIND_SO = ROOT / "int-llm_amd" / "refbind" / "_out" / "libllama_int_q48.so"

needs_so = pytest.mark.skipif(
    not REFBIND_SO.exists(),
    reason="refbind library not built (its build needs /root/reference)")


def _lib():
    lib = C.CDLL(str(REFBIND_SO))
    lib.lq48_model_load_mgw.restype = C.c_void_p
    lib.lq48_model_load_mgw.argtypes = [C.c_char_p]
    lib.lq48_model_free.argtypes = [C.c_void_p]
    lib.lq48_model_config.argtypes = [C.c_void_p, C.POINTER(C.c_int * 9)]
    lib.lq48_attach.argtypes = [C.c_void_p, C.c_int]
    lib.lq48_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    lib.lq48_generate.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                  C.c_void_p, C.c_int, C.POINTER(C.c_int)]
    return lib


class RefModel:
    """A llama_model_t loaded by the reference's mgw_load from a .mgw that
    the C host wrote for the synthetic model (config, seed)."""

    def __init__(self, lib, config, seed):
        self.lib = lib
        self.cfg = intllm.Config(*config)
        self.tmp = tempfile.TemporaryDirectory()
        path = os.path.join(self.tmp.name, "m.mgw")
        rc = intllm.host_lib().q48h_mgw_write_synth(path.encode(), C.byref(self.cfg), seed, 4)
        assert rc == 0
        self.m = lib.lq48_model_load_mgw(path.encode())
        assert self.m

    def generate(self, prompt, max_new):
        out = (C.c_int * (len(prompt) + max_new))()
        hs = (C.c_uint64 * (len(prompt) + max_new))()
        n = C.c_int()
        p = (C.c_int * len(prompt))(*prompt)
        total = self.lib.lq48_generate(self.m, p, len(prompt), max_new, out, hs, len(hs),
                                       C.byref(n))
        return total, list(out[:max(total, 0)]), ["%016x" % h for h in hs[:n.value]]

    def free(self):
        self.lib.lq48_model_free(self.m)
        self.tmp.cleanup()


@needs_so
def test_refbind_links_library_and_exports():
    """Built against llama_int.c's types, linked to libintllm_hip (a NEEDED
    entry resolved in-tree), exporting the binding's entry points."""
    out = subprocess.run(["readelf", "-d", str(REFBIND_SO)], capture_output=True, text=True,
                         check=True).stdout
    assert "libintllm_hip.so" in out
    lib = _lib()
    for name in ("lq48_attach", "lq48_detach", "lq48_generate", "lq48_forward",
                 "lq48_model_load_mgw", "lq48_model_free", "llama_int_main"):
        assert hasattr(lib, name)


@needs_so
def test_refbind_cpu_route_unchanged():
    """Nothing attached: llama_forward is the reference's own CPU forward,
    the model comes from the reference's mgw_load, and the logits equal the
    oracle's (the routing macro left the rest of the unit alone)."""
    lib = _lib()
    rm = RefModel(lib, spec.TINY, 11)
    try:
        cfg = (C.c_int * 9)()
        lib.lq48_model_config(rm.m, C.byref(cfg))
        assert tuple(cfg) == (256, 8, 2, 32, 2, 688, 512, 2048, 10000)
        om = O.Model(spec.TINY, 11)
        for pos, tok in enumerate([5, 100, 511]):
            lg = np.empty(512, dtype=np.int64)
            assert lib.lq48_forward(rm.m, tok, pos, lg.ctypes.data) == 0
            rc, want = om.forward(tok, pos)
            assert rc == 0 and np.array_equal(lg, want)
        lg = np.empty(512, dtype=np.int64)
        assert lib.lq48_forward(rm.m, 512, 3, lg.ctypes.data) == -1   # token range
        assert lib.lq48_forward(rm.m, 7, 2048, lg.ctypes.data) == -1  # pos range
        om.free()
    finally:
        rm.free()


@needs_so
@pytest.mark.gpu
def test_refbind_generate_config1_on_device():
    """Config 1 through the reference's own generate() with llama_forward
    on the device: the 48 golden tokens and all 47 logits hashes."""
    g = golden("tiny_generate.json")
    lib = _lib()
    rm = RefModel(lib, spec.TINY, g["seed"])
    try:
        assert lib.lq48_attach(rm.m, 0) == 0
        total, toks, hs = rm.generate(g["prompt"], g["max_new"])
        assert total == len(g["tokens"])
        assert toks == g["tokens"]
        assert hs == g["step_fnv"]
        # out-of-range calls return NULL (-1) as llama_forward does
        lg = np.empty(512, dtype=np.int64)
        assert lib.lq48_forward(rm.m, 512, 0, lg.ctypes.data) == -1
        assert lib.lq48_forward(rm.m, 3, 2048, lg.ctypes.data) == -1
        lib.lq48_detach()
    finally:
        rm.free()
