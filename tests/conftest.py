"""pytest configuration: the `gpu` marker and shared fixtures.

CPU tests (-m "not gpu") cover the oracle against the golden vectors, the
host logic and the C-ABI library's exports.  GPU tests (-m gpu) are the
parity tests proper: they call libintllm_hip through its C ABI and compare
with the oracle / golden vectors bit for bit.  They fail (never skip) when
the HIP library is missing, so a GPU run cannot pass on anything but the
native path.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests"))
sys.path.insert(0, str(ROOT / "int-llm_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X, gfx950) and libintllm_hip")


GOLD = ROOT / "tests" / "golden"


def golden(name: str):
    p = GOLD / name
    if not p.exists():
        pytest.fail(f"golden fixture {p} is missing (tests/golden/make_golden.py writes it)")
    return json.loads(p.read_text())


def bf16_reference():
    """bfloat16_to_q1648 (safetensors.h:115-152) of all 65536 bit patterns,
    as the compiled reference computed them (tests/golden/bf16_to_q48.npz)."""
    import numpy as np
    meta = golden("bf16_to_q48.json")
    with np.load(GOLD / meta["file"], allow_pickle=False) as z:
        v = z["v"]
    assert v.dtype == np.int64 and v.size == meta["n"] == 65536
    return v


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def ctx():
    import intllm
    c = intllm.Context(0)
    yield c
    c.close()
