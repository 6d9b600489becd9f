"""Shared fixtures: the CPU oracle (test infrastructure), the compiled reference subset when present, and the
product library. GPU tests are marked `gpu`; everything else runs on the CPU."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bitllm.c_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


def P(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


@pytest.fixture(scope="session")
def oracle():
    import oracle_api
    return oracle_api.load(ORACLE_SO)


@pytest.fixture(scope="session")
def ref():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libref.so not built (reference tree absent)")
    import oracle_api
    return oracle_api.load_ref(REF_SO)


@pytest.fixture(scope="session")
def gpu():
    """The product library with a live gfx950 device (only for tests marked gpu)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import bitllm_hip
    lib = bitllm_hip.load()
    rc = lib.eif_hip_init(0)
    assert rc == 0, f"eif_hip_init failed: {rc}"
    return bitllm_hip
