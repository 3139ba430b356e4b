"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

# torch is imported before the HIP library is loaded so that both share one
# HIP runtime in the process (tests hand torch-allocated device buffers to the
# library); importing it does not touch the GPU.
try:
    import torch  # noqa: F401
except ImportError:  # the CPU-only checks do not need it
    torch = None

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "index-tts2-metal_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    import mit2cfm
    from oracle import oracle

    if not mit2cfm.LIB_PATH.exists() or not oracle.LIB_PATH.exists():
        import __graft_entry__

        __graft_entry__.build()


@pytest.fixture(scope="session")
def mit2():
    _ensure_built()
    import mit2cfm

    mit2cfm.lib()
    return mit2cfm


@pytest.fixture(scope="session")
def orc():
    _ensure_built()
    from oracle import oracle

    oracle.set_threads(oracle.default_threads())
    return oracle


@pytest.fixture(scope="session")
def tensors(mit2):
    """The benchmark's synthetic weights: every tensor N(0, 0.02) f16."""
    return mit2.synthetic_tensors(20240605, 0.02)


@pytest.fixture(scope="session")
def tensors_unit(mit2):
    """Activation-preserving synthetic weights (fan-in scaled)."""
    return mit2.synthetic_tensors(7, 0.0)


@pytest.fixture(scope="session")
def model(orc, tensors):
    return orc.Model(tensors)


@pytest.fixture(scope="session")
def model_unit(orc, tensors_unit):
    return orc.Model(tensors_unit)


def sincos_series(n: int, a: float, b: float, amp1: float, amp2: float, mod: int) -> np.ndarray:
    """Deterministic input series of the reference's stage tests
    (e.g. dit_cfm_bigvgan.cpp:82-91): sin(i*a)*amp1 + cos((i % mod)*b)*amp2."""
    i = np.arange(n, dtype=np.float32)
    return (np.sin(i * np.float32(a)) * np.float32(amp1)
            + np.cos((np.arange(n) % mod).astype(np.float32) * np.float32(b)) * np.float32(amp2)).astype(np.float32)
