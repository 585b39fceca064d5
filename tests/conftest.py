"""pytest setup: the `gpu` marker, import paths for the package and the oracle, shared helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "nemicli-terminal_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu on the MI355X box)")


def pytest_collection_modifyitems(config, items):
    # print the test id before each GPU test starts, so a hang or fault names its case
    pass


@pytest.fixture
def tune():
    """Launch-plan overrides for one test (nmq_set_tuning), restored to the defaults afterwards:
    tune(MVM=2, MVT_MAX=1)."""
    from ggufengine_amd import _native
    touched = set()

    def set_knobs(**knobs):
        for name, value in knobs.items():
            touched.add(name)
            _native.set_tuning(name, value)

    yield set_knobs
    for name in touched:
        _native.set_tuning(name, None)


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    return O


def random_blocks(fmt: str, n_blocks: int, seed: int) -> np.ndarray:
    """Random block bytes with small finite fp16 scales (the reference's `zufallsbloecke`,
    tests/test_gguf_iq.py:81-101 and tests/test_mmvq.py:34-45): every byte random, then the scale
    fields set to fp16 values in [0.001, 0.011)."""
    sizes = {"Q4_0": 18, "Q8_0": 34, "Q4_K": 144, "Q6_K": 210, "IQ2_XXS": 66, "TQ2_0": 66}
    fields = {"Q4_0": (0,), "Q8_0": (0,), "Q4_K": (0, 2), "Q6_K": (208,), "IQ2_XXS": (0,), "TQ2_0": (64,)}
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n_blocks, sizes[fmt]), dtype=np.uint8)
    for o in fields[fmt]:
        s = (rng.random(n_blocks) * 0.01 + 0.001).astype(np.float16)
        raw[:, o:o + 2] = s.view(np.uint8).reshape(n_blocks, 2)
    return raw.reshape(-1)
