import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "golden_ref.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture
def tune():
    """tune(key=value, ...) forces kernel choices (bf16x_set_tuning) until the
    test ends, then restores them."""
    import bfloat16x_amd as bx
    active = []

    def apply(**overrides):
        t = bx.tuning(**overrides)
        t.__enter__()
        active.append(t)

    yield apply
    for t in reversed(active):
        t.__exit__(None, None, None)


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_dict_cases(g):
    """[(key, bits_in, sub, fields...)] for every dict case in the fixture."""
    keys = sorted({k[: k.index("_in")] for k in g if k.startswith("dict_") and k.endswith("_in")})
    cases = []
    for key in keys:
        sub = int(key.rsplit("_s", 1)[1])
        cases.append((key, g[key + "_in"], sub))
    return cases
