import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU oracle work")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def load(name):
        with np.load(GOLDEN / name, allow_pickle=False) as z:
            return {k: z[k] for k in z.files}

    return load


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as O

    O.build(ref=False)
    O.set_threads(int(os.environ.get("SOC_ORACLE_THREADS", str(min(16, os.cpu_count() or 1)))))
    return O


@pytest.fixture(scope="session")
def gpu_ctx():
    from soc_amd import Context

    ctx = Context(0)
    yield ctx
    ctx.close()
