import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def known_answers():
    return json.loads((GOLDEN / "reference_known_answers.json").read_text())


@pytest.fixture(scope="session")
def ora():
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def dev():
    """Initialises the HIP library on device 0; fails loudly if it is not built."""
    import doe_amd
    if not doe_amd.LIB_PATH.exists():
        pytest.fail(f"{doe_amd.LIB_PATH} is missing: build it before running GPU tests")
    doe_amd.init(0)
    info = doe_amd.device_info()
    print(f"[dev] {info}", flush=True)
    return doe_amd


@pytest.fixture(params=[1, 2], ids=["dot_kernel", "mfma_kernel"])
def gemv_kernel(request, dev):
    """Forces one Q4_K GEMV kernel (1: per-chunk dot products, 2: matrix
    cores) and restores the automatic choice afterwards.  The automatic choice
    is the matrix-core kernel (K split over workgroups past k = 16384); the
    dot-product kernel runs only when forced, where its LDS holds the
    activation."""
    from doe_amd import ops
    ops.tune("q4k_gemv.kernel", request.param)
    yield request.param
    ops.tune("q4k_gemv.kernel", 0)
