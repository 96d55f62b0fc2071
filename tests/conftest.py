import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs through the C ABI on the device")
    config.addinivalue_line("markers", "ref: needs the reference build in oracle/_ref (this container only)")
    config.addinivalue_line("markers", "perf: timing bounds on an MI355X (clock, rate, ranking, cost model); not "
                                       "correctness, so outside -m gpu: run them with -m perf on a GPU box")


def pytest_collection_modifyitems(config, items):
    # Timing tests need the device; on a machine without one they are skipped, not failed.
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="perf: timing bounds need an MI355X")
    for it in items:
        if "perf" in it.keywords:
            it.add_marker(skip)


def _has_gpu() -> bool:
    # Counting devices does not initialise HIP in this image's runtime; the library's own
    # device check runs inside the tests.
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def uk():
    import unikern_amd

    return unikern_amd


@pytest.fixture(scope="session")
def gpu(uk):
    arch = uk.device_check()
    assert arch.startswith("gfx950"), arch
    return uk


@pytest.fixture(scope="session")
def ref():
    import _oracle

    if not _oracle.ref_available():
        pytest.skip("oracle/_ref/libukref.so not built (it is compiled from the reference tree, which only the build "
                    "container holds; a tree without that build skips the reference cross-checks)")
    return _oracle.ref()
