import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs the native GPU path")
    # GPU runs compare against the reference engine in a worker process; it
    # is started here, before any test touches the GPU
    markexpr = getattr(config.option, "markexpr", "") or ""
    if "gpu" in markexpr and "not gpu" not in markexpr:
        from oracle import ref_lib

        if ref_lib.available():
            import ref_worker

            ref_worker.start()


def pytest_unconfigure(config):
    import sys as _sys

    rw = _sys.modules.get("ref_worker")
    if rw is not None:
        rw.stop()


@pytest.fixture(scope="session")
def tmpdir_session(tmp_path_factory):
    return tmp_path_factory.mktemp("pdefa")
