import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "feather-ops_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _built() -> bool:
    pkg = ROOT / "feather-ops_amd" / "feather_ops"
    return (pkg / "_C.so").exists() and (pkg / "libfeather_ops_gfx950.so").exists() and (
        ROOT / "oracle" / "_build" / "liboracle.so"
    ).exists()


def pytest_sessionstart(session):
    # Tests load what is built; they build only when nothing is.
    if not _built():
        import __graft_entry__

        __graft_entry__.build()


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
