import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "local-research-small-language-model_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libsparda.so")


import pytest  # noqa: E402


@pytest.fixture(autouse=True, scope="session")
def _in_tree_library():
    """Every test binds the in-tree libsparda.so unless SPARDA_LIBRARY names
    another build explicitly."""
    from sparda import _lib
    if not os.environ.get("SPARDA_LIBRARY"):
        want = os.path.join(PKG, "sparda", "libsparda.so")
        assert os.path.abspath(_lib.LIB_PATH) == os.path.abspath(want), _lib.LIB_PATH
    yield
