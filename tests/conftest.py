"""Test configuration: import paths, the `gpu` marker, and on-demand builds.

CPU tests (-m "not gpu") check the oracle against the reference's known
answers, the Python surface and the C-ABI library's exports. GPU tests
(-m gpu) call libvcx through the C ABI and compare with the CPU oracle.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "cake-opt-vc_attention_amd"
for p in (str(PKG), str(ROOT), str(Path(__file__).resolve().parent)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libvcx.so")


@pytest.fixture(scope="session", autouse=True)
def _built_artifacts():
    """Build the oracle and libvcx only if nothing is built yet."""
    from oracle import vc_oracle
    if not vc_oracle._LIB_PATH.exists():
        vc_oracle.build()
    lib = PKG / "lib" / "libvcx.so"
    if not lib.exists():
        sys.path.insert(0, str(PKG))
        import build as vcx_build
        vcx_build.build()
    yield
