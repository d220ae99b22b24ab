import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

# The engine package (directory nexterabert.cpp_amd/) as the module nexterabert_cpp_amd, so
# that test modules can import its submodules (gguf_writer, synth, encoder) by name.
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (built on first use)."""
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def nxg():
    """The engine package (nexterabert.cpp_amd), loaded from the repository."""
    import __graft_entry__
    return __graft_entry__.load_package()
