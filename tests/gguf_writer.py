"""The package's GGUF writer (nexterabert.cpp_amd/gguf_writer.py) under the name the tests import."""
import __graft_entry__

__graft_entry__.load_package()

from nexterabert_cpp_amd.gguf_writer import *  # noqa: E402,F401,F403
from nexterabert_cpp_amd.gguf_writer import _scalar, _string  # noqa: E402,F401
