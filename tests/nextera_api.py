"""ctypes binding of libnexterabert.so derived from include/nexterabert.h itself: every
NEXTERA_API declaration is parsed and bound with the argument and return types it states, so
a test that calls through this table also checks that the header and the library agree.
Shared by tests/test_nextera_api.py (CPU) and tests/test_gpu_nextera_api.py (GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path
from typing import Dict, List, Tuple

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "nexterabert.h"
LIB = ROOT / "nexterabert.cpp_amd" / "libnexterabert.so"


class Params(ctypes.Structure):
    """struct nextera_params, in the order the header declares its fields."""
    _fields_ = [("n_threads", ctypes.c_int32), ("use_int8", ctypes.c_int32),
                ("use_repack", ctypes.c_int32), ("verbosity", ctypes.c_int32)]


def _strip_comments(text: str) -> str:
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))


def declarations(text: str) -> Dict[str, Tuple[str, List[str]]]:
    """name -> (return type, [argument types]) of every NEXTERA_API function declaration,
    whitespace normalised and parameter names dropped."""
    out = {}
    for m in re.finditer(r"NEXTERA_API\s+([^;{]*?)\b(nextera_\w+)\s*\(([^)]*)\)\s*;", _strip_comments(text)):
        ret = " ".join(m.group(1).split())
        args = []
        for a in m.group(3).split(","):
            a = " ".join(a.split())
            if not a or a == "void":
                continue
            a = re.sub(r"\s*\*\s*", " * ", a).strip()
            toks = a.split()
            if len(toks) > 1 and re.fullmatch(r"[a-z_]\w*", toks[-1]) and toks[-1] not in (
                    "int32_t", "double", "float", "char", "nextera_params", "nextera_context"):
                toks = toks[:-1]                                  # the parameter's name
            args.append(" ".join(toks))
        out[m.group(2)] = (" ".join(re.sub(r"\s*\*\s*", " * ", ret).split()), args)
    return out


def struct_fields(text: str) -> List[str]:
    m = re.search(r"struct\s+nextera_params\s*\{(.*?)\};", _strip_comments(text), flags=re.S)
    return [" ".join(f.split()) for f in m.group(1).split(";") if f.strip()]


_CTYPES = {
    "void": None,
    "int32_t": ctypes.c_int32,
    "double": ctypes.c_double,
    "const char *": ctypes.c_char_p,
    "struct nextera_params": Params,
    "struct nextera_context *": ctypes.c_void_p,
    "const struct nextera_context *": ctypes.c_void_p,
    "const int32_t *": ctypes.POINTER(ctypes.c_int32),
    "float *": ctypes.POINTER(ctypes.c_float),
}


def ctype(decl: str):
    if decl not in _CTYPES:
        raise KeyError(f"no ctypes mapping for {decl!r}")
    return _CTYPES[decl]


def bind(path: Path = LIB) -> ctypes.CDLL:
    lib = ctypes.CDLL(str(path))
    for name, (ret, args) in declarations(HEADER.read_text()).items():
        fn = getattr(lib, name)
        fn.restype = ctype(ret)
        fn.argtypes = [ctype(a) for a in args]
    return lib
