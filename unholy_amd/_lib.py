"""ctypes binding of libunholy_amd.so, typed from include/unholy_amd.h.

The prototypes are read from the C header itself, so every declared entry point is bound with its argument
types and nothing is declared twice. Calls go through `call(name, *args)`, which raises UhError with the
library's message when an entry point returns nonzero. There is no fallback: if the library is missing the
import of a kernel fails loudly (build it with `python -m unholy_amd.build`).
"""
from __future__ import annotations

import ctypes
import pathlib
import re

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
HEADER = ROOT / "include" / "unholy_amd.h"
LIB_PATH = PKG / "libunholy_amd.so"


class UhError(RuntimeError):
    pass


_SCALARS = {
    "int": ctypes.c_int,
    "unsigned": ctypes.c_uint,
    "size_t": ctypes.c_size_t,
    "float": ctypes.c_float,
    "double": ctypes.c_double,
    "uint64_t": ctypes.c_uint64,
    "uint32_t": ctypes.c_uint32,
    "int32_t": ctypes.c_int32,
    "void": None,
}


def _ctype(decl: str):
    decl = decl.replace("const", " ").strip()
    if "*" in decl:
        base = decl.replace("*", " ").split()
        if base == ["char"]:
            return ctypes.c_char_p
        return ctypes.c_void_p
    words = decl.split()
    # drop the parameter name if present
    if len(words) > 1 and words[-1] not in _SCALARS:
        words = words[:-1]
    key = " ".join(words)
    if key not in _SCALARS:
        raise ValueError(f"unhandled C type in {HEADER.name}: {decl!r}")
    return _SCALARS[key]


def parse_header(path: pathlib.Path = HEADER) -> dict[str, tuple]:
    """name -> (restype, [argtypes]) for every uh_* prototype in the header."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    protos = {}
    for m in re.finditer(r"^[ \t]*([A-Za-z_][\w \t\*]*?)\b(uh_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S | re.M):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        ret_t = _ctype(ret + (" x" if "*" not in ret else ""))
        argt = []
        a = " ".join(args.split())
        if a and a != "void":
            for part in a.split(","):
                part = part.strip()
                if "*" in part:
                    argt.append(_ctype(part))
                else:
                    argt.append(_ctype(part))
        protos[name] = (ret_t, argt)
    return protos


_lib = None
_protos = None
# Entry points whose int result is a value, not a status.
_NOT_STATUS = {"uh_version", "uh_mx_gemm_set_exact", "uh_pack_xxh64"}


def lib() -> ctypes.CDLL:
    global _lib, _protos
    if _lib is None:
        if not LIB_PATH.exists():
            raise UhError(f"{LIB_PATH} is not built: run `python -m unholy_amd.build`")
        l = ctypes.CDLL(str(LIB_PATH))
        _protos = parse_header()
        for name, (rt, at) in _protos.items():
            f = getattr(l, name)  # AttributeError here = a declared symbol the library does not export
            f.restype = rt
            f.argtypes = at
        _lib = l
    return _lib


def prototypes() -> dict[str, tuple]:
    lib()
    return dict(_protos)


def last_error() -> str:
    return lib().uh_last_error().decode()


def call(name: str, *args):
    """Calls an entry point; device buffers may be passed as objects with a `ptr` (kept alive for the call)."""
    f = getattr(lib(), name)
    rc = f(*[a.ptr if hasattr(a, "ptr") else a for a in args])
    if f.restype is ctypes.c_int and name not in _NOT_STATUS and rc != 0:
        raise UhError(f"{name}: {last_error()}")
    return rc
