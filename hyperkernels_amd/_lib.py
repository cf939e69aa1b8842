"""Loads ``libhk_amd.so`` and binds the C ABI of ``include/hk.h`` through ctypes.

The argument types are read from the header itself (every ``HK_API`` declaration), so the
binding cannot drift from the ABI. torch is imported first on purpose: torch's bundled HIP
runtime has the same soname as ROCm's (``libamdhip64.so.7``), so once torch is loaded the
library resolves to that runtime and shares torch's device allocations and streams.

There is no CPU fallback: if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import pathlib
import re
import threading

import torch  # noqa: F401  (load torch's HIP runtime before the kernel library)

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "libhk_amd.so"
HEADER = PKG.parent / "include" / "hk.h"

_C_TYPES = {
    "void": None,
    "int": ctypes.c_int,
    "int32_t": ctypes.c_int32,
    "int64_t": ctypes.c_int64,
    "long long": ctypes.c_longlong,
    "float": ctypes.c_float,
    "hk_bf16": ctypes.c_uint16,
    "hk_f16": ctypes.c_uint16,
    "hipError_t": ctypes.c_int,
    "hipStream_t": ctypes.c_void_p,
    "size_t": ctypes.c_size_t,
}

_DECL = re.compile(r"HK_API\s+([\w\s\*]+?)\s*\b(hk_\w+)\s*\(([^)]*)\)\s*;", re.S)


def _ctype(decl: str):
    decl = decl.replace("const", " ").strip()
    if decl.endswith("*") or "*" in decl:
        base = decl.replace("*", "").strip()
        return ctypes.c_char_p if base == "char" and decl.count("*") == 1 else ctypes.c_void_p
    if decl not in _C_TYPES:
        raise RuntimeError(f"hk.h: unsupported C type {decl!r}")
    return _C_TYPES[decl]


def parse_header(path: pathlib.Path = HEADER) -> dict[str, tuple[object, list[object]]]:
    """Returns {symbol: (restype, [argtypes])} for every HK_API declaration of the header."""
    text = re.sub(r"/\*.*?\*/", " ", path.read_text(), flags=re.S)
    out: dict[str, tuple[object, list[object]]] = {}
    for ret, name, args in _DECL.findall(text):
        argtypes = []
        args = " ".join(args.split())
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name (last identifier), keep the type with its stars
                m = re.match(r"(.*?)(\w+)$", a)
                if m is None:
                    raise RuntimeError(f"hk.h: cannot parse parameter {a!r} of {name}")
                argtypes.append(_ctype(m.group(1).strip()))
        out[name] = (_ctype(ret.strip()), argtypes)
    return out


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library with every header symbol bound; raises if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m hyperkernels_amd.build` "
                    "(the HIP kernels have no CPU fallback)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in parse_header().items():
                fn = getattr(handle, name)  # AttributeError: symbol missing from the library
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


class HKError(RuntimeError):
    """A C-ABI entry point returned a non-success hipError_t."""

    def __init__(self, fn: str, status: int):
        text = lib().hk_error_string(status)
        super().__init__(f"{fn} failed: hipError {status} ({text.decode() if text else '?'})")
        self.status = status


def call(fn: str, *args) -> None:
    """Calls one entry point and raises HKError on a non-success status."""
    status = getattr(lib(), fn)(*args)
    if status != 0:
        raise HKError(fn, status)
