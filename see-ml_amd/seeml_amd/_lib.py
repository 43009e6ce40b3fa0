"""ctypes binding of the backend's C-ABI (include/seeml_hip.h).

Signatures are read from the header itself, so the Python view can never
drift from the declared boundary. Loading fails loudly when the built
library is missing: there is no CPU fallback for the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import re

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_ROOT = os.path.dirname(PKG_ROOT)
HEADER = os.path.join(REPO_ROOT, "include", "seeml_hip.h")
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libseeml_hip.so")

_TYPES = {
    "int": C.c_int,
    "void": None,
    "float": C.c_float,
    "uint64_t": C.c_uint64,
    "uint32_t": C.c_uint32,
    "int32_t": C.c_int32,
    "double": C.c_double,
    # callback typedefs: passed as a ctypes CFUNCTYPE object cast to c_void_p
    "seeml_hip_tune_reward_fn": C.c_void_p,
    "seeml_hip_arm_reward_fn": C.c_void_p,
}


def _ctype(t: str):
    t = t.strip()
    t = re.sub(r"\s+", " ", t)
    if t == "const char*":
        return C.c_char_p
    if t.endswith("*"):
        return C.c_void_p
    t = t.replace("const ", "")
    if t not in _TYPES:
        raise TypeError(f"unmapped C type in seeml_hip.h: {t!r}")
    return _TYPES[t]


def parse_header(path: str = HEADER) -> dict:
    """name -> (restype, [argtypes]) for every prototype in the header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"^\s*([\w\s\*]+?)\s*\b(seeml_hip_\w+)\s*\(([^;]*?)\)\s*;", text, re.M):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        ret = ret.strip()
        if ret.endswith("*"):
            rtype = C.c_char_p if ret.replace(" ", "") == "constchar*" else C.c_void_p
        else:
            rtype = _ctype(ret)
        argtypes = []
        args = " ".join(args.split())
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                mm = re.match(r"(.*?)(\w+)$", a)
                argtypes.append(_ctype(mm.group(1)))
        protos[name] = (rtype, argtypes)
    return protos


_lib = None


def lib():
    """The loaded backend library with every header prototype bound."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is not built — run __graft_entry__.build() "
                "(hipcc for gfx950); the backend has no CPU fallback")
        # torch ships its own HIP runtime (torch/lib/libamdhip64.so, soname
        # libamdhip64.so.7, linked by that file name). Loaded first, it is
        # the one this library's libamdhip64.so.7 dependency binds to; loaded
        # after this library, torch would bring a second runtime into the
        # process, and this library's HIP calls then fail. The tests and the
        # bench hand this library torch tensors, so torch's runtime goes in
        # first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = C.CDLL(LIB_PATH)
        for name, (rtype, argtypes) in parse_header().items():
            fn = getattr(handle, name)
            fn.restype = rtype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def kernel_error() -> str:
    return lib().seeml_hip_kernel_error().decode()


def check_kernel(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {kernel_error()}")
