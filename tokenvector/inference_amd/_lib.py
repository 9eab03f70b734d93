"""ctypes binding of libtkv_hip, generated from ``include/tkv_hip.h``.

Every ``int32_t tkv_hip_*(...)`` prototype of the public header is bound
with matching argument types, so the header is the single source of truth
for the C ABI.  Loading fails loudly: there is no CPU fallback behind this
module.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libtkv_hip.so")
HEADER_PATH = os.path.abspath(os.path.join(_PKG, "..", "..", "include", "tkv_hip.h"))
CSRC = os.path.join(_PKG, "csrc")

OK = 0
UNSUPPORTED = -1
NO_DEVICE = -2
OOM = -3
BAD_ARG = -4
DEVICE_ERROR = -5


class TkvHipError(RuntimeError):
    """A libtkv_hip call returned a negative rc other than BAD_ARG."""

    def __init__(self, rc: int, msg: str):
        super().__init__(f"libtkv_hip rc={rc}: {msg}")
        self.rc = rc


class QParamsDev(C.Structure):
    """tkv_hip_qparams_dev (device-resident per-tensor parameters)."""
    _fields_ = [("scale", C.c_float), ("min_val", C.c_float), ("max_val", C.c_float),
                ("zero_point", C.c_int32), ("inv", C.c_double), ("reserved", C.c_double)]


_SCALARS = {
    "int32_t": C.c_int32,
    "int64_t": C.c_int64,
    "float": C.c_float,
    "double": C.c_double,
    "void": None,
}


def _ctype(decl: str):
    decl = decl.strip()
    if "*" in decl:
        return C.c_void_p
    words = [w for w in decl.replace("const ", "").split() if w]
    return _SCALARS[words[0]]


def parse_header(path: str = HEADER_PATH):
    """Return {name: (restype, [argtypes])} for every tkv_hip_* prototype."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    protos = {}
    for m in re.finditer(r"\b(int32_t|void)\s+(tkv_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        argtypes = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name
                a = re.sub(r"\b\w+$", "", a) if not a.endswith("*") else a
                argtypes.append(_ctype(a))
        protos[name] = (_SCALARS[ret], argtypes)
    return protos


def build() -> None:
    """Compile every HIP source for gfx950 into libtkv_hip.so (hipcc)."""
    jobs = str(min(16, os.cpu_count() or 4))
    subprocess.run(["make", "-s", "-j", jobs, "-C", CSRC], check=True)


_lib = None


def lib() -> C.CDLL:
    """Load libtkv_hip.so.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C {CSRC}` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in parse_header().items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(1024)
    lib().tkv_hip_last_error(buf, 1024)
    return buf.value.decode(errors="replace")


def check(rc: int) -> int:
    """Map an rc to the reference's error behaviour: BAD_ARG is the
    ValueError the .tkv function raises; anything else negative is fatal."""
    if rc == OK:
        return rc
    msg = last_error()
    if rc == BAD_ARG:
        raise ValueError(msg)
    raise TkvHipError(rc, msg)
