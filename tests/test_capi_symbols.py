"""The C ABI library loads without a GPU and exports every entry point that
include/tkv_hip.h declares (no compute calls here)."""
import ctypes as C
import os
import re
import subprocess

from tokenvector.inference_amd import _lib


def _declared():
    return set(_lib.parse_header().keys())


def test_header_parses_every_prototype():
    text = open(_lib.HEADER_PATH).read()
    raw = set(re.findall(r"\b(tkv_hip_\w+)\s*\(", text))
    assert raw == _declared()
    assert len(raw) >= 50


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "build libtkv_hip.so first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (tkv_hip_\w+)", out))
    missing = _declared() - exported
    assert not missing, sorted(missing)


def test_library_loads_and_binds():
    L = _lib.lib()
    for name in _declared():
        assert getattr(L, name) is not None
    assert L.tkv_hip_version() >= 100
    buf = C.create_string_buffer(16)
    assert L.tkv_hip_last_error(buf, 16) >= 0


def test_rc_mapping():
    import pytest
    assert _lib.check(_lib.OK) == 0
    with pytest.raises(ValueError):
        _lib.check(_lib.BAD_ARG)
    with pytest.raises(_lib.TkvHipError):
        _lib.check(_lib.UNSUPPORTED)
