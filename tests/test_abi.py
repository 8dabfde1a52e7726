"""The C-ABI library loads and exports every symbol include/eoship.h declares
(no compute calls: CPU only)."""
import ctypes
import os
import re

import pytest

from eos_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:int|void|int64_t)\s+(eoship_\w+)\s*\(", text, re.M))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 25
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert declared == set(_lib.exported_symbols())


def test_abi_version():
    assert _lib.load().eoship_abi_version() == 4


def test_runtime_create_without_gpu_fails_cleanly():
    """On a host without a gfx950 device the runtime refuses with a message."""
    import torch  # only to ask whether a device exists
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(_lib.EosHipError):
        from eos_amd.runtime import Runtime
        Runtime(0)


def test_null_arguments_are_errors():
    lib = _lib.load()
    err = ctypes.c_char_p()
    assert lib.eoship_runtime_create(0, None, ctypes.byref(err)) != 0
    assert b"NULL" in err.value
    lib.eoship_free_cstring(ctypes.cast(err, ctypes.c_void_p))
    assert lib.eoship_sync(None, None) != 0
    assert lib.eoship_runtime_destroy(None, None) == 0
