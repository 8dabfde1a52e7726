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
    assert _lib.load().eoship_abi_version() == 6


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


def test_turboquant_vector_bytes():
    """turboquantVectorBytes (runtime/turboquant_bytes.go:14-25): the published
    136 B at dim 256 / bit width 4 (docs/anchors/eos-mixed-rerank-eval-v021/
    nfcorpus.b4-o200-fp16.metrics.json:10,79), 248 B at dim 384 / bit width 5
    (4-bit MSE + signs + both norms), and the reference test's cases as
    ceil(d (b - 1) / 8) + ceil(d / 8) + 8."""
    from eos_amd.turboquant import turboquant_mse_vector_bytes, turboquant_vector_bytes
    assert turboquant_vector_bytes(256, 4) == 136
    assert turboquant_vector_bytes(384, 5) == 248
    for d, b in ((8, 1), (8, 2), (128, 2), (128, 4), (128, 8), (256, 4), (3072, 8)):
        assert turboquant_vector_bytes(d, b) == -(-d * (b - 1) // 8) + -(-d // 8) + 8
    assert turboquant_mse_vector_bytes(384, 4) == 196     # the benchmark's c2 layout
    assert turboquant_mse_vector_bytes(128, 2) == 36      # c5
    assert turboquant_mse_vector_bytes(40, 4) == 24
    with pytest.raises(_lib.EosHipError):
        turboquant_vector_bytes(0, 4)
    with pytest.raises(_lib.EosHipError):
        turboquant_vector_bytes(64, 9)


def test_string_id_rank_is_go_string_order():
    from eos_amd.turboquant import string_id_rank
    ids = ["d2", "d10", "d1", "b", "B", "é", "e"]
    # bytewise: "B" < "b" < "d1" < "d10" < "d2" < "e" < "é" (0xc3 0xa9)
    assert list(string_id_rank(ids)) == [4, 3, 2, 1, 0, 6, 5]
    with pytest.raises(ValueError):
        string_id_rank(["a", "a"])
