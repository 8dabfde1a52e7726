"""Benchmark config c1: the examples/embed.eos pipeline on the GPU against the
oracle (f32 matmul in k order, f64 sum of squares, f16 output) and the
reference known answer (runtime/runtime_test.go:616-686 with the weights of
:1911-1922). f16 results are compared in f16 units in the last place; the
computation order is the oracle's, so they are expected to be identical."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    ai = a.astype(np.float16).view(np.int16).astype(np.int32)
    bi = b.astype(np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def test_tiny_embed_known_answer(rt):
    print("[case] tiny embed known answer", flush=True)
    from eos_amd.encoder import TinyEmbed
    table = np.array([[1, 0], [0, 1], [1, 1]], np.float16)
    m = TinyEmbed(rt, table, np.eye(2, dtype=np.float16))
    out = m.embed(np.array([0, 2], np.int32))
    np.testing.assert_array_equal(out, np.array([[1, 0], [0.70710677, 0.70710677]], np.float16))


def test_tiny_embed_c1_matches_oracle(rt):
    print("[case] tiny embed c1 30522x256 -> 128, T=128", flush=True)
    from eos_amd.encoder import TinyEmbed
    table = (0.02 * datagen.normal(1, 30522 * 256)).astype(np.float16).reshape(30522, 256)
    proj = (0.02 * datagen.normal(101, 256 * 128)).astype(np.float16).reshape(256, 128)
    tokens = datagen.uniform_int(2, 128, 0, 30522).astype(np.int32)
    m = TinyEmbed(rt, table, proj)
    got = m.embed(tokens)
    want = oracle.tiny_embed(table.astype(np.float32), proj.astype(np.float32), tokens)
    u = _ulps(got, want.astype(np.float16))
    print(f"  exact {np.mean(u == 0):.4f}, max ulp {u.max()}", flush=True)
    assert u.max() <= 1
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float32), axis=1), 1.0, atol=2e-3)


def test_tiny_embed_rejects_bad_token(rt):
    print("[case] tiny embed validation", flush=True)
    from eos_amd._lib import EosHipError
    from eos_amd.encoder import TinyEmbed
    m = TinyEmbed(rt, np.ones((5, 8), np.float16), np.ones((8, 4), np.float16))
    with pytest.raises(EosHipError, match="out of range"):
        m.embed(np.array([1, 5], np.int32))
    assert m.embed(np.zeros(0, np.int32)).shape == (0, 4)
