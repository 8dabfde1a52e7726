"""Run by tests/test_sanitize.py in a process that preloads the ASan/UBSan
runtimes: drives the sanitized builds of the host shim (the MLL reader, the
plan classifiers, BLAKE3, byte accounting; no GPU call) and of the C oracle
over valid and corrupted inputs. Any sanitizer report aborts the process."""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

from eos_amd import _lib  # noqa: E402

_lib.LIB_PATH = sys.argv[1]
import oracle  # noqa: E402

oracle.LIB_PATH = sys.argv[2]

from eos_amd._lib import EosHipError  # noqa: E402
from eos_amd.mll import MllPackage  # noqa: E402
from oracle.blake3 import blake3  # noqa: E402

import mll_synth  # noqa: E402

SHIPPED = os.path.join(HERE, "golden", "default_embedder", "corkscrewdb-default-embedder.mll")


def exercise(data: bytes) -> bool:
    """Open, walk and classify a package; False if the reader refused it."""
    try:
        with MllPackage(data) as m:
            for i in range(m.n_tensors):
                m.tensor(i)
            for tag in ("STRG", "TNSR", "XMTA", "ZZZZ"):
                try:
                    m.section(tag)
                except EosHipError:
                    pass
            for fn in (m.classify, lambda: _classify_retrieval(m)):
                try:
                    fn()
                except EosHipError:
                    pass
        return True
    except EosHipError:
        return False


def _classify_retrieval(m):
    import ctypes as C
    plan = _lib.EosHipRetrievalPlan()
    _lib.call("eoship_mll_classify_retrieval", m.handle, None, C.byref(plan))


def resealed(data: bytes, tag: str, body: bytes) -> bytes:
    """data with section `tag` replaced by `body` (same size) and its digest
    recomputed, so the parsers behind the digest check see the bytes."""
    n = struct.unpack_from("<Q", data, 16)[0]
    for i in range(n):
        e = 24 + 64 * i
        if data[e:e + 4].decode("latin-1") == tag:
            off, size = struct.unpack_from("<QQ", data, e + 4)
            assert len(body) == size
            out = bytearray(data)
            out[off:off + size] = body
            out[e + 20:e + 52] = blake3(body)
            return bytes(out)
    raise KeyError(tag)


def section_body(data: bytes, tag: str) -> bytes:
    n = struct.unpack_from("<Q", data, 16)[0]
    for i in range(n):
        e = 24 + 64 * i
        if data[e:e + 4].decode("latin-1") == tag:
            off, size = struct.unpack_from("<QQ", data, e + 4)
            return data[off:off + size]
    raise KeyError(tag)


def main():
    rng = np.random.default_rng(20261202)
    shipped = open(SHIPPED, "rb").read()
    assert exercise(shipped)
    small = mll_synth.package(*_synth())
    assert exercise(small)
    # the shipped package: framing damage only (every open hashes its 4.9 MB)
    for cut in (0, 3, 8, 23, 24, 88, len(shipped) // 2, len(shipped) - 1):
        exercise(shipped[:cut])
    for pos in (4, 5, 8, 16, 24 + 4, 24 + 12, 24 + 52, 24 + 64 * 9 + 4):
        bad = bytearray(shipped)
        bad[pos] ^= 0x40
        exercise(bytes(bad))
    for data in (small,):
        # truncations and framing damage
        for cut in sorted(set(rng.integers(0, len(data), 24).tolist()) | {0, 3, 8, 23, 24, 87, 88}):
            exercise(data[:cut])
        for pos in rng.integers(0, min(len(data), 24 + 64 * 14), 40):
            bad = bytearray(data)
            bad[pos] ^= 1 << int(rng.integers(0, 8))
            exercise(bytes(bad))
        # damage behind the digest check: bytes of STRG / TNSR / XMTA changed
        # and the section resealed
        for tag in ("STRG", "TNSR", "XMTA"):
            body = section_body(data, tag)
            if not body:
                continue
            for _ in range(25):
                b = bytearray(body)
                for pos in rng.integers(0, len(b), int(rng.integers(1, 4))):
                    b[pos] = int(rng.integers(0, 256))
                exercise(resealed(data, tag, bytes(b)))
            for val in (0, 0xFFFFFFFF, 0x7FFFFFFF, 1 << 20):
                b = bytearray(body)
                struct.pack_into("<I", b, 0, val)
                exercise(resealed(data, tag, bytes(b)))
    # BLAKE3 over block, chunk and tree edges
    import ctypes as C
    for n in (0, 1, 64, 1023, 1024, 1025, 4096, 9000):
        payload = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        out = (C.c_uint8 * 32)()
        _lib.call("eoship_blake3", C.c_char_p(payload) if payload else None, C.c_uint64(n), out)
        assert bytes(out) == blake3(payload)
    # byte accounting, valid and refused arguments
    for dim, bits in ((256, 4), (384, 2), (1, 1), (0, 4), (-3, 4), (256, 3), (1 << 30, 8)):
        nb = C.c_int64()
        try:
            _lib.call("eoship_tq_vector_bytes", C.c_int32(dim), C.c_int32(bits), C.byref(nb))
        except EosHipError:
            pass
    # the C oracle on small inputs of every family
    _oracle_smoke(rng)
    print("OK", flush=True)


def _synth():
    layers = [dict(q="q1", k="k1", v="v1", o="o1", up="up1", down="down1")] * 2
    names = ["token_embedding"] + sorted(set(layers[0].values()))
    w = mll_synth.weights(50, 32, 64, names, seed=7)
    return mll_synth.encoder_artifact(layers, masked=True), w


def _oracle_smoke(rng):
    from eos_amd import datagen
    c = datagen.TurboQuantCorpus(300, 48, 4, 1, 2, 3)
    q = datagen.unit_rows(datagen.normal(5, 3 * 48).reshape(3, 48)).astype(np.float32)
    oracle.tq_scores(q, c.rotation, 48, 4, c.codebook, c.codebook_scale, c.codes, c.norms)
    oracle.tq_topk(q, c.rotation, 48, 4, c.codebook, c.codebook_scale, c.codes, c.norms, 10)
    x = rng.normal(size=(20, 48)).astype(np.float32)
    oracle.tq_encode(x, c.rotation, 48, 4, c.codebook, c.codebook_scale)
    perm = rng.permutation(12).astype(np.int32)
    s1 = rng.choice([-1.0, 1.0], 12).astype(np.float32)
    s2 = rng.choice([-1.0, 1.0], 12).astype(np.float32)
    cent = np.sort(rng.normal(size=4)).astype(np.float32)
    bnd = ((cent[:-1] + cent[1:]) / 2).astype(np.float32)
    img = rng.normal(size=(2, 12, 3, 5)).astype(np.float32)
    co, nc = oracle.hq_encode(img, perm, s1, s2, bnd, 4)
    oracle.hq_decode(co, nc, perm, s1, s2, cent, 4)
    docs = rng.normal(size=(30, 17)).astype(np.float32)
    for op in ("dot", "cosine", "l2_distance"):
        oracle.score_rows(op, docs[0], docs)


if __name__ == "__main__":
    main()
