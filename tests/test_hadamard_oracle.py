"""Pins the CPU restatement of the Hadamard TurboQuant codec
(oracle/retrieval_oracle.c hq_*), test infrastructure for the eos_hq_* kernels.

* The normalized FWHT against the closed form H[i][j] = (-1)^popcount(i & j)
  / sqrt(2^k) on basis vectors, its block structure on widths that are not a
  power of two, and its involution (applying it twice returns the input).
* The 8-bit log norm code against known answers of quantizeQNorm /
  dequantizeQNorm (runtime/backend/image_ops.go:759-780; the reference test
  fixture image_ops_test.go:157 uses quantizeQNorm(1)).
* Encode against its definition computed independently in numpy (rotation,
  nearest centroid by brute force when the boundaries are midpoints), and
  the encode -> decode round trip against the bound that the norm code and
  the codebook spacing give."""
import numpy as np
import pytest

import oracle


def _hadamard(k):
    n = 1 << k
    i = np.arange(n)
    return np.where(np.bitwise_count(i[:, None] & i[None, :]) % 2 == 0, 1.0, -1.0) / np.sqrt(n)


@pytest.mark.parametrize("k", [0, 1, 2, 3, 5, 7, 9])
def test_fwht_closed_form(k):
    n = 1 << k
    H = _hadamard(k).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(n))
    for j in sorted({0, min(1, n - 1), n - 1, n // 3}):
        e = np.zeros(n, np.float32)
        e[j] = 1
        got = oracle.hq_fwht(e)
        np.testing.assert_array_equal(got, np.sign(H[:, j]) * scale if n > 1 else e)


def test_fwht_blocks_and_involution():
    rng = np.random.default_rng(0)
    for c in [13, 96, 100, 511]:
        x = rng.normal(size=c).astype(np.float32)
        got = oracle.hq_fwht(x).astype(np.float64)
        want, off, rem = np.zeros(c), 0, c
        while rem:
            size = 1 << (rem.bit_length() - 1)
            k = size.bit_length() - 1
            want[off:off + size] = _hadamard(k) @ x[off:off + size].astype(np.float64)
            off += size
            rem -= size
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(oracle.hq_fwht(oracle.hq_fwht(x)), x, rtol=1e-5, atol=1e-6)


def test_norm_code_known_answers():
    assert oracle.hq_norm_code(1.0) == 128          # t = 0.5, 127.5 rounds away from zero
    assert oracle.hq_norm_code(0.0) == 0 and oracle.hq_norm_code(-1.0) == 0
    assert oracle.hq_norm_code(float("nan")) == 0 and oracle.hq_norm_code(float("inf")) == 255
    assert oracle.hq_norm_code(np.exp(-17.0)) == 0 and oracle.hq_norm_code(np.exp(17.0)) == 255
    assert oracle.hq_norm_code(np.exp(-16.0 + 32.0 * 10 / 255)) == 10
    assert oracle.hq_norm_value(0) == np.float32(np.exp(-16.0))
    assert oracle.hq_norm_value(255) == np.float32(np.exp(16.0))
    assert oracle.hq_norm_value(128) == np.float32(np.exp(-16.0 + 32.0 * 128 / 255))
    for code in range(256):
        assert oracle.hq_norm_code(oracle.hq_norm_value(code)) == code


def _spec(c, bits, seed):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(c).astype(np.int32)
    s1 = rng.choice([-1.0, 1.0], c).astype(np.float32)
    s2 = rng.choice([-1.0, 1.0], c).astype(np.float32)
    levels = 1 << bits
    cent = np.sort(rng.normal(size=levels) / np.sqrt(c)).astype(np.float32)
    bnd = ((cent[:-1].astype(np.float64) + cent[1:]) / 2).astype(np.float32)
    return perm, s1, s2, cent, bnd, levels


def test_encode_matches_definition():
    rng = np.random.default_rng(1)
    c, bits = 48, 4
    perm, s1, s2, cent, bnd, levels = _spec(c, bits, 2)
    x = rng.normal(size=(2, c, 3, 5)).astype(np.float32)
    coords, norms = oracle.hq_encode(x, perm, s1, s2, bnd, levels)
    for img in range(2):
        for y in range(3):
            for xx in range(5):
                v = x[img, :, y, xx].astype(np.float64)
                norm = np.sqrt((v * v).sum())
                work = v[perm] / norm * s1
                off, rem = 0, c
                while rem:
                    size = 1 << (rem.bit_length() - 1)
                    work[off:off + size] = _hadamard(size.bit_length() - 1) @ work[off:off + size]
                    off += size
                    rem -= size
                rot = np.zeros(c)
                rot[perm] = work * s2
                want = np.abs(rot[:, None] - cent[None, :].astype(np.float64)).argmin(axis=1)
                # brute-force nearest centroid (boundaries are midpoints); a
                # value within 1e-6 of a boundary may fall either side
                near = np.abs(rot[:, None] - bnd[None, :]).min(axis=1) < 1e-6
                got = coords[img, :, y, xx]
                assert np.all((got == want) | near)
                assert norms[img, y, xx] == oracle.hq_norm_code(np.float32(norm))


def test_round_trip_bound():
    rng = np.random.default_rng(3)
    c, bits = 64, 8
    perm, s1, s2, _, _, levels = _spec(c, bits, 4)
    cent = np.linspace(-0.5, 0.5, levels).astype(np.float32)   # fine uniform codebook
    bnd = ((cent[:-1].astype(np.float64) + cent[1:]) / 2).astype(np.float32)
    x = rng.normal(size=(1, c, 4, 4)).astype(np.float32)
    coords, norms = oracle.hq_encode(x, perm, s1, s2, bnd, levels)
    back = oracle.hq_decode(coords, norms, perm, s1, s2, cent, levels)
    a = x.reshape(c, -1).T.astype(np.float64)
    b = back.reshape(c, -1).T.astype(np.float64)
    cos = (a * b).sum(1) / np.linalg.norm(a, axis=1) / np.linalg.norm(b, axis=1)
    assert cos.min() > 0.9995
    ratio = np.linalg.norm(b, axis=1) / np.linalg.norm(a, axis=1)
    assert np.all(np.abs(np.log(ratio)) < 16.0 / 255 + 0.01)
