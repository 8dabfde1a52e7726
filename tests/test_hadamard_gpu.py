"""GPU parity of the Hadamard TurboQuant codec (eos_hq_encode /
eos_hq_decode) against its CPU restatement (oracle hq_encode / hq_decode).
Bar: bit-exact centroid indices, norm codes and decoded values."""
import numpy as np
import pytest

import oracle
from eos_amd._lib import EosHipError
from eos_amd.hadamard import HadamardTQ

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _spec(c, bits, seed):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(c).astype(np.int32)
    s1 = rng.choice([-1.0, 1.0], c).astype(np.float32)
    s2 = rng.choice([-1.0, 1.0], c).astype(np.float32)
    levels = 1 << bits
    cent = np.sort(rng.normal(size=levels) / np.sqrt(c)).astype(np.float32)
    bnd = ((cent[:-1].astype(np.float64) + cent[1:]) / 2).astype(np.float32)
    return perm, s1, s2, cent, bnd


@pytest.mark.parametrize("c,bits,shape", [(5, 4, (1, 2, 2)), (64, 2, (2, 16, 16)),
                                          (96, 8, (3, 7, 9)), (512, 4, (1, 8, 8)),
                                          (200, 8, (2, 33, 1))])
def test_codec_matches_oracle(rt, c, bits, shape):
    _case(f"hadamard codec C={c} bits={bits} shape={shape}")
    rng = np.random.default_rng(c * 10 + bits)
    n, h, w = shape
    perm, s1, s2, cent, bnd = _spec(c, bits, c + bits)
    x = (rng.normal(size=(n, c, h, w)) * np.exp(rng.normal(size=(n, 1, h, w)) * 3)).astype(np.float32)
    x[0, :, 0, 0] = 0.0                                  # zero vector: scale 1, code 0
    if h * w > 2:
        x.reshape(n, c, h * w)[0, :, 1] *= np.float32(1e-9)   # below the norm code's range
    codec = HadamardTQ(rt, perm, s1, s2, cent, bnd, bits)
    coords, norms = codec.encode(x)
    wc, wn = oracle.hq_encode(x, perm, s1, s2, bnd, 1 << bits)
    np.testing.assert_array_equal(coords, wc)
    np.testing.assert_array_equal(norms, wn)
    back = codec.decode(coords, norms)
    np.testing.assert_array_equal(back, oracle.hq_decode(coords, norms, perm, s1, s2, cent, 1 << bits))
    codec.release()


def test_codec_rejects_bad_tables(rt):
    _case("hadamard codec table validation")
    perm, s1, s2, cent, bnd = _spec(8, 4, 1)
    bad = perm.copy()
    bad[0] = bad[1]
    with pytest.raises(EosHipError, match="permutation"):
        HadamardTQ(rt, bad, s1, s2, cent, bnd, 4)
    with pytest.raises(EosHipError, match="non-decreasing"):
        HadamardTQ(rt, perm, s1, s2, cent, bnd[::-1].copy(), 4)
    with pytest.raises(EosHipError, match="bits"):
        HadamardTQ(rt, perm, s1, s2, np.zeros(8, np.float32), np.zeros(7, np.float32), 3)
