"""GPU parity of the inner-product first stage (eoship_tq_ip_bind_corpus +
eoship_tq_ip_topk_device: the promoted profile's IPQuantized top-k) against
the CPU oracle: tq_ip_scores (the same estimator) then the (score desc,
index asc) top-k. Bar: bit-exact ids and scores (integer dots, fixed f32
expression)."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen
from eos_amd.turboquant import IPQuantizer

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _setup(d, mse_bits, seed):
    rng = np.random.default_rng(seed)
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32)
    S = rng.normal(size=(d, d)).astype(np.float32)
    cb, s_c = datagen.turboquant_codebook(mse_bits, d)
    return rng, rot, S, np.asarray(cb, np.int8), s_c


def _want(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm, k):
    sc = oracle.tq_ip_scores(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm)
    ids, scs = [], []
    for row in sc:
        i, s = oracle.topk_scores(row, k)
        ids.append(i)
        scs.append(s)
    return np.stack(ids), np.stack(scs)


@pytest.mark.parametrize("d,bits,n,k", [(384, 3, 20_000, 100), (256, 2, 9_000, 50),
                                        (100, 1, 5_003, 10), (512, 3, 7_777, 200)])
def test_ip_topk_matches_oracle(rt, d, bits, n, k):
    """Encoded vectors (the GPU encoder), duplicated rows (ties by index),
    a partial last tile, dimensions not a multiple of 32, and more queries
    than one batch."""
    _case(f"ip top-k d={d} mse bits={bits} n={n} k={k}")
    rng, rot, S, cb, s_c = _setup(d, bits, d + bits)
    qz = IPQuantizer(rt, d, bits, cb, s_c, rot, S)
    x = rng.normal(size=(n, d)).astype(np.float32)
    x[17] = x[4000]
    x[18] = x[4000]
    codes, signs, rn, nm = qz.encode(x)
    oc, osg, orn, onm = oracle.tq_encode_ip(x[:64], rot, S, d, bits, cb, s_c)
    np.testing.assert_array_equal(codes[:64], oc)
    np.testing.assert_array_equal(signs[:64], osg)
    idx = qz.bind(codes, signs, rn, nm)
    q = rng.normal(size=(70, d)).astype(np.float32)
    q[3] = x[4000]
    ids, sc = idx.top_k(q, k)
    wid, wsc = _want(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm, k)
    np.testing.assert_array_equal(ids, wid)
    np.testing.assert_array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    assert ids[3][:3].tolist() == [17, 18, 4000]
    idx.release()
    qz.release()


def test_ip_topk_small_corpus_and_k_edges(rt):
    """n below the candidate capacity (no sample pass), k = 0 (all), k > n."""
    _case("ip top-k small corpus")
    d, bits = 64, 3
    rng, rot, S, cb, s_c = _setup(d, bits, 5)
    qz = IPQuantizer(rt, d, bits, cb, s_c, rot, S)
    x = rng.normal(size=(300, d)).astype(np.float32)
    codes, signs, rn, nm = qz.encode(x)
    idx = qz.bind(codes, signs, rn, nm)
    q = rng.normal(size=(5, d)).astype(np.float32)
    for k in (0, 1, 300, 1000):
        ids, sc = idx.top_k(q, k)
        wid, wsc = _want(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm, k)
        np.testing.assert_array_equal(ids, wid)
        np.testing.assert_array_equal(sc, wsc)
    idx.release()
    qz.release()


def test_ip_bind_refuses_bad_norms(rt):
    _case("ip bind norm policy")
    from eos_amd._lib import EosHipError
    d, bits = 64, 3
    rng, rot, S, cb, s_c = _setup(d, bits, 6)
    qz = IPQuantizer(rt, d, bits, cb, s_c, rot, S)
    x = rng.normal(size=(40, d)).astype(np.float32)
    x[5] = 0
    codes, signs, rn, nm = qz.encode(x)
    assert nm[5] == 0
    with pytest.raises(EosHipError, match="Norm 0"):
        qz.bind(codes, signs, rn, nm)
    zv = np.zeros(40, np.uint8)
    zv[5] = 1
    idx = qz.bind(codes, signs, rn, nm, zero_vector_allowed=zv)
    ids, sc = idx.top_k(rng.normal(size=(2, d)).astype(np.float32), 40)
    assert sorted(ids[0].tolist()) == list(range(40))
    idx.release()
    bad = nm.copy()
    bad[3] = -1
    with pytest.raises(EosHipError, match="invalid norm"):
        qz.bind(codes, signs, rn, bad)
    qz.release()
