"""Pins the TurboQuant CPU oracle (oracle/tq_oracle.c) against known answers,
closed forms and brute force, and checks the host-side layout logic the GPU
scan depends on. CPU only."""
import math

import numpy as np
import pytest

import oracle
from eos_amd import datagen

# Lloyd-Max reconstruction points of N(0,1) (J. Max, 1960, Table I).
MAX_1960 = {
    4: [0.4528, 1.5104],
    16: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326],
}


@pytest.mark.parametrize("levels", [4, 16])
def test_lloyd_max_matches_max_1960(levels):
    c = datagen.lloyd_max_normal(levels)
    pos = c[levels // 2:]
    np.testing.assert_allclose(pos, MAX_1960[levels], atol=6e-4)
    np.testing.assert_allclose(c, -c[::-1], atol=1e-12)


def test_codebook_grid():
    cb, s = datagen.turboquant_codebook(4, 384)
    assert cb.dtype == np.int8 and cb.shape == (16,)
    assert int(np.max(np.abs(cb))) == 127
    c = datagen.lloyd_max_normal(16) / math.sqrt(384)
    assert np.max(np.abs(cb * s - c)) <= 0.5 * s * 1.0001


def test_splitmix64_known_answer():
    # splitmix64 reference outputs for seed 0 (Vigna's splitmix64.c).
    out = datagen.splitmix64(0, 3)
    assert [int(x) for x in out] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_unpack_roundtrip(bits):
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 1 << bits, size=(17, 45))
    packed = datagen.pack_codes(codes, bits)
    assert packed.shape == (17, (45 * bits + 7) // 8)
    np.testing.assert_array_equal(datagen.unpack_codes(packed, bits, 45), codes)
    if bits == 4:  # low nibble first, as the q4 packer (runtime/mll_export.go:950-958)
        assert packed[0, 0] == (codes[0, 0] | (codes[0, 1] << 4))


def _small(n=300, d=64, bits=4, seed=11, rotation=True):
    corpus = datagen.TurboQuantCorpus(n, d, bits, seed, seed + 1, seed + 2, rotation=rotation)
    q = datagen.baseline_queries(5, d, seed + 3)
    return corpus, q


@pytest.mark.parametrize("bits,d", [(4, 64), (2, 32), (4, 384)])
def test_dots_brute_force(bits, d):
    corpus, q = _small(n=200, d=d, bits=bits)
    qs, alpha = oracle.tq_prepare(q[0], corpus.rotation, corpus.codebook, corpus.codebook_scale)
    codes = datagen.unpack_codes(corpus.codes, bits, d)
    want = (corpus.codebook.astype(np.int64)[codes] @ qs.astype(np.int64))
    got = oracle.tq_dots(qs, corpus.codes, bits, corpus.codebook)
    np.testing.assert_array_equal(got, want)


def test_prepare_permutation_closed_form():
    """R = permutation: q' is q permuted exactly; Qs = rint(q' * qmax / max|q'|)."""
    d = 64
    perm = np.random.default_rng(1).permutation(d)
    R = np.zeros((d, d), np.float32)
    R[np.arange(d), perm] = 1.0
    q = datagen.baseline_queries(1, d, 9)[0]
    cb, s = datagen.turboquant_codebook(4, d)
    qs, alpha = oracle.tq_prepare(q, R, cb, s)
    qp = q.astype(np.float64)[perm]
    qmax = oracle.tq_qmax(cb, d)
    m = np.max(np.abs(qp))
    np.testing.assert_array_equal(qs, np.rint(qp * (qmax / m)).astype(np.int16))
    assert alpha == np.float32((m / qmax) * float(np.float32(s)))


def test_one_hot_query_scores_centroid():
    """R = I, query e_j: score = Norm * c[code_j] (the closed form of the estimator)."""
    corpus, _ = _small(n=64, d=32, bits=4, rotation=False)
    cb, s = corpus.codebook, corpus.codebook_scale
    codes = datagen.unpack_codes(corpus.codes, 4, 32)
    for j in (0, 7, 31):
        q = np.zeros((1, 32), np.float32)
        q[0, j] = 1.0
        _, sc = oracle.tq_scores(q, None, 32, 4, cb, s, corpus.codes, corpus.norms)
        want = corpus.norms.astype(np.float64) * s * cb[codes[:, j]].astype(np.float64)
        np.testing.assert_allclose(sc[0], want, rtol=2e-6, atol=1e-12)


def test_zero_norm_and_zero_query():
    corpus, q = _small(n=40, d=32, bits=4)
    norms = corpus.norms.copy()
    norms[[3, 5]] = 0.0
    _, sc = oracle.tq_scores(q, corpus.rotation, 32, 4, corpus.codebook, corpus.codebook_scale,
                             corpus.codes, norms)
    assert np.all(sc[:, [3, 5]] == 0.0)
    assert not np.any(np.signbit(sc[:, [3, 5]]))
    zq = np.zeros((1, 32), np.float32)
    ids, s = oracle.tq_topk(zq, corpus.rotation, 32, 4, corpus.codebook, corpus.codebook_scale,
                            corpus.codes, norms, 7)
    np.testing.assert_array_equal(ids[0], np.arange(7))
    assert np.all(s == 0.0)


@pytest.mark.parametrize("bits,d", [(4, 384), (2, 128)])
def test_integer_scores_within_tolerance_of_float_estimator(bits, d):
    """Scores meet the 1e-4 relative contract against the f64 estimator, and the
    deviation stays inside the bound the int16 query rounding implies."""
    corpus, q = _small(n=500, d=d, bits=bits)
    dots, sc = oracle.tq_scores(q, corpus.rotation, d, bits, corpus.codebook,
                                corpus.codebook_scale, corpus.codes, corpus.norms)
    ref = oracle.tq_scores_f64(q, corpus.rotation, d, bits, corpus.codebook,
                               corpus.codebook_scale, corpus.codes, corpus.norms)
    codes = datagen.unpack_codes(corpus.codes, bits, d)
    cvals = corpus.codebook_scale * corpus.codebook.astype(np.float64)[codes]
    qmax = oracle.tq_qmax(corpus.codebook, d)
    for i in range(q.shape[0]):
        qp = corpus.rotation.astype(np.float64) @ q[i].astype(np.float64)
        sq = np.max(np.abs(qp)) / qmax
        bound = corpus.norms * (0.5 * sq * np.sum(np.abs(cvals), axis=1)) + 4e-7 * np.abs(ref[i])
        assert np.all(np.abs(sc[i] - ref[i]) <= bound * 1.001 + 1e-30)
        scale = corpus.norms * np.linalg.norm(qp) * np.linalg.norm(cvals, axis=1)
        assert np.max(np.abs(sc[i] - ref[i]) / scale) < 1e-4


def test_topk_heap_matches_full_sort_with_planted_ties():
    rng = np.random.default_rng(3)
    s = rng.integers(0, 5, size=1000).astype(np.float32)  # many exact ties
    for k in (1, 7, 100, 999, 1000, 0, 5000):
        ids, out = oracle.topk_scores(s, k)
        order = np.lexsort((np.arange(1000), -s))
        kk = 1000 if (k <= 0 or k > 1000) else k
        np.testing.assert_array_equal(ids, order[:kk])
        np.testing.assert_array_equal(out, s[order[:kk]])


def test_topk_tie_to_lower_id_reference_case():
    """runtime/turboquant_retrieval_pruning_test.go:80-99: two zero vectors tie,
    the lower ID wins the single slot."""
    corpus, q = _small(n=2, d=32, bits=4)
    norms = np.zeros(2, np.float32)
    ids, s = oracle.tq_topk(q[:1], corpus.rotation, 32, 4, corpus.codebook, corpus.codebook_scale,
                            corpus.codes, norms, 1)
    assert ids[0, 0] == 0 and s[0, 0] == 0.0


@pytest.mark.parametrize("bits,d", [(4, 384), (2, 128), (4, 40)])
def test_topk_equals_exhaustive_sort(bits, d):
    corpus, q = _small(n=2000, d=d, bits=bits)
    _, sc = oracle.tq_scores(q, corpus.rotation, d, bits, corpus.codebook, corpus.codebook_scale,
                             corpus.codes, corpus.norms)
    for k in (1, 7, 100, 255):
        ids, s = oracle.tq_topk(q, corpus.rotation, d, bits, corpus.codebook,
                                corpus.codebook_scale, corpus.codes, corpus.norms, k)
        for i in range(q.shape[0]):
            order = np.lexsort((np.arange(2000), -sc[i]))[:k]
            np.testing.assert_array_equal(ids[i], order)
            np.testing.assert_array_equal(s[i], sc[i][order])


# ---------------------------------------------------------------- layout model
# Python model of the device pack (eos_tq_pack) and decode (decode_step):
# decode(pack(codes)) must place codebook value C[code_{v,k}] at fragment byte i
# of K-step s for lane group g exactly when k = 32 s + 16 g + i.

def _perm(s0, s1, sel):
    data = (int(s0) << 32) | int(s1)
    out = 0
    for b in range(4):
        s = (sel >> (8 * b)) & 0xFF
        if s >= 13:
            v = 0xFF
        elif s == 12:
            v = 0
        elif s in (8, 9, 10, 11):
            bit = {8: 15, 9: 31, 10: 47, 11: 63}[s]
            v = 0xFF if (data >> bit) & 1 else 0
        else:
            v = (data >> (8 * s)) & 0xFF
        out |= v << (8 * b)
    return out


def _solve_lut4(cb):
    c = [int(x) & 0xFF for x in cb]
    sx = lambda b: 0xFF if b & 0x80 else 0
    kb = [0] * 8
    ka = [0] * 16
    kb[5] = kb[6] = kb[7] = 0xFF
    ka[13] = ka[14] = ka[15] = 0xFF
    kb[2] = sx(~c[13] & 0xFF)
    kb[3] = sx(~c[15] & 0xFF)
    ka[10] = sx(~c[5] & 0xFF)
    ka[11] = sx(~c[7] & 0xFF)
    ka[9] = sx(c[3] ^ kb[3])
    kb[1] = sx(c[11] ^ ka[11])
    kb[0] = sx(c[9] ^ ka[9])
    ka[8] = sx(c[1] ^ kb[1])
    ta = [c[u] ^ kb[u] for u in range(8)]
    tb = [c[u + 8] ^ ka[u + 8] for u in range(8)]
    w = lambda t: t[0] | (t[1] << 8) | (t[2] << 16) | (t[3] << 24)
    return w(ta[:4]), w(ta[4:]), w(tb[:4]), w(tb[4:])


@pytest.mark.parametrize("seed", range(20))
def test_lut16_decode_exhaustive(seed):
    rng = np.random.default_rng(seed)
    cb = rng.integers(-128, 128, size=16).astype(np.int8) if seed else datagen.turboquant_codebook(4, 384)[0]
    l0, l1, l2, l3 = _solve_lut4(cb)
    for x in range(16):
        sel = x * 0x01010101
        r = _perm(l1, l0, sel) ^ _perm(l3, l2, sel ^ 0x08080808)
        assert r == (int(cb[x]) & 0xFF) * 0x01010101


def _pack_model(codes_ref, n, d, bits, ks):
    spl = 8 // bits
    nload = (ks + spl - 1) // spl
    ntiles = (n + 31) // 32
    cpb, dps = 8 // bits, bits // 2
    full = datagen.unpack_codes(codes_ref, bits, d)
    out = np.zeros((ntiles, nload, 64, 4), np.uint32)
    for t in range(ntiles):
        for c in range(nload):
            for lane in range(64):
                m, g = lane & 31, lane >> 5
                v = t * 32 + m
                for wd in range(4):
                    h, fbase = wd // dps, (wd % dps) * cpb
                    s = c * spl + h
                    word = 0
                    if v < n and s < ks:
                        for b in range(4):
                            for e in range(cpb):
                                k = 32 * s + 16 * g + 4 * (fbase + e) + b
                                if k < d:
                                    word |= int(full[v, k]) << (8 * b + e * bits)
                    out[t, c, lane, wd] = word
    return out


def _decode_model(packed, cb, bits, ks, t, lane):
    """Fragment bytes (int8) of every K-step for one lane of one tile."""
    spl = 8 // bits
    frags = {}
    lut = _solve_lut4(cb) if bits == 4 else None
    for s in range(ks):
        c, h = divmod(s, spl)
        raw = [int(x) for x in packed[t, c, lane]]
        dw = []
        if bits == 4:
            w0, w1 = (raw[0], raw[1]) if h == 0 else (raw[2], raw[3])
            for x in (w0 & 0x0F0F0F0F, (w0 >> 4) & 0x0F0F0F0F, w1 & 0x0F0F0F0F, (w1 >> 4) & 0x0F0F0F0F):
                dw.append(_perm(lut[1], lut[0], x) ^ _perm(lut[3], lut[2], x ^ 0x08080808))
        else:
            t0 = sum((int(cb[i]) & 0xFF) << (8 * i) for i in range(4))
            w = raw[h]
            for e in range(4):
                dw.append(_perm(0, t0, (w >> (2 * e)) & 0x03030303))
        fr = []
        for f in range(4):
            for b in range(4):
                byte = (dw[f] >> (8 * b)) & 0xFF
                fr.append(byte - 256 if byte >= 128 else byte)
        frags[s] = fr
    return frags


@pytest.mark.parametrize("bits,d,ks", [(4, 64, 2), (4, 100, 4), (2, 128, 4), (2, 40, 2)])
def test_pack_decode_layout_roundtrip(bits, d, ks):
    n = 45
    rng = np.random.default_rng(bits * 100 + d)
    codes = rng.integers(0, 1 << bits, size=(n, d))
    ref = datagen.pack_codes(codes, bits)
    cb = rng.integers(-127, 128, size=1 << bits).astype(np.int8)
    packed = _pack_model(ref, n, d, bits, ks)
    for t in range(packed.shape[0]):
        for lane in (0, 5, 31, 32, 40, 63):
            m, g = lane & 31, lane >> 5
            v = t * 32 + m
            frags = _decode_model(packed, cb, bits, ks, t, lane)
            for s, fr in frags.items():
                for i in range(16):
                    k = 32 * s + 16 * g + i
                    if v < n and k < d:
                        assert fr[i] == int(cb[codes[v, k]]), (t, lane, s, i)


def test_query_split_hi_lo_exact():
    qs = np.arange(-32639, 32640, dtype=np.int64)
    lo = ((qs + 128) & 255) - 128
    hi = (qs - lo) >> 8
    assert lo.min() >= -128 and lo.max() <= 127 and hi.min() >= -128 and hi.max() <= 127
    np.testing.assert_array_equal(hi * 256 + lo, qs)


def test_qmax_keeps_int32_exact():
    for d in (32, 384, 1024):
        cb, _ = datagen.turboquant_codebook(4, d)
        qmax = oracle.tq_qmax(cb, d)
        assert (qmax + 128) * 127 * d <= 2**31 - 1
        assert qmax <= 127 * 256 + 127


@pytest.mark.parametrize("bits,d,n", [(4, 384, 20000), (2, 128, 20000), (4, 64, 5000)])
def test_topk_scores_relative_to_their_own_magnitude(bits, d, n):
    """The returned top-100 scores against the f64 estimator of the same
    vectors, relative to |score| itself (the north-star's 1e-4 relative
    contract), at the c2 / c5 shapes on a 20k-vector sample."""
    corpus = datagen.TurboQuantCorpus(n, d, bits, 61, 62, 63)
    q = datagen.baseline_queries(64, d, 64)
    ids, sc = oracle.tq_topk(q, corpus.rotation, d, bits, corpus.codebook, corpus.codebook_scale,
                             corpus.codes, corpus.norms, 100)
    ref = oracle.tq_scores_f64(q, corpus.rotation, d, bits, corpus.codebook,
                               corpus.codebook_scale, corpus.codes, corpus.norms)
    want = np.take_along_axis(ref, ids, axis=1)
    rel = np.abs(sc.astype(np.float64) - want) / np.abs(want)
    print(f"max relative error of the top-100 scores: {rel.max():.3e}")
    assert rel.max() <= 1e-4
