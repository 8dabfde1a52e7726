"""Pins the CPU oracle of the two-stage retrieval's second stage (f16 rerank).

* float32ToHalf (runtime/mll_export.go:1007-1041): known answers where it
  departs from round-to-nearest-even (ties round away from zero; finite values
  >= 2^16 keep mantissa bits under the all-ones exponent), agreement with
  numpy's float16 cast everywhere else, and the exact round trip of all 63,488
  finite halves.
* halfToFloat32 (runtime/weight_file.go:461-483): equals numpy's exact
  float16 -> float32 widening for every non-NaN half.
* The rerank score is a sequential f32 sum of f32 products: known answers that
  an f64 accumulator, another summation order or a fused multiply-add fail.
* applyTurboQuantFP16RerankRescue: the reference's three rescue tests
  (runtime/retrieval_eval_test.go:1336-1380, fixture :1434-1445) restated.
* topFP16RerankScores: brute force (Python sort by (score desc, id asc)).
"""
import numpy as np
import pytest

import oracle


def _bits(x):
    return int(np.float32(x).view(np.uint32))


def _f(u):
    return np.uint32(u).view(np.float32)


@pytest.mark.parametrize("value,want", [
    (1.0, 0x3C00),
    (_f(0x3F801000), 0x3C01),        # 1 + 2^-11: tie, away from zero (RNE gives 0x3C00)
    (_f(0xBF801000), 0xBC01),        # negative tie
    (_f(0x3F803000), 0x3C02),        # 1 + 3*2^-11: tie to 0x3C02 either way
    (65504.0, 0x7BFF),
    (65519.0, 0x7BFF),
    (65520.0, 0x7C00),               # tie at the top rounds up to infinity
    (70000.0, 0x7C45),               # finite >= 2^16 keeps mantissa bits: NaN pattern
    (float("inf"), 0x7C00),
    (2.0 ** -24, 0x0001),
    (2.0 ** -25, 0x0001),            # subnormal tie rounds up (RNE gives 0)
    (2.0 ** -26, 0x0000),
    (-0.0, 0x8000),
])
def test_f32_to_half_known_answers(value, want):
    assert int(oracle.f32_to_half(np.array([value], np.float32))[0]) == want


def test_f32_to_half_matches_rne_off_ties():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-12, 10, 200000))).astype(np.float32)
    u = x.view(np.uint32)
    ex = ((u >> 23) & 0xFF).astype(np.int64) - 127
    normal = (ex >= -14) & (ex <= 15)
    tie = (u & 0x1FFF) == 0x1000
    sel = normal & ~tie
    got = oracle.f32_to_half(x[sel])
    want = x[sel].astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_half_round_trip_and_widening_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (h & 0x7C00) != 0x7C00
    wide = oracle.half_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    notnan = ~np.isnan(ref)
    assert np.array_equal(wide[notnan].view(np.uint32), ref[notnan].view(np.uint32))
    assert np.array_equal(oracle.f32_to_half(ref[finite]), h[finite])


def _one(q, row_halves, k=1):
    rows = np.array([row_halves], np.uint16)
    ids, scores = oracle.fp16_rerank(np.array([q], np.float32), rows, np.array([[0]], np.int64),
                                     np.array([[0.0]], np.float32), k)
    return scores[0, 0]


def test_score_is_sequential_f32():
    # 1 + 2^-24 + 2^-24 + 2^-24 in order stays 1 in f32; f64 or a reversed
    # order gives a larger value.
    s = _one([1, 1, 1, 1], [0x3C00, 0x0001, 0x0001, 0x0001])
    assert _bits(s) == _bits(1.0)


def test_score_has_no_fused_multiply_add():
    # -1 + fl(fl(1/3) * 3) = -1 + 1 = 0; with a fused multiply-add it is 2^-25-ish.
    third = np.float32(1.0) / np.float32(3.0)
    s = _one([1.0, third], [0xBC00, 0x4200])
    assert _bits(s) == 0


def _rescue_fixture(n):
    ids = np.arange(1, n + 1, dtype=np.int64)
    scores = (n - np.arange(n)).astype(np.float32)
    return ids, scores, np.arange(1, n + 1), scores.copy()


def test_rescue_leaves_incomplete_window_unchanged():
    ids, s, ranks, comp = _rescue_fixture(119)
    assert np.array_equal(oracle.apply_rescue(ids, s, ranks, comp), ids)


def test_rescue_promotes_strong_compact_boundary_candidate():
    ids, s, ranks, comp = _rescue_fixture(121)
    comp[119], ranks[119] = 10000, 1          # d120
    got = oracle.apply_rescue(ids, s, ranks, comp)
    assert 120 in got[:100] and 100 not in got[:100]
    assert got[99] == 120


def test_rescue_compact_tie_break():
    ids, s, ranks, comp = _rescue_fixture(121)
    comp[109] = comp[110] = 10000             # d110, d111
    ranks[109] = ranks[110] = 7
    assert oracle.apply_rescue(ids, s, ranks, comp)[99] == 111


def test_rerank_brute_force_no_rescue():
    rng = np.random.default_rng(11)
    n, d, c = 300, 24, 150
    rows = oracle.f32_to_half(rng.standard_normal((n, d)).astype(np.float32) * 0.2)
    rows[7] = rows[8]                           # a score tie: id order decides
    q = rng.standard_normal((2, d)).astype(np.float32)
    cid = np.stack([rng.permutation(n)[:c] for _ in range(2)]).astype(np.int64)
    cid[0, :2] = [8, 7]
    cid[1, 5] = n + 3                           # no row: skipped
    ids, scores = oracle.fp16_rerank(q, rows, cid, np.zeros_like(cid, np.float32), 40)
    for i in range(2):
        sc = []
        for j in cid[i]:
            if j >= n:
                continue
            acc = np.float32(0)
            for t in range(d):
                acc = np.float32(acc + np.float32(q[i, t] * np.float32(rows[j, t].view(np.float16))))
            sc.append((-float(acc), int(j), acc))
        sc.sort()
        assert [j for _, j, _ in sc[:40]] == ids[i].tolist()
        assert np.array_equal(np.array([a for _, _, a in sc[:40]], np.float32), scores[i])


def test_dense_rerank_oracle_pins():
    """topDenseRerankScores: the sequential f32 sum (a known answer an f64 or
    pairwise accumulator fails), brute force order (score desc, id asc),
    skipped ids outside [0, n), and the string-ID order through id_rank."""
    big = np.float32(2.0 ** 24)
    rows = np.array([[big, 1.0, 1.0, -big], [1.0, 1.0, big, -big]], np.float32)
    q = np.ones((1, 4), np.float32)
    _, sc = oracle.dense_rerank(q, rows, np.array([[0, 1]]), 0)
    # row 0: 2^24 + 1 -> 2^24 (rounded), + 1 -> 2^24, - 2^24 = 0; row 1: 2 + 2^24 - 2^24 = 2
    assert sc[0].tolist() == [2.0, 0.0]
    rng = np.random.default_rng(3)
    rows = rng.normal(size=(300, 24)).astype(np.float32)
    rows[7] = rows[9]
    q = rng.normal(size=(4, 24)).astype(np.float32)
    cid = np.stack([rng.permutation(300)[:80] for _ in range(4)]).astype(np.int64)
    cid[:, :2] = [9, 7]
    cid[0, 5] = 400
    ids, sc = oracle.dense_rerank(q, rows, cid, 30)
    for i in range(4):
        live = [j for j in cid[i] if 0 <= j < 300]
        s = {j: np.float32(0) for j in live}
        for j in live:
            acc = np.float32(0)
            for t in range(24):
                acc = np.float32(acc + np.float32(q[i, t] * rows[j, t]))
            s[j] = acc
        want = sorted(live, key=lambda j: (-s[j], j))[:30]
        assert ids[i].tolist() == want
        assert sc[i].tolist() == [s[j] for j in want]
    rank = np.arange(300)[::-1].copy()
    ids_r, _ = oracle.dense_rerank(q[:1], np.ones((300, 24), np.float32), cid[:1], 3, id_rank=rank)
    live = [j for j in cid[0] if 0 <= j < 300]
    assert ids_r[0].tolist() == sorted(live, key=lambda j: rank[j])[:3]


def test_reconstruct_rerank_oracle_pins():
    """The reconstruct contract (dequantize to the original frame, then the
    reference's f32 index-order dot): the dequantized vector equals an
    independent numpy f64 construction norm * R^T codebook[code] to f32
    rounding; the scores equal the f32 dots of those vectors bit for bit;
    they track the f64 estimator tq_scores_f64 to f32 accumulation error;
    the identity rotation and a one-hot query reduce to norm * codebook
    value; and a slip in the row layout or the frame (R instead of R^T) is
    caught."""
    rng = np.random.default_rng(5)
    d, bits, n = 64, 4, 200
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32)
    codes = rng.integers(0, 256, size=(n, d * bits // 8)).astype(np.uint8)
    norms = np.exp(0.2 * rng.normal(size=n)).astype(np.float32)
    cbi = np.array([-127, -90, -64, -45, -30, -18, -8, -2, 2, 8, 18, 30, 45, 64, 90, 127], np.int8)
    s_c = np.float32(0.004)
    cb = (cbi.astype(np.float32) * s_c).astype(np.float32)
    q = rng.normal(size=(3, d)).astype(np.float32)
    cid = np.tile(np.arange(n, dtype=np.int64), (3, 1))
    ids, sc = oracle.reconstruct_rerank(q, rot, codes, bits, norms, cb, cid, 0)
    full = np.zeros((3, n), np.float32)
    for i in range(3):
        full[i, ids[i]] = sc[i]
    lo, hi = codes & 0xF, codes >> 4
    code = np.stack([lo, hi], axis=2).reshape(n, d)
    xhat64 = (norms[:, None].astype(np.float64) *
              (cb.astype(np.float64)[code] @ rot.astype(np.float64)))
    xhat = np.stack([oracle.tq_dequantize(rot, codes[v], bits, norms[v], cb) for v in range(n)])
    np.testing.assert_allclose(xhat, xhat64, rtol=1e-6, atol=1e-7)
    assert np.max(np.abs(xhat - xhat64.astype(np.float32))) <= 1.2e-7 * np.abs(xhat64).max()
    # scores: dotRetrievalVectors over the dequantized f32 vectors
    for i in range(3):
        want = np.zeros(n, np.float32)
        for k in range(d):
            want = (want + (q[i, k] * xhat[:, k]).astype(np.float32)).astype(np.float32)
        np.testing.assert_array_equal(full[i], want)
    est = oracle.tq_scores_f64(q, rot, d, bits, cbi, s_c, codes, norms)
    np.testing.assert_allclose(full, est, rtol=1e-5, atol=2e-6)
    # R^T, not R: the same codes under R dequantize elsewhere
    wrong = norms[:, None].astype(np.float64) * (cb.astype(np.float64)[code] @ rot.T.astype(np.float64))
    assert np.max(np.abs(xhat - wrong)) > 1e-2
    one = np.zeros((1, d), np.float32)
    one[0, 5] = 1.0
    ids1, sc1 = oracle.reconstruct_rerank(one, None, codes, bits, norms, cb, cid[:1], 0)
    want = norms[ids1[0]] * cb[code[ids1[0], 5]]
    np.testing.assert_array_equal(sc1[0], want.astype(np.float32))


def test_reconstruct_three_bit_rows_straddle_bytes():
    """3-bit codes (the (b - 1)-bit MSE part of an inner-product set at b =
    4) packed low bits first across byte boundaries: code j sits at bits
    3j .. 3j + 2 of the row."""
    d, bits = 16, 3
    want_codes = np.arange(16) % 8
    bitsv = np.zeros(d * bits, np.uint8)
    for j, v in enumerate(want_codes):
        for b in range(bits):
            bitsv[j * bits + b] = (v >> b) & 1
    row = np.packbits(bitsv, bitorder="little")
    assert row.size == 6
    cb = np.arange(8, dtype=np.float32) - 3.5
    x = oracle.tq_dequantize(None, row, bits, 2.0, cb)
    np.testing.assert_array_equal(x, 2.0 * cb[want_codes])


def test_reconstruct_inner_product_set_adds_the_qjl_term():
    """Inner-product code sets (MSE codes + QJL signs + ResNorm + Norm): the
    dequantized vector is norm * R^T (c[code] + sqrt(pi/2)/d * ResNorm *
    S^T sign) (TurboQuant_prod's dequantizer), built independently in numpy
    f64 here; its inner product with a query equals the inner-product
    estimator tq_ip_scores (the same estimator through int16 query grids, to
    their rounding); and over many sketches it is unbiased for <q, x> where
    the MSE part alone is biased."""
    rng = np.random.default_rng(8)
    d, bits = 64, 3
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32)
    pts = np.sort(rng.normal(size=1 << bits))
    cbi = np.clip(np.rint(pts / np.abs(pts).max() * 127), -127, 127).astype(np.int8)
    s_c = float(np.float32(2.2 / np.sqrt(d) / 127))
    cb = (cbi.astype(np.float32) * np.float32(s_c)).astype(np.float32)
    x = rng.normal(size=(40, d)).astype(np.float32)
    q = rng.normal(size=(2, d)).astype(np.float32)
    S = rng.normal(size=(d, d)).astype(np.float32)
    codes, signs, rn, nm = oracle.tq_encode_ip(x, rot, S, d, bits, cbi, s_c)
    bitsv = np.unpackbits(codes, axis=1, bitorder="little")[:, :d * bits].reshape(40, d, bits)
    code = (bitsv * (1 << np.arange(bits))).sum(2)
    sg = np.unpackbits(signs, axis=1, bitorder="little")[:, :d].astype(np.float64) * 2 - 1
    y = cb.astype(np.float64)[code] + (np.sqrt(np.pi / 2) / d) * rn[:, None].astype(np.float64) * (
        sg @ S.astype(np.float64))
    xhat64 = nm[:, None].astype(np.float64) * (y @ rot.astype(np.float64))
    xhat = np.stack([oracle.tq_dequantize(rot, codes[v], bits, nm[v], cb, signs[v], rn[v], S)
                     for v in range(40)])
    np.testing.assert_allclose(xhat, xhat64, rtol=2e-6, atol=1e-6)
    cid = np.tile(np.arange(40, dtype=np.int64), (2, 1))
    ids, sc = oracle.reconstruct_rerank(q, rot, codes, bits, nm, cb, cid, 0, signs=signs,
                                        resnorms=rn, sketch=S)
    full = np.zeros((2, 40), np.float32)
    for i in range(2):
        full[i, ids[i]] = sc[i]
    ip = oracle.tq_ip_scores(q, rot, S, d, bits, cbi, s_c, codes, signs, rn, nm)
    scale = np.linalg.norm(q, axis=1)[:, None] * nm[None, :]
    assert np.max(np.abs(full - ip) / scale) < 2e-4
    # unbiasedness over sketches (one vector, one query)
    xv, qv = x[0], q[0]
    true = float(np.dot(qv.astype(np.float64), xv.astype(np.float64)))
    ests, mses = [], []
    for t in range(300):
        St = np.random.default_rng(100 + t).normal(size=(d, d)).astype(np.float32)
        c1, s1, r1, n1 = oracle.tq_encode_ip(xv[None], rot, St, d, bits, cbi, s_c)
        xi = oracle.tq_dequantize(rot, c1[0], bits, n1[0], cb, s1[0], r1[0], St)
        xm = oracle.tq_dequantize(rot, c1[0], bits, n1[0], cb)
        ests.append(float(np.dot(qv, xi)))
        mses.append(float(np.dot(qv, xm)))
    ests = np.array(ests)
    assert abs(ests.mean() - true) < 4 * ests.std() / np.sqrt(len(ests))
    assert np.std(mses) < 1e-9                       # the MSE part does not move
