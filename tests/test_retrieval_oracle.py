"""Pins the CPU restatement of the retrieval score ops (oracle.score_rows:
dotRows / cosineRows / l2DistanceRows, runtime/backend/tensor_ops.go:
1967-2089) to the reference's own known answers and to closed forms chosen so
that a plausible slip fails one of them:
  - the reference values for query [1, 0] against docs [[1,0],[0,1],[1,1]]
    (runtime/runtime_test.go:1702-1716);
  - dot: an f32 sum in index order with the product rounded before the add
    (a fused multiply-add or another summation order gives another value);
  - cosine: f64 accumulation (an f32 dot loses the cancelling terms), the
    zero-denominator rule, and agreement with an f64 numpy form;
  - l2: the difference taken in f32 before the f64 square."""
import math

import numpy as np

import oracle

F32 = np.float32


def _rows(op, q, docs):
    return oracle.score_rows(op, np.asarray(q, F32), np.asarray(docs, F32))


def test_reference_known_answers():
    q = [1, 0]
    docs = [[1, 0], [0, 1], [1, 1]]
    want = {
        "dot": [1, 0, 1],
        "cosine": [1, 0, 0.70710677],
        "l2_distance": [0, 1.4142135, 1],
    }
    for op, w in want.items():
        got = _rows(op, q, docs)
        np.testing.assert_array_equal(got, np.asarray(w, F32), err_msg=op)


def test_dot_rounds_each_product_and_sums_in_index_order():
    # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24: the f32 product drops 2^-24 (a tie to
    # even), so the unfused sum is exactly 2^-11; a fused multiply-add would
    # keep 2^-11 + 2^-24.
    a = 1 + 2.0 ** -12
    got = _rows("dot", [a, -1], [[a, 1]])[0]
    assert got == F32(2.0 ** -11)
    assert got != F32(2.0 ** -11 + 2.0 ** -24)
    # Index order: (1 + 1e8) rounds to 1e8 in f32, then - 1e8 gives 0; a
    # pairwise or magnitude-sorted sum keeps the 1.
    assert _rows("dot", [1, 1e8, -1e8], [[1, 1, 1]])[0] == F32(0)
    assert _rows("dot", [1e8, -1e8, 1], [[1, 1, 1]])[0] == F32(1)


def test_cosine_accumulates_in_f64():
    # dot = 1e8 - 1e8 + 1 = 1 exactly in f64 (0 in f32 index order).
    q = [1e8, -1e8, 1]
    x = [1, 1, 1]
    want = F32(1.0 / (math.sqrt(2e16 + 1) * math.sqrt(3.0)))
    got = _rows("cosine", q, [x])[0]
    assert got == want and got > 0
    # Zero denominator (a zero document row, or a zero query) scores 0.
    np.testing.assert_array_equal(_rows("cosine", [1, 2], [[0, 0], [3, 4]]),
                                  np.asarray([0, F32(11 / (math.sqrt(5) * 5))], F32))
    np.testing.assert_array_equal(_rows("cosine", [0, 0], [[3, 4]]), np.zeros(1, F32))


def test_cosine_matches_an_f64_numpy_form():
    rng = np.random.default_rng(5)
    q = rng.normal(size=96).astype(F32)
    docs = rng.normal(size=(2000, 96)).astype(F32) * rng.lognormal(0, 3, (2000, 1)).astype(F32)
    got = _rows("cosine", q, docs)
    qd, xd = q.astype(np.float64), docs.astype(np.float64)
    ref = (xd @ qd) / (np.sqrt(qd @ qd) * np.sqrt(np.sum(xd * xd, axis=1)))
    want = ref.astype(F32)
    # Sum order differs from numpy's in the last f64 bits only: after the f32
    # rounding nearly every score is identical, none is more than 1 ulp off.
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert np.mean(ulp == 0) > 0.99


def test_l2_takes_the_difference_in_f32():
    # A case where the f32 difference decides the last bit: with it the
    # distance is 0.32919002, with an f64 difference 0.32919 (the inputs are
    # exact f32 values, found by a search over random triples).
    q = [-4.9591071729082614e-05, 0.3289696276187897, -2.5857254513539374e-05]
    x = [6.333526107482612e-05, -0.00022035099391359836, 5.202897227718495e-06]
    qf, xf = np.asarray(q, F32), np.asarray(x, F32)
    diff32 = (qf - xf).astype(np.float64)
    diff64 = qf.astype(np.float64) - xf.astype(np.float64)
    assert F32(math.sqrt(sum(v * v for v in diff32))) != F32(math.sqrt(sum(v * v for v in diff64)))
    assert _rows("l2_distance", q, [x])[0] == F32(math.sqrt(sum(v * v for v in diff32)))
    assert _rows("l2_distance", q, [x])[0] == F32(0.32919002)
    rng = np.random.default_rng(9)
    q = rng.normal(size=40).astype(F32)
    docs = rng.normal(size=(500, 40)).astype(F32)
    diff = (q[None, :] - docs).astype(np.float64)
    want = np.sqrt(np.sum(diff * diff, axis=1)).astype(F32)
    got = _rows("l2_distance", q, docs)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1 and np.mean(ulp == 0) > 0.99


def test_topk_ties_and_signed_zero():
    # topKTensor: value descending, index ascending; -0 == +0 ties by index.
    s = np.asarray([-0.0, 0.0, -1.0, 0.5, 0.5], F32)
    idx, sc = oracle.topk_scores(s, 4)
    assert idx.tolist() == [3, 4, 0, 1]
