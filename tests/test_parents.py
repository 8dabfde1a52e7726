"""Parent (multivector child) aggregation: topTurboQuantMultiVectorParentScores
(runtime/retrieval_multivector_turboquant.go:746-908) over ragged parents.

CPU: the oracle (oracle/tq_oracle.c tq_parent_topk) reproduces the
reference's own ordering case (retrieval_eval_test.go:2913-2950: "max" ranks
the spiky parent first, "top2-mean" the steady one, whose best child is the
lower id of a tie), agrees with a sort-based brute force over the pinned
per-vector scores for every aggregation and penalty, and reduces to the
pinned MaxSim child-max with "max" and no penalty. GPU: parent ids, scores,
best child ids and best child scores are bit-exact against the oracle."""
import math

import numpy as np
import pytest

import oracle
from eos_amd import datagen

AGGS = {"max": 1, "top2-mean": 2, "top3-mean": 3, "top5-mean": 5}


def _corpus(n, d, bits, seed):
    return datagen.TurboQuantCorpus(n, d, bits, seed, seed + 1, seed + 2)


def _ragged_offsets(n, nparents, seed):
    """Sorted cut points with empty parents, single-child parents and long ones."""
    cuts = np.sort(datagen.uniform_int(seed, nparents - 1, 0, n + 1)).astype(np.int64)
    off = np.concatenate([[0], cuts, [n]]).astype(np.int64)
    off[3] = off[2]  # an empty parent
    return off


def _brute(scores, off, top_n, penalty, k):
    """Per parent: mean of the top_n best child scores (f64, descending),
    minus penalty * log1p(count); rank by (score desc, id asc)."""
    rows = []
    for q in range(scores.shape[0]):
        entries = []
        for p in range(len(off) - 1):
            ch = scores[q, off[p]:off[p + 1]]
            if ch.size == 0:
                continue
            top = np.sort(ch)[::-1][:min(top_n, 5, ch.size)]
            s = 0.0
            for v in top:
                s += float(v)
            s /= len(top)
            if penalty != 0:
                s -= penalty * math.log1p(ch.size)
            best = int(np.argmax(ch))  # first maximum: the lowest child index
            entries.append((np.float32(s), p, off[p] + best, ch[best]))
        entries.sort(key=lambda e: (-float(e[0]), e[1]))
        kk = len(entries) if (k <= 0 or k > len(entries)) else k
        rows.append(entries[:kk])
    ids = np.array([[e[1] for e in r] for r in rows], np.int64)
    sc = np.array([[e[0] for e in r] for r in rows], np.float32)
    bc = np.array([[e[2] for e in r] for r in rows], np.int64)
    bs = np.array([[e[3] for e in r] for r in rows], np.float32)
    return ids, sc, bc, bs


def test_reference_top2_mean_reorders_parents():
    """retrieval_eval_test.go:2913-2950 on TurboQuant codes: with the identity
    rotation and the query e0, a child's score is norm * x * sign, where the
    sign comes from the extreme centroid its coordinate 0 takes."""
    d, bits = 8, 2
    cb, s = datagen.turboquant_codebook(bits, d)
    hi, lo = int(np.argmax(cb)), int(np.argmin(cb))
    assert cb[hi] == -cb[lo]
    codes = np.zeros((4, d), np.uint8)
    codes[:, 0] = [hi, hi, hi, lo]     # steady-a, steady-b, spiky-a, spiky-b
    packed = datagen.pack_codes(codes, bits)
    norms = np.array([0.9, 0.9, 1.0, 1.0], np.float32)
    off = np.array([0, 2, 4], np.int64)  # steady = parent 0, spiky = parent 1
    q = np.zeros((1, d), np.float32)
    q[0, 0] = 1.0
    ids, sc, bc, _ = oracle.tq_parent_topk(q, None, d, bits, cb, s, packed, norms, off, 2, 1)
    np.testing.assert_array_equal(ids[0], [1, 0])            # max: spiky first
    ids, sc, bc, bs = oracle.tq_parent_topk(q, None, d, bits, cb, s, packed, norms, off, 2, 2)
    np.testing.assert_array_equal(ids[0], [0, 1])            # top2-mean: steady first
    assert bc[0, 0] == 0                                     # tie: steady-a, the lower id
    assert sc[0, 1] == 0.0                                   # (x + -x) / 2
    assert sc[0, 0] == bs[0, 0]                              # mean of two equal scores


@pytest.mark.parametrize("agg", list(AGGS))
@pytest.mark.parametrize("penalty", [0.0, 0.05])
def test_oracle_matches_sort_brute_force(agg, penalty):
    c = _corpus(3000, 64, 2, seed=41)
    off = _ragged_offsets(3000, 150, 43)
    q = datagen.baseline_queries(3, 64, 44)
    _, flat = oracle.tq_scores(q, c.rotation, 64, 2, c.codebook, c.codebook_scale, c.codes, c.norms)
    for k in (1, 10, 0):
        got = oracle.tq_parent_topk(q, c.rotation, 64, 2, c.codebook, c.codebook_scale, c.codes,
                                    c.norms, off, k, AGGS[agg], penalty)
        want = _brute(flat, off, AGGS[agg], penalty, k)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)


def test_max_without_penalty_is_maxsim_child_max():
    c = _corpus(40 * 64, 64, 4, seed=45)
    q = datagen.baseline_queries(2, 64, 46)
    off = np.arange(0, 40 * 64 + 1, 64, dtype=np.int64)
    ids, sc, _, _ = oracle.tq_parent_topk(q, c.rotation, 64, 4, c.codebook, c.codebook_scale,
                                          c.codes, c.norms, off, 40, 1)
    ms = oracle.tq_maxsim_scores(q, c.rotation, 64, 4, c.codebook, c.codebook_scale, c.codes,
                                 c.norms, 64)
    for r in range(2):
        order = np.lexsort((np.arange(40), -ms[r]))
        np.testing.assert_array_equal(ids[r], order)
        np.testing.assert_array_equal(sc[r], ms[r][order])


def test_penalty_closed_form_and_empty_parents():
    """Two parents with the same best child: the one with more children loses
    penalty * (log1p(3) - log1p(1)); empty parents never rank."""
    d, bits = 8, 2
    cb, s = datagen.turboquant_codebook(bits, d)
    hi, lo = int(np.argmax(cb)), int(np.argmin(cb))
    codes = np.zeros((4, d), np.uint8)
    codes[:, 0] = [hi, hi, lo, lo]
    packed = datagen.pack_codes(codes, bits)
    norms = np.ones(4, np.float32)
    off = np.array([0, 0, 1, 1, 4, 4], np.int64)  # parents 0, 2, 4 empty
    q = np.zeros((1, d), np.float32)
    q[0, 0] = 1.0
    ids, sc, bc, bs = oracle.tq_parent_topk(q, None, d, bits, cb, s, packed, norms, off, 0, 1, 0.1)
    np.testing.assert_array_equal(ids[0], [1, 3])
    x = float(bs[0, 0])
    assert sc[0, 0] == np.float32(x - 0.1 * math.log1p(1))
    assert sc[0, 1] == np.float32(x - 0.1 * math.log1p(3))
    np.testing.assert_array_equal(bc[0], [0, 1])


# ----------------------------------------------------------------------- GPU

def _dev(rt, c):
    from eos_amd.turboquant import TurboQuantIndex
    return TurboQuantIndex(rt, c.codes, c.norms, c.dim, c.bits, c.codebook, c.codebook_scale,
                           c.rotation)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,d,n,np_", [(2, 128, 20000, 700), (4, 384, 9000, 2000),
                                          (4, 64, 5000, 5000)])
def test_parent_topk_matches_oracle(rt, bits, d, n, np_):
    from eos_amd.turboquant import TurboQuantParents
    print(f"[case] parents bits={bits} d={d} n={n} parents={np_}", flush=True)
    c = _corpus(n, d, bits, seed=d + n % 89)
    off = _ragged_offsets(n, np_, n % 53)
    q = datagen.baseline_queries(70, d, 47)
    idx = _dev(rt, c)
    par = TurboQuantParents(idx, off)
    for agg in AGGS:
        for penalty in (0.0, 0.05):
            for k in (1, 100, 0):
                got = par.top_k(q, k, agg, penalty)
                want = oracle.tq_parent_topk(q, c.rotation, d, bits, c.codebook, c.codebook_scale,
                                             c.codes, c.norms, off, k, AGGS[agg], penalty)
                for g, w in zip(got, want):
                    np.testing.assert_array_equal(g, w)
    par.release()
    idx.release()


@pytest.mark.gpu
def test_parent_topk_reference_case_and_validation(rt):
    from eos_amd._lib import EosHipError
    from eos_amd.turboquant import (TurboQuantIndex, TurboQuantParents,
                                    top_turboquant_multivector_parent_scores)
    print("[case] parents reference case + validation", flush=True)
    d, bits = 32, 2
    cb, s = datagen.turboquant_codebook(bits, d)
    hi, lo = int(np.argmax(cb)), int(np.argmin(cb))
    codes = np.zeros((4, d), np.uint8)
    codes[:, 0] = [hi, hi, hi, lo]
    idx = TurboQuantIndex(rt, datagen.pack_codes(codes, bits),
                          np.array([0.9, 0.9, 1.0, 1.0], np.float32), d, bits, cb, s, None)
    par = TurboQuantParents(idx, np.array([0, 2, 4], np.int64))
    q = np.zeros(d, np.float32)
    q[0] = 1.0
    mx = top_turboquant_multivector_parent_scores(par, q, 2)
    t2 = top_turboquant_multivector_parent_scores(par, q, 2, "top2-mean")
    assert [r.id for r in mx] == [1, 0] and [r.id for r in t2] == [0, 1]
    assert t2[0].child_id == 0 and t2[1].score == 0.0
    with pytest.raises(EosHipError, match="non-negative"):
        par.top_k(q[None], 2, "max", -0.1)
    with pytest.raises(ValueError, match="aggregation"):
        par.top_k(q[None], 2, "top4-mean")
    with pytest.raises(EosHipError, match="offsets"):
        TurboQuantParents(idx, np.array([0, 3, 2, 4], np.int64))
    with pytest.raises(EosHipError, match="corpus size"):
        TurboQuantParents(idx, np.array([0, 2], np.int64))
    par.release()
    idx.release()


@pytest.mark.gpu
def test_parent_topk_c5_shape(rt):
    """Benchmark config c5 corpus (100k parents x 128 children, d = 128, 2-bit)
    with one query vector per query: "max" equals the MaxSim child max of the
    same corpus on one token, and the top5-mean rows equal the oracle's for
    two queries."""
    from eos_amd.turboquant import TurboQuantMultiVectorIndex, TurboQuantParents
    print("[case] parents c5 shape", flush=True)
    c = datagen.TurboQuantCorpus(100_000 * 128, 128, 2, 11, 12, 13)
    q = datagen.baseline_queries(8, 128, 14)
    idx = _dev(rt, c)
    par = TurboQuantParents(idx, np.arange(0, 100_000 * 128 + 1, 128, dtype=np.int64))
    ids, sc, _, _ = par.top_k(q, 100, "max")
    mids, msc = TurboQuantMultiVectorIndex(idx, 128).top_k(q, 100)
    np.testing.assert_array_equal(ids, mids)
    np.testing.assert_array_equal(sc, msc)
    got = par.top_k(q[:2], 100, "top5-mean", 0.01)
    off = np.arange(0, 100_000 * 128 + 1, 128, dtype=np.int64)
    want = oracle.tq_parent_topk(q[:2], c.rotation, 128, 2, c.codebook, c.codebook_scale, c.codes,
                                 c.norms, off, 100, 5, 0.01)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    par.release()
    idx.release()
