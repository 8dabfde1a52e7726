"""GPU parity of the retrieval plans (score step, topk, gathers,
pack_candidates) against the plan run step by step on the CPU
(oracle/plan_oracle.py over the C restatements of dotRows / cosineRows /
l2DistanceRows and topKTensor). Bar: bit-exact scores, indices, ids and
document rows (score and selection arithmetic is the reference's own)."""
import zlib

import numpy as np
import pytest

from eos_amd._lib import EosHipError
from eos_amd.mll import MllPackage
from eos_amd.retrieval import MllRetrieval, score_topk
from oracle import plan_oracle
from tests import mll_synth

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _q4_values(codes, scale):
    return codes.astype(np.float32) * np.float32(scale)


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("form", ["score", "select", "rerank", "retrieve"])
def test_param_document_plans(rt, op, form):
    """examples/score.eos, select.eos, rerank.eos, retrieve.eos: documents are
    a packed q4 param of the package (odd width: rows straddle bytes), with
    planted duplicate rows (ties broken by index) and an all-zero row
    (cosine 0)."""
    _case(f"param documents {form} {op}")
    rng = np.random.default_rng(zlib.crc32(f"{form}/{op}".encode()))
    n, d = 3000, 37
    codes = rng.integers(-8, 8, (n, d)).astype(np.int8)
    codes[17] = codes[2900]
    codes[5] = codes[2900]
    codes[100] = 0
    scale = 0.0625
    art = mll_synth.retrieval_artifact(form, op, k=7)
    pkg = MllPackage(mll_synth.retrieval_package(art, codes, scale))
    ret = MllRetrieval(rt, pkg)
    docs = _q4_values(codes, scale)
    for trial in range(3):
        query = rng.normal(size=d).astype(np.float32)
        if trial == 1:
            query = docs[2900] + np.float32(0.0)      # ties at the top
        got = ret.run(query)
        want = plan_oracle.run(art, {"docs": docs}, form, {"query": query})
        rets = art["steps"][-1]["outputs"]
        assert len(got) == len(rets)
        for g, name in zip(got, rets):
            np.testing.assert_array_equal(g, want[name], err_msg=f"{form} {op} {name}")
    ret.release()


@pytest.mark.parametrize("form", ["candidates", "packed", "batch"])
def test_candidate_table_plans(rt, form):
    """examples/candidates.eos, packed_candidates.eos, batch_candidates.eos:
    query, candidate documents and ids are inputs (RunCandidateTable)."""
    _case(f"candidate table {form}")
    rng = np.random.default_rng(7)
    art = mll_synth.retrieval_artifact(form, "cosine", k=2)
    ret = MllRetrieval(rt, MllPackage(mll_synth.retrieval_package(art)))
    d = 64
    if form == "batch":
        q, n = 5, 300
        query = rng.normal(size=(q, d)).astype(np.float32)
        docs = rng.normal(size=(q, n, d)).astype(np.float32)
        ids = rng.integers(0, 2**40, size=(q, n)).astype(np.int64)
        docs[2, 7] = docs[2, 250]
    else:
        n = 500
        query = rng.normal(size=d).astype(np.float32)
        docs = rng.normal(size=(n, d)).astype(np.float32)
        ids = rng.permutation(10**6)[:n].astype(np.int64)
    got = ret.run(query, docs, ids)
    want = plan_oracle.run(art, {}, form, {"query": query, "docs": docs, "candidate_ids": ids})
    rets = art["steps"][-1]["outputs"]
    for g, name in zip(got, rets):
        w = want[name]
        if isinstance(w, tuple):
            for gg, ww in zip(g, w):
                np.testing.assert_array_equal(gg, ww)
        else:
            np.testing.assert_array_equal(g, w, err_msg=name)
    ret.release()


def test_score_topk_large_and_errors(rt):
    """Direct entry at 200k rows x 384 (f32 documents, 4 queries, k 100) and
    the errors the reference raises (k above the row count)."""
    _case("score_topk 200k x 384")
    rng = np.random.default_rng(11)
    n, d, q = 200_000, 384, 4
    docs = rng.normal(size=(n, d)).astype(np.float32)
    queries = rng.normal(size=(q, d)).astype(np.float32)
    docs[123_456] = docs[7]
    queries[1] = docs[7]
    res = score_topk(rt, "cosine", queries, docs, k=100)
    for i in range(q):
        want = plan_oracle.oracle.score_rows("cosine", queries[i], docs)
        np.testing.assert_array_equal(res["scores"][i], want)
        idx, sc = plan_oracle.oracle.topk_scores(want, 100)
        np.testing.assert_array_equal(res["top_index"][i], idx)
        np.testing.assert_array_equal(res["top_scores"][i], sc)
        np.testing.assert_array_equal(res["top_docs"][i], docs[idx])
    assert res["top_index"][1][:2].tolist() == [7, 123_456]
    with pytest.raises(EosHipError, match="topk limit"):
        score_topk(rt, "dot", queries[:1], docs[:10], k=11)


@pytest.mark.parametrize("op,want", [("dot", [1, 0, 1]), ("cosine", [1, 0, 0.70710677]),
                                     ("l2_distance", [0, 1.4142135, 1])])
def test_reference_score_known_answers(rt, op, want):
    """The reference's score-op known answers (runtime/runtime_test.go:
    1702-1716): query [1, 0] against docs [[1,0],[0,1],[1,1]]."""
    _case(f"score known answers {op}")
    q = np.asarray([[1, 0]], np.float32)
    docs = np.asarray([[1, 0], [0, 1], [1, 1]], np.float32)
    res = score_topk(rt, op, q, docs, k=3)
    np.testing.assert_array_equal(res["scores"][0], np.asarray(want, np.float32))


def test_signed_zero_ties_rank_by_index(rt):
    """A cosine that underflows to -0 (dot -1e-30 against a norm of 1e20)
    ties with a +0 cosine, as Go's -0 == +0 comparison makes it: the lower
    index ranks first, whichever zero it holds."""
    _case("signed zero ties")
    q = np.asarray([[1, 0]], np.float32)
    docs = np.asarray([[-1, 0], [-1e-30, 1e20], [0, 1], [0.5, 0.5], [0, 3]], np.float32)
    want = plan_oracle.oracle.score_rows("cosine", q[0], docs)
    assert np.signbit(want[1]) and want[1] == 0 and not np.signbit(want[2])
    res = score_topk(rt, "cosine", q, docs, k=3)
    np.testing.assert_array_equal(res["scores"][0], want)
    assert res["top_index"][0].tolist() == [3, 1, 2]
    idx, _ = plan_oracle.oracle.topk_scores(want, 3)
    assert idx.tolist() == [3, 1, 2]
