"""MaxSim (multivector late interaction) on the TurboQuant scan.

CPU: the oracle's MaxSim is pinned to the flat scorer -- with one query token
it equals the reference child-max (per document, the best child score,
runtime/retrieval_multivector_turboquant.go:746-783), and the token sum is
the stated pairwise tree. GPU: document scores and top-k ids are bit-exact
against the oracle; at benchmark config c5 size (100k docs x 128 vectors,
d = 128, 2-bit, 32 queries x 32 tokens) the device top-k must equal the sort
of the device's exhaustive document scores, and those equal the oracle's on a
sampled subset of documents."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen


def _corpus(ndocs, doc_len, d, bits, seed=31):
    return datagen.TurboQuantCorpus(ndocs * doc_len, d, bits, seed, seed + 1, seed + 2)


def _tokens(q, t, d, seed):
    return datagen.unit_rows(datagen.normal(seed, q * t * d).reshape(q, t, d)).astype(np.float32)


def test_one_token_is_child_max():
    c = _corpus(20, 64, 64, 2)
    q = _tokens(3, 1, 64, 5)
    ms = oracle.tq_maxsim_scores(q, c.rotation, 64, 2, c.codebook, c.codebook_scale, c.codes,
                                 c.norms, 64)
    _, flat = oracle.tq_scores(q[:, 0], c.rotation, 64, 2, c.codebook, c.codebook_scale, c.codes,
                               c.norms)
    np.testing.assert_array_equal(ms, flat.reshape(3, 20, 64).max(axis=2))


def test_token_sum_is_pairwise_tree():
    c = _corpus(10, 32, 32, 4)
    q = _tokens(2, 7, 32, 6)
    ms = oracle.tq_maxsim_scores(q, c.rotation, 32, 4, c.codebook, c.codebook_scale, c.codes,
                                 c.norms, 32)
    per_tok = np.stack([oracle.tq_scores(q[:, t], c.rotation, 32, 4, c.codebook,
                                         c.codebook_scale, c.codes, c.norms)[1]
                        .reshape(2, 10, 32).max(axis=2) for t in range(7)], axis=2)
    slots = np.zeros((2, 10, 32), np.float32)
    slots[:, :, :7] = per_tok
    for o in (1, 2, 4, 8, 16):
        slots = (slots + slots[:, :, np.arange(32) ^ o]).astype(np.float32)
    np.testing.assert_array_equal(ms, slots[:, :, 0])
    # and it is the plain sum up to f32 rounding
    np.testing.assert_allclose(ms, per_tok.astype(np.float64).sum(axis=2), rtol=1e-5, atol=1e-6)


def _dev_index(rt, c):
    from eos_amd.turboquant import TurboQuantIndex
    return TurboQuantIndex(rt, c.codes, c.norms, c.dim, c.bits, c.codebook, c.codebook_scale,
                           c.rotation)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,d,doc_len,ntok,nq", [(2, 128, 128, 32, 9), (4, 384, 64, 5, 4),
                                                    (2, 64, 32, 1, 6), (4, 128, 96, 32, 1)])
def test_maxsim_matches_oracle(rt, bits, d, doc_len, ntok, nq):
    print(f"[case] maxsim bits={bits} d={d} doc_len={doc_len} tokens={ntok} Q={nq}", flush=True)
    from eos_amd.turboquant import TurboQuantMultiVectorIndex
    c = _corpus(300, doc_len, d, bits, seed=d + bits)
    q = _tokens(nq, ntok, d, 7)
    mv = TurboQuantMultiVectorIndex(_dev_index(rt, c), doc_len)
    got = mv.scores(q)
    want = oracle.tq_maxsim_scores(q, c.rotation, d, bits, c.codebook, c.codebook_scale, c.codes,
                                   c.norms, doc_len)
    np.testing.assert_array_equal(got, want)
    sub = mv.scores(q, 17, 100)
    np.testing.assert_array_equal(sub, want[:, 17:117])
    for k in (1, 10, 100, 0):
        ids, sc = mv.top_k(q, k)
        kk = 300 if k <= 0 else k
        for i in range(nq):
            order = np.lexsort((np.arange(300), -want[i]))[:kk]
            np.testing.assert_array_equal(ids[i], order)
            np.testing.assert_array_equal(sc[i], want[i][order])


@pytest.mark.gpu
def test_maxsim_topk_chunked_selection_with_ties(rt):
    """Enough documents that the top-k is selected per row chunk and then
    merged: copies of query 0's best document sit at the chunk edges (exact
    score ties, ranked by lower document index), and k covers the chunked
    sizes and one too large to merge (one workgroup per row)."""
    print("[case] maxsim chunked top-k 12000 docs with planted ties", flush=True)
    from eos_amd.turboquant import TurboQuantIndex, TurboQuantMultiVectorIndex
    ndocs, doc_len, d, bits = 12000, 32, 64, 2
    c = _corpus(ndocs, doc_len, d, bits, seed=41)
    q = _tokens(3, 2, d, 43)
    args = (c.rotation, d, bits, c.codebook, c.codebook_scale)
    first = oracle.tq_maxsim_scores(q[:1], *args, c.codes, c.norms, doc_len)
    best = int(np.argmax(first[0]))
    codes = c.codes.reshape(ndocs, doc_len, -1).copy()
    norms = c.norms.reshape(ndocs, doc_len).copy()
    for dst in (0, 2399, 2400, 4800, 11999):
        codes[dst], norms[dst] = codes[best], norms[best]
    codes = codes.reshape(ndocs * doc_len, -1)
    norms = norms.reshape(-1)
    want = oracle.tq_maxsim_scores(q, *args, codes, norms, doc_len)
    idx = TurboQuantIndex(rt, codes, norms, d, bits, c.codebook, c.codebook_scale, c.rotation)
    mv = TurboQuantMultiVectorIndex(idx, doc_len)
    for k in (1, 7, 100, 500, 2000):
        ids, sc = mv.top_k(q, k)
        for i in range(3):
            order = np.lexsort((np.arange(ndocs), -want[i]))[:k]
            np.testing.assert_array_equal(ids[i], order, err_msg=f"k={k} query {i}")
            np.testing.assert_array_equal(sc[i], want[i][order])
    tied = sorted({0, 2399, 2400, 4800, 11999, best})
    ids, _ = mv.top_k(q[:1], len(tied))
    assert ids[0].tolist() == tied
    idx.release()


@pytest.mark.gpu
def test_maxsim_zero_scores_keep_the_oracle_sign(rt):
    """Documents whose vectors all have norm 0 score (D * alpha) * 0, which is
    -0 for a negative dot; the score's + 0.0f makes it +0 before the token
    maximum. The device sums must carry the oracle's bits, sign of zero
    included (a float comparison would take -0 == +0)."""
    print("[case] maxsim zero-norm documents", flush=True)
    from eos_amd.turboquant import TurboQuantIndex, TurboQuantMultiVectorIndex
    d, bits, doc_len = 64, 2, 32
    c = _corpus(40, doc_len, d, bits, seed=29)
    norms = c.norms.copy()
    norms[: 10 * doc_len] = 0.0           # documents 0..9: every vector of norm 0
    norms[20 * doc_len: 21 * doc_len] = 0.0
    q = _tokens(3, 4, d, 31)
    idx = TurboQuantIndex(rt, c.codes, norms, c.dim, c.bits, c.codebook, c.codebook_scale,
                          c.rotation, zero_vector_allowed=True)
    mv = TurboQuantMultiVectorIndex(idx, doc_len)
    got = mv.scores(q)
    want = oracle.tq_maxsim_scores(q, c.rotation, d, bits, c.codebook, c.codebook_scale, c.codes,
                                   norms, doc_len)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(got[:, :10].view(np.uint32) == 0)  # +0, not -0
    idx.release()


@pytest.mark.gpu
def test_maxsim_rejects_bad_shapes(rt):
    print("[case] maxsim validation", flush=True)
    from eos_amd._lib import EosHipError
    from eos_amd.turboquant import TurboQuantMultiVectorIndex
    c = _corpus(4, 64, 64, 2)
    idx = _dev_index(rt, c)
    with pytest.raises(ValueError):
        TurboQuantMultiVectorIndex(idx, 48)
    mv = TurboQuantMultiVectorIndex(idx, 64)
    with pytest.raises(ValueError):
        mv.top_k(np.zeros((1, 33, 64), np.float32), 1)
    mv.doc_len = 96  # bypass the host check: the library must refuse too
    with pytest.raises(EosHipError):
        mv.scores(np.zeros((1, 2, 64), np.float32), 0, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,d", [(2, 64), (4, 96)])
def test_maxsim_bound_filter_matches_oracle(rt, bits, d):
    """20,000 documents take the bound-filtered top-k (sampled threshold,
    high-half bound filter, exact rescoring of the listed documents): ids and
    scores equal the oracle's, with copies of query 0's best document planted
    (exact ties, ranked by lower index), five queries (two passes of query
    groups) and k from 1 to the filtered path's limit; k = 600 takes the
    exhaustive path."""
    print(f"[case] maxsim bound filter 20000 docs bits={bits} d={d}", flush=True)
    from eos_amd.turboquant import TurboQuantIndex, TurboQuantMultiVectorIndex
    ndocs, doc_len = 20000, 32
    c = _corpus(ndocs, doc_len, d, bits, seed=53 + bits)
    q = _tokens(5, 8, d, 57 + bits)
    args = (c.rotation, d, bits, c.codebook, c.codebook_scale)
    first = oracle.tq_maxsim_scores(q[:1], *args, c.codes, c.norms, doc_len)
    best = int(np.argmax(first[0]))
    codes = c.codes.reshape(ndocs, doc_len, -1).copy()
    norms = c.norms.reshape(ndocs, doc_len).copy()
    for dst in (0, 7, 9999, 10000, 19999):
        codes[dst], norms[dst] = codes[best], norms[best]
    codes = codes.reshape(ndocs * doc_len, -1)
    norms = norms.reshape(-1)
    want = oracle.tq_maxsim_scores(q, *args, codes, norms, doc_len)
    idx = TurboQuantIndex(rt, codes, norms, d, bits, c.codebook, c.codebook_scale, c.rotation)
    mv = TurboQuantMultiVectorIndex(idx, doc_len)
    for k in (1, 6, 100, 512, 600):
        ids, sc = mv.top_k(q, k)
        for i in range(5):
            order = np.lexsort((np.arange(ndocs), -want[i]))[:k]
            np.testing.assert_array_equal(ids[i], order, err_msg=f"k={k} query {i}")
            np.testing.assert_array_equal(sc[i], want[i][order])
    idx.release()


@pytest.mark.gpu
def test_maxsim_bound_filter_falls_back_exactly(rt):
    """Cases the filter cannot prune are recomputed exhaustively on the
    device: identical documents (every document listed: the list overflows)
    and zero query tokens (every score 0, so tau = 0 prunes nothing); the top
    k is then documents 0 .. k-1, as the oracle ranks them."""
    print("[case] maxsim bound filter fallback", flush=True)
    from eos_amd.turboquant import TurboQuantIndex, TurboQuantMultiVectorIndex
    ndocs, doc_len, d, bits = 17000, 32, 64, 2
    c = _corpus(1, doc_len, d, bits, seed=61)
    codes = np.tile(c.codes, (ndocs, 1))
    norms = np.tile(c.norms, ndocs)
    q = _tokens(4, 3, d, 62)
    q[2] = 0.0  # a query whose every token is zero
    args = (c.rotation, d, bits, c.codebook, c.codebook_scale)
    want = oracle.tq_maxsim_scores(q, *args, codes[: 40 * doc_len], norms[: 40 * doc_len], doc_len)
    idx = TurboQuantIndex(rt, codes, norms, d, bits, c.codebook, c.codebook_scale, c.rotation)
    mv = TurboQuantMultiVectorIndex(idx, doc_len)
    ids, sc = mv.top_k(q, 30)
    for i in range(4):
        np.testing.assert_array_equal(ids[i], np.arange(30), err_msg=f"query {i}")
        np.testing.assert_array_equal(sc[i], want[i][:30])
    assert np.all(sc[2] == 0.0)
    idx.release()


@pytest.mark.gpu
def test_baseline_c5_full_size(rt):
    print("[case] c5 full size 100k x 128 x 128", flush=True)
    from eos_amd.turboquant import TurboQuantMultiVectorIndex
    c = datagen.TurboQuantCorpus(100_000 * 128, 128, 2, 11, 12, 13)
    q = _tokens(32, 32, 128, 14)
    mv = TurboQuantMultiVectorIndex(_dev_index(rt, c), 128)
    ids, sc = mv.top_k(q, 100)
    dense = mv.scores(q)
    for i in range(32):
        order = np.argsort(-dense[i], kind="stable")[:100]
        np.testing.assert_array_equal(ids[i], order)
        np.testing.assert_array_equal(sc[i], dense[i][order])
    docs = np.unique(np.concatenate([ids[:2].ravel(), np.arange(0, 100_000, 1000)]))
    sub_codes = c.codes.reshape(100_000, 128, -1)[docs].reshape(-1, c.codes.shape[1])
    sub_norms = c.norms.reshape(100_000, 128)[docs].reshape(-1)
    want = oracle.tq_maxsim_scores(q[:2], c.rotation, 128, 2, c.codebook, c.codebook_scale,
                                   sub_codes, sub_norms, 128)
    np.testing.assert_array_equal(dense[:2, docs], want)
