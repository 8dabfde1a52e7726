"""GPU parity of the TurboQuant scan (libeoship on gfx950) against the CPU oracle.

Bar: prepared queries, integer code dot products, scores and top-k ids are
bit-exact against oracle/tq_oracle.c on the same seeded inputs; at the
benchmark size (1M x 384, 4-bit, 64 queries, k = 100) the filtered top-k must
equal the exhaustive device scores sorted by (score desc, id asc), and the
exhaustive scores must equal the oracle's on a sampled subset."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen
from eos_amd.turboquant import TurboQuantIndex, top_turboquant_retrieval_scores_with_stats

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _corpus(n, d, bits, seed=21, rotation=True):
    return datagen.TurboQuantCorpus(n, d, bits, seed, seed + 1, seed + 2, rotation=rotation)


def _index(rt, c, norms=None, codes=None, **kw):
    return TurboQuantIndex(rt, c.codes if codes is None else codes,
                           c.norms if norms is None else norms, c.dim, c.bits, c.codebook,
                           c.codebook_scale, c.rotation, **kw)


def _oracle_scores(c, q, norms=None, codes=None, begin=0, count=None):
    return oracle.tq_scores(q, c.rotation, c.dim, c.bits, c.codebook, c.codebook_scale,
                            c.codes if codes is None else codes,
                            c.norms if norms is None else norms, begin, count)


def test_prepare_bit_exact(rt):
    _case("prepare d=384 Q=70")
    c = _corpus(64, 384, 4)
    q = datagen.baseline_queries(70, 384, 7)
    idx = _index(rt, c)
    qs, alpha = idx.prepare_query(q)
    for i in range(70):
        oqs, oal = oracle.tq_prepare(q[i], c.rotation, c.codebook, c.codebook_scale)
        np.testing.assert_array_equal(qs[i], oqs)
        assert alpha[i] == oal


@pytest.mark.parametrize("bits,d,n,nq", [(4, 384, 1000, 64), (4, 384, 517, 33), (2, 128, 1000, 64),
                                         (4, 64, 300, 1), (4, 100, 333, 40), (2, 40, 95, 70),
                                         (4, 768, 200, 16), (2, 1024, 100, 5)])
def test_scores_and_dots_bit_exact(rt, bits, d, n, nq):
    _case(f"scores bits={bits} d={d} n={n} Q={nq}")
    c = _corpus(n, d, bits, seed=d + bits)
    q = datagen.baseline_queries(nq, d, 8)
    idx = _index(rt, c)
    dots, sc = idx.inner_product_prepared(q)
    odots, osc = _oracle_scores(c, q)
    np.testing.assert_array_equal(dots, odots)
    np.testing.assert_array_equal(sc, osc)
    # an unaligned slice
    b, cnt = n // 3 + 1, n // 2
    dots2, sc2 = idx.inner_product_prepared(q, b, cnt)
    np.testing.assert_array_equal(dots2, odots[:, b:b + cnt])
    np.testing.assert_array_equal(sc2, osc[:, b:b + cnt])


@pytest.mark.parametrize("n", [1000, 8192, 8193, 20000, 100000])
@pytest.mark.parametrize("bits,d", [(4, 384), (2, 128)])
def test_topk_matches_oracle(rt, n, bits, d):
    _case(f"topk n={n} bits={bits} d={d}")
    c = _corpus(n, d, bits, seed=n % 97 + bits)
    q = datagen.baseline_queries(64, d, 9)
    idx = _index(rt, c)
    for k in (1, 7, 100, 255):
        ids, sc, stats = idx.top_k(q, k)
        oids, osc = oracle.tq_topk(q, c.rotation, d, bits, c.codebook, c.codebook_scale, c.codes,
                                   c.norms, k)
        np.testing.assert_array_equal(ids, oids)
        np.testing.assert_array_equal(sc, osc)
        assert stats.candidate_count == 64 * n


def test_topk_multiple_batches(rt):
    _case("topk Q=130 n=30000")
    c = _corpus(30000, 384, 4, seed=5)
    q = datagen.baseline_queries(130, 384, 10)
    idx = _index(rt, c)
    ids, sc, stats = idx.top_k(q, 50)
    oids, osc = oracle.tq_topk(q, c.rotation, 384, 4, c.codebook, c.codebook_scale, c.codes,
                               c.norms, 50)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(sc, osc)
    assert stats.batches == 3


def test_topk_ties_at_the_cut_filter_path(rt):
    """Every vector appears 8 times (copies 5000 ids apart), so the k-th best
    score is tied across the cut; the filtered path (no fallback) must keep the
    lowest ids of the tied group, as the oracle's heap does."""
    _case("topk ties at the cut n=40000")
    c = _corpus(5000, 384, 4, seed=13)
    codes = np.tile(c.codes, (8, 1))
    norms = np.tile(c.norms, 8)
    q = datagen.baseline_queries(64, 384, 14)
    idx = _index(rt, c, norms=norms, codes=codes)
    for k in (1, 7, 100, 255):
        ids, sc, stats = idx.top_k(q, k)
        oids, osc = oracle.tq_topk(q, c.rotation, 384, 4, c.codebook, c.codebook_scale, codes,
                                   norms, k)
        np.testing.assert_array_equal(ids, oids)
        np.testing.assert_array_equal(sc, osc)
        assert stats.fallback_queries == 0


@pytest.mark.parametrize("k", [1024, 1025, 3000, 8192])
def test_topk_large_k_sorted_on_device(rt, k):
    """n <= the candidate capacity keeps every vector; large k orders the kept
    set with the bitonic sort instead of rank counting."""
    _case(f"topk n=8192 k={k}")
    c = _corpus(8192, 128, 2, seed=15)
    q = datagen.baseline_queries(5, 128, 16)
    idx = _index(rt, c)
    ids, sc, stats = idx.top_k(q, k)
    oids, osc = oracle.tq_topk(q, c.rotation, 128, 2, c.codebook, c.codebook_scale, c.codes,
                               c.norms, k)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(sc, osc)
    assert stats.fallback_queries == 0


def test_topk_all_ties_uses_exact_fallback(rt):
    """Every vector scores the same: the filter overflows, the exhaustive path
    must return ids 0..k-1 (ties to the lower id)."""
    _case("topk all ties n=20000")
    c = _corpus(20000, 384, 4, seed=6)
    codes = np.full_like(c.codes, 0x55)
    norms = np.ones(20000, np.float32)
    q = datagen.baseline_queries(8, 384, 11)
    idx = _index(rt, c, norms=norms, codes=codes)
    ids, sc, stats = idx.top_k(q, 100)
    np.testing.assert_array_equal(ids, np.tile(np.arange(100), (8, 1)))
    oids, osc = oracle.tq_topk(q, c.rotation, 384, 4, c.codebook, c.codebook_scale, codes, norms, 100)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(sc, osc)
    assert stats.fallback_queries == 8


def test_topk_deferred_status_and_repair(rt):
    """The deferred device path flags exactly the rows the filter cannot prove;
    after repair_device every row equals the oracle's (clean corpus: no flags,
    same rows as the gated device path; all-ties corpus: every row flagged)."""
    from eos_amd.runtime import DeviceBuffer
    _case("topk deferred + repair")
    c = _corpus(30000, 384, 4, seed=17)
    q = datagen.baseline_queries(70, 384, 18)
    for codes, norms, expect_flags in ((c.codes, c.norms, False),
                                       (np.full_like(c.codes, 0x55), np.ones(c.n, np.float32), True)):
        idx = _index(rt, c, norms=norms, codes=codes)
        k = 100
        dq = DeviceBuffer.from_array(rt, q)
        dids = DeviceBuffer(rt, 70 * k * 8)
        dsc = DeviceBuffer(rt, 70 * k * 4)
        dst = DeviceBuffer(rt, 70 * 4)
        idx.top_k_device_deferred(dq, 70, k, dids, dsc, dst)
        status = dst.download(np.int32, (70,))
        assert bool(np.any(status != 0)) == expect_flags
        if expect_flags:
            assert np.all(status != 0)
        idx.repair_device(dq, 70, k, dids, dsc, dst)
        ids = dids.download(np.int64, (70, k))
        sc = dsc.download(np.float32, (70, k))
        oids, osc = oracle.tq_topk(q, c.rotation, 384, 4, c.codebook, c.codebook_scale, codes,
                                   norms, k)
        np.testing.assert_array_equal(ids, oids)
        np.testing.assert_array_equal(sc, osc)
        idx.release()


def test_shared_handle_concurrent_batches(rt):
    """eoship_tq_share: a second handle on another runtime (stream) shares the
    resident corpus; batches enqueued on both streams at once give the
    oracle's rows, and the second handle keeps working after the original is
    released (the corpus is freed with the last handle)."""
    from eos_amd.runtime import DeviceBuffer, Runtime
    _case("shared handle, two streams")
    c = _corpus(50000, 384, 4, seed=23)
    qa = datagen.baseline_queries(64, 384, 24)
    qb = datagen.baseline_queries(40, 384, 25)
    k = 50
    idx = _index(rt, c)
    rt2 = Runtime(0)
    idx2 = idx.share(rt2)
    bufs = []
    for r, q in ((rt, qa), (rt2, qb)):
        bufs.append((DeviceBuffer.from_array(r, q), DeviceBuffer(r, len(q) * k * 8),
                     DeviceBuffer(r, len(q) * k * 4)))
    for rep in range(3):
        idx.top_k_device(bufs[0][0], 64, k, bufs[0][1], bufs[0][2], with_stats=False)
        idx2.top_k_device(bufs[1][0], 40, k, bufs[1][1], bufs[1][2], with_stats=False)
    rt.wait_for(rt2)
    rt.sync()
    for (dq, dids, dsc), q in zip(bufs, (qa, qb)):
        ids = dids.download(np.int64, (len(q), k))
        sc = dsc.download(np.float32, (len(q), k))
        oids, osc = oracle.tq_topk(q, c.rotation, 384, 4, c.codebook, c.codebook_scale, c.codes,
                                   c.norms, k)
        np.testing.assert_array_equal(ids, oids)
        np.testing.assert_array_equal(sc, osc)
    idx.release()
    ids, sc, _ = idx2.top_k(qb, k)
    oids, osc = oracle.tq_topk(qb, c.rotation, 384, 4, c.codebook, c.codebook_scale, c.codes,
                               c.norms, k)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(sc, osc)
    for b in bufs:
        for x in b:
            x.free()
    idx2.release()
    rt2.close()


def test_topk_zero_norms_zero_query_and_k_semantics(rt):
    _case("topk edge cases")
    c = _corpus(500, 384, 4, seed=7)
    norms = c.norms.copy()
    norms[::3] = 0.0
    idx = _index(rt, c, norms=norms, zero_vector_allowed=True)
    q = datagen.baseline_queries(3, 384, 12)
    q[1] = 0.0
    for k in (0, -5, 500, 10_000, 1):
        ids, sc, _ = idx.top_k(q, k)
        oids, osc = oracle.tq_topk(q, c.rotation, 384, 4, c.codebook, c.codebook_scale, c.codes,
                                   norms, k)
        assert ids.shape == oids.shape
        np.testing.assert_array_equal(ids, oids)
        np.testing.assert_array_equal(sc, osc)
    ids, sc, _ = idx.top_k(q[1:2], 10)
    np.testing.assert_array_equal(ids[0], np.arange(10))
    assert np.all(sc == 0.0) and not np.any(np.signbit(sc))


def test_reference_tie_case(rt):
    """runtime/turboquant_retrieval_pruning_test.go:80-99 with integer ids."""
    _case("reference tie case")
    c = _corpus(2, 32, 4, seed=8)
    idx = _index(rt, c, norms=np.zeros(2, np.float32), zero_vector_allowed=True)
    q = np.zeros((1, 32), np.float32)
    q[0, 0] = 1.0
    docs, _ = top_turboquant_retrieval_scores_with_stats(idx, q, 1)
    assert len(docs[0]) == 1 and docs[0][0].id == 0 and docs[0][0].score == 0.0


def test_bind_rejects_bad_norms(rt):
    _case("bind validation")
    from eos_amd._lib import EosHipError
    c = _corpus(10, 32, 4, seed=9)
    bad = c.norms.copy()
    bad[4] = -1.0
    with pytest.raises(EosHipError, match="Norm"):
        _index(rt, c, norms=bad)
    bad[4] = np.nan
    with pytest.raises(EosHipError, match="Norm"):
        _index(rt, c, norms=bad)
    bad[4] = np.inf
    with pytest.raises(EosHipError, match="Norm"):
        _index(rt, c, norms=bad)
    with pytest.raises(EosHipError, match="Norm"):   # -1 even when zero vectors are allowed
        bad[4] = -1.0
        _index(rt, c, norms=bad, zero_vector_allowed=True)


def test_zero_norm_needs_zero_vector_allowed(rt):
    """validateEosQuantizedVectorNorm (runtime/turboquant_quantized_vector.go:
    25-34): Norm == 0 is the dropped-norm footgun unless the caller confirms a
    genuine zero vector, per vector."""
    _case("bind zero-norm policy")
    from eos_amd._lib import EosHipError
    c = _corpus(10, 32, 4, seed=9)
    z = c.norms.copy()
    z[6] = 0.0
    with pytest.raises(EosHipError, match="vector 6 has Norm 0"):
        _index(rt, c, norms=z)
    allow = np.zeros(10, bool)
    allow[5] = True                                  # another vector: still refused
    with pytest.raises(EosHipError, match="vector 6 has Norm 0"):
        _index(rt, c, norms=z, zero_vector_allowed=allow)
    allow[6] = True
    idx = _index(rt, c, norms=z, zero_vector_allowed=allow)
    q = datagen.baseline_queries(2, 32, 3)
    _, sc = idx.inner_product_prepared(q)
    assert np.all(sc[:, 6] == 0.0)
    idx.release()
    _index(rt, c, zero_vector_allowed=allow).release()   # positive norms need no flag


def _ranked_oracle(c, codes, norms, q, k, rank):
    """The oracle on the corpus laid out in string-ID order, mapped back: its
    index tie order is then the string-ID order."""
    inv = np.empty_like(rank)
    inv[rank] = np.arange(rank.size)
    pids, psc = oracle.tq_topk(q, c.rotation, c.dim, c.bits, c.codebook, c.codebook_scale,
                               codes[inv], norms[inv], k)
    return inv[pids], psc


def test_string_id_tie_order(rt):
    """Equal scores rank by string ID (retrievalScoreBetter,
    runtime/retrieval_eval.go:1153-1161): with IDs "d0".."d11" and all scores
    equal the order is d0, d1, d10, d11, d2, ..., not the index order."""
    _case("string id ties (small)")
    from eos_amd.turboquant import string_id_rank
    c = _corpus(12, 64, 4, seed=41)
    codes = np.repeat(c.codes[:1], 12, axis=0)
    norms = np.ones(12, np.float32)
    names = [f"d{i}" for i in range(12)]
    idx = _index(rt, c, norms=norms, codes=codes, ids=names)
    q = datagen.baseline_queries(2, 64, 5)
    ids, sc, _ = idx.top_k(q, 5)
    want = [0, 1, 10, 11, 2]
    np.testing.assert_array_equal(ids, [want, want])
    assert np.all(sc == sc[:, :1])
    rank = string_id_rank(names)
    np.testing.assert_array_equal(rank, [0, 1, 4, 5, 6, 7, 8, 9, 10, 11, 2, 3])
    # scores are still addressed by vector index
    _, dense = idx.inner_product_prepared(q, 3, 6)
    np.testing.assert_array_equal(dense, np.repeat(sc[:, :1], 6, axis=1))
    idx.release()


def test_string_id_ties_at_the_cut_filter_path(rt):
    """Filter path (n > 8192) with heavy exact ties at the top-k cut: 20000
    vectors drawn from 40 distinct code rows, IDs with mixed widths."""
    _case("string id ties (filter path)")
    c = _corpus(20000, 128, 4, seed=43)
    rng = np.random.default_rng(44)
    pick = rng.integers(0, 40, size=20000)
    codes = np.ascontiguousarray(c.codes[pick])
    norms = np.ones(20000, np.float32)
    names = [f"doc-{int(i)}" for i in rng.permutation(20000)]
    idx = _index(rt, c, norms=norms, codes=codes, ids=names)
    q = datagen.baseline_queries(8, 128, 45)
    for k in (100, 700):
        ids, sc, _ = idx.top_k(q, k)
        wids, wsc = _ranked_oracle(c, codes, norms, q, k, idx.id_rank)
        np.testing.assert_array_equal(ids, wids)
        np.testing.assert_array_equal(sc, wsc)
        plain, _ = oracle.tq_topk(q, c.rotation, 128, 4, c.codebook, c.codebook_scale, codes,
                                  norms, k)
        assert not np.array_equal(plain, wids)   # the two tie orders differ here
    idx.release()


def test_ranked_corpus_refuses_documents_and_parents(rt):
    _case("ranked corpus: documents / parents refused")
    from eos_amd._lib import EosHipError
    from eos_amd.turboquant import TurboQuantMultiVectorIndex, TurboQuantParents
    c = _corpus(64, 32, 4, seed=46)
    idx = _index(rt, c, ids=[str(i) for i in range(64)])
    with pytest.raises(EosHipError, match="index order"):
        TurboQuantMultiVectorIndex(idx, 32).scores(datagen.baseline_queries(1, 32, 1))
    with pytest.raises(EosHipError, match="index order"):
        TurboQuantParents(idx, np.array([0, 10, 64]))
    with pytest.raises(EosHipError, match="permutation"):
        _lib_bind_bad_rank(rt, c)
    idx.release()


def _lib_bind_bad_rank(rt, c):
    import ctypes as C
    from eos_amd import _lib
    rank = np.zeros(c.n, np.int64)   # not a permutation
    cb = np.ascontiguousarray(c.codebook, np.int8)
    desc = _lib.EosHipTQDesc(dim=c.dim, bits=c.bits, codebook_scale=float(c.codebook_scale),
                             codebook=cb.ctypes.data_as(C.POINTER(C.c_int8)), rotation=None)
    opts = _lib.EosHipTQBindOptions()
    opts.id_rank = rank.ctypes.data_as(C.POINTER(C.c_int64))
    h = C.c_void_p()
    _lib.call("eoship_tq_bind_corpus_opts", rt.handle, C.byref(desc),
              c.codes.ctypes.data_as(C.c_void_p), c.norms.ctypes.data_as(C.c_void_p),
              C.c_int64(c.n), C.byref(opts), C.byref(h))


def test_baseline_c2_full_size(rt):
    """Benchmark config c2 at full size: 1M x 384 4-bit, 64 queries, k = 100."""
    _case("c2 full size 1M x 384")
    c = datagen.baseline_flat_corpus()
    q = datagen.baseline_queries(64, 384)
    idx = _index(rt, c)
    ids, sc, stats = idx.top_k(q, 100)
    assert stats.fallback_queries == 0
    dots, dense = idx.inner_product_prepared(q)
    for i in range(64):
        order = np.argsort(-dense[i], kind="stable")[:100]
        np.testing.assert_array_equal(ids[i], order)
        np.testing.assert_array_equal(sc[i], dense[i][order])
    rng = np.random.default_rng(0)
    sub = np.sort(rng.choice(c.n, 2048, replace=False))
    odots, osc = oracle.tq_scores(q, c.rotation, 384, 4, c.codebook, c.codebook_scale,
                                  c.codes[sub], c.norms[sub])
    np.testing.assert_array_equal(dots[:, sub], odots)
    np.testing.assert_array_equal(dense[:, sub], osc)
    oids, osc2 = oracle.tq_topk(q[:2], c.rotation, 384, 4, c.codebook, c.codebook_scale, c.codes,
                                c.norms, 100)
    np.testing.assert_array_equal(ids[:2], oids)
    np.testing.assert_array_equal(sc[:2], osc2)
