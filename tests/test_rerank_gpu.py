"""GPU parity of the two-stage retrieval's second stage (eos_tq_f16_sidecar,
eos_tq_fp16_rerank through the C ABI) against the CPU oracle. Bar: halves,
rerank ids and f32 scores bit-exact, including the rank-100 rescue of the
b4 / overfetch 200 / top 100 profile and the reference's own rescue fixture."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen
from eos_amd.runtime import DeviceBuffer
from eos_amd.turboquant import (F16Sidecar, TurboQuantIndex, top_fp16_rerank_scores_device,
                                turboquant_fp16_rerank_top_k)

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _rerank(rt, side, q, cid, cs, k, bits, overfetch):
    nq, c = cid.shape
    d_q = DeviceBuffer.from_array(rt, np.ascontiguousarray(q, np.float32))
    d_cid = DeviceBuffer.from_array(rt, np.ascontiguousarray(cid, np.int64))
    d_cs = DeviceBuffer.from_array(rt, np.ascontiguousarray(cs, np.float32))
    kk = c if (k <= 0 or k > c) else k
    d_ids, d_sc = DeviceBuffer(rt, nq * kk * 8), DeviceBuffer(rt, nq * kk * 4)
    top_fp16_rerank_scores_device(side, d_q, nq, d_cid, d_cs, c, k, bits, overfetch, d_ids, d_sc)
    return d_ids.download(np.int64, (nq, kk)), d_sc.download(np.float32, (nq, kk))


def test_sidecar_bit_exact(rt):
    _case("f16 sidecar 4096 x 37 incl. ties, subnormals, overflow")
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4096, 37)) * np.exp(rng.uniform(-18, 12, (4096, 37)))).astype(np.float32)
    special = np.array([1.0, np.uint32(0x3F801000).view(np.float32), 65519.0, 65520.0, 70000.0,
                        np.inf, -np.inf, 2.0 ** -25, 2.0 ** -24, -0.0, 0.0], np.float32)
    x.ravel()[:special.size] = special
    side = F16Sidecar(rt, x)
    assert np.array_equal(side.halves(), oracle.f32_to_half(x))


def test_rerank_known_answer_sums(rt):
    _case("rerank sequential-sum and no-FMA known answers")
    third = np.float32(1.0) / np.float32(3.0)
    for q, row, want in (([1, 1, 1, 1], [1.0, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24], 1.0),
                         ([1.0, third], [-1.0, 3.0], 0.0)):
        side = F16Sidecar(rt, np.array([row], np.float32))
        ids, sc = _rerank(rt, side, np.array([q], np.float32), np.array([[0]], np.int64),
                          np.zeros((1, 1), np.float32), 1, 4, 200)
        assert ids[0, 0] == 0 and sc[0, 0].view(np.uint32) == np.float32(want).view(np.uint32)


@pytest.mark.parametrize("n", [119, 121])
def test_reference_rescue_fixture(rt, n):
    _case(f"rescue fixture n={n}")
    d = 8
    x = np.zeros((n + 1, d), np.float32)
    x[1:, 0] = (n - np.arange(n)).astype(np.float32)   # doc i+1 scores n-i
    side = F16Sidecar(rt, x)
    q = np.zeros((1, d), np.float32)
    q[0, 0] = 1
    order = list(range(1, n + 1))
    comp = [float(n - i) for i in range(n)]
    if n == 121:   # d120 strongest at the first stage (rank 1)
        order = [120] + [i for i in order if i != 120]
        comp = [10000.0] + [float(n - i + 1) for i in order[1:]]
    cid = np.array([order], np.int64)
    cs = np.array([comp], np.float32)
    ids, sc = _rerank(rt, side, q, cid, cs, 100, 4, 200)
    wids, wsc = oracle.fp16_rerank(q, side.halves(), cid, cs, 100, 4, 200)
    assert np.array_equal(ids, wids) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    if n == 121:
        assert ids[0, 99] == 120 and 100 not in ids[0, :100].tolist()
    else:
        assert ids[0].tolist() == list(range(1, 101))


def test_rerank_edges(rt):
    _case("rerank edges: missing ids, k=0, k>c, odd dim")
    rng = np.random.default_rng(9)
    n, d = 500, 13
    side = F16Sidecar(rt, rng.standard_normal((n, d)).astype(np.float32))
    q = rng.standard_normal((3, d)).astype(np.float32)
    cid = np.stack([rng.permutation(n)[:64] for _ in range(3)]).astype(np.int64)
    cid[0, 3], cid[1, 10], cid[2, :] = -1, n + 7, -1
    cs = rng.standard_normal(cid.shape).astype(np.float32)
    for k in (0, 10, 64, 100):
        ids, sc = _rerank(rt, side, q, cid, cs, k, 4, 200)
        wids, wsc = oracle.fp16_rerank(q, side.halves(), cid, cs, k, 4, 200)
        assert np.array_equal(ids, wids) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    assert (ids[2] == -1).all()


@pytest.mark.parametrize("k,overfetch", [(100, 200), (100, 300), (150, 200)])
def test_two_stage_end_to_end(rt, k, overfetch):
    _case(f"two-stage 20000 x 384 b4 Q=16 k={k} overfetch={overfetch}")
    c = datagen.TurboQuantCorpus(20000, 384, 4, 41, 42, 43, rotation=True)
    rng = np.random.default_rng(44)
    docs = rng.standard_normal((c.n, c.dim)).astype(np.float32)
    docs /= np.linalg.norm(docs, axis=1, keepdims=True)
    q = rng.standard_normal((16, c.dim)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    idx = TurboQuantIndex(rt, c.codes, c.norms, c.dim, c.bits, c.codebook, c.codebook_scale,
                          c.rotation)
    side = F16Sidecar(rt, docs)
    ids, sc, cand = turboquant_fp16_rerank_top_k(idx, side, q, k, overfetch, bit_width=4)
    wc_ids, wc_sc = oracle.tq_topk(q, c.rotation, c.dim, c.bits, c.codebook, c.codebook_scale,
                                   c.codes, c.norms, overfetch)
    assert np.array_equal(cand, wc_ids)
    wids, wsc = oracle.fp16_rerank(q, oracle.f32_to_half(docs), wc_ids, wc_sc, k, 4, overfetch)
    assert np.array_equal(ids, wids) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))


def test_rerank_subnormal_and_infinite_rows(rt):
    """Rows holding subnormal halves, signed zeros and infinities (d a multiple
    of 8, the vectorised path): scores equal the oracle's bit for bit."""
    _case("rerank subnormal / inf rows")
    rng = np.random.default_rng(12)
    n, d = 64, 16
    x = (rng.standard_normal((n, d)) * 2.0 ** rng.integers(-26, -12, (n, d))).astype(np.float32)
    x[5, 3], x[6, 0], x[7, 7] = np.inf, -np.inf, -0.0
    side = F16Sidecar(rt, x)
    h = side.halves()
    assert np.any((h & 0x7c00) == 0) and np.any(((h & 0x7c00) == 0) & ((h & 0x3ff) != 0))
    q = rng.standard_normal((4, d)).astype(np.float32)
    q[3] = np.abs(q[3])
    cid = np.stack([rng.permutation(n)[:40] for _ in range(4)]).astype(np.int64)
    cs = np.zeros(cid.shape, np.float32)
    ids, sc = _rerank(rt, side, q, cid, cs, 40, 4, 200)
    wids, wsc = oracle.fp16_rerank(q, h, cid, cs, 40, 4, 200)
    assert np.array_equal(ids, wids) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))


def test_rerank_large_candidate_lists(rt):
    """c above the old 1024 limit (the reference takes any overfetch), up to the
    4096 this kernel holds; 4097 is refused with a message."""
    _case("rerank c=3000 and c=4096; c=4097 refused")
    from eos_amd._lib import EosHipError
    rng = np.random.default_rng(13)
    n, d = 6000, 64
    side = F16Sidecar(rt, rng.standard_normal((n, d)).astype(np.float32))
    q = rng.standard_normal((3, d)).astype(np.float32)
    for c in (3000, 4096):
        cid = np.stack([rng.permutation(n)[:c] for _ in range(3)]).astype(np.int64)
        cs = np.sort(rng.standard_normal(cid.shape).astype(np.float32), axis=1)[:, ::-1].copy()
        for k in (100, 0):
            ids, sc = _rerank(rt, side, q, cid, cs, k, 4, c)
            wids, wsc = oracle.fp16_rerank(q, side.halves(), cid, cs, k, 4, c)
            assert np.array_equal(ids, wids)
            assert np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    cid = np.zeros((1, 4097), np.int64)
    with pytest.raises(EosHipError, match="4096"):
        _rerank(rt, side, q[:1], cid, np.zeros((1, 4097), np.float32), 100, 4, 4097)


def test_rerank_string_id_ties(rt):
    """Equal rerank scores rank by string ID when the ID order is given
    (retrievalScoreBetter, runtime/retrieval_eval.go:1153-1161)."""
    _case("rerank string-id ties")
    from eos_amd.turboquant import string_id_rank
    rng = np.random.default_rng(14)
    n, d = 300, 24
    x = rng.standard_normal((n, d)).astype(np.float32)
    x[rng.integers(0, n, 200)] = x[7]          # many exact duplicates of row 7
    side = F16Sidecar(rt, x)
    names = [f"p{int(i)}" for i in rng.permutation(n)]
    rank = string_id_rank(names)
    q = rng.standard_normal((2, d)).astype(np.float32)
    cid = np.stack([rng.permutation(n)[:150] for _ in range(2)]).astype(np.int64)
    cs = np.zeros(cid.shape, np.float32)
    d_q = DeviceBuffer.from_array(rt, q)
    d_cid = DeviceBuffer.from_array(rt, cid)
    d_cs = DeviceBuffer.from_array(rt, cs)
    d_rank = DeviceBuffer.from_array(rt, rank)
    d_ids, d_sc = DeviceBuffer(rt, 2 * 150 * 8), DeviceBuffer(rt, 2 * 150 * 4)
    top_fp16_rerank_scores_device(side, d_q, 2, d_cid, d_cs, 150, 0, 4, 200, d_ids, d_sc, d_rank)
    ids = d_ids.download(np.int64, (2, 150))
    sc = d_sc.download(np.float32, (2, 150))
    # the oracle over rows laid out in ID order ranks ties by position = ID order
    inv = np.empty_like(rank)
    inv[rank] = np.arange(n)
    wpos, wsc = oracle.fp16_rerank(q, side.halves()[inv], rank[cid], cs, 0, 4, 200)
    assert np.array_equal(ids, inv[wpos])
    assert np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    plain, _ = oracle.fp16_rerank(q, side.halves(), cid, cs, 0, 4, 200)
    assert not np.array_equal(plain, ids)


@pytest.mark.parametrize("k,overfetch", [(100, 200), (100, 250)])
def test_two_stage_inner_product_first_stage(rt, k, overfetch):
    """The promoted profile as the reference runs it: an inner-product (b = 4:
    3-bit MSE + QJL) first stage over the encoded documents, top-overfetch,
    then the f16 rerank whose rescue gate sees bit width 4: ids and scores
    bit-exact vs the oracle's IP scores + top-k + f16 rerank."""
    _case(f"two-stage IP b4 first stage k={k} overfetch={overfetch}")
    from eos_amd.turboquant import IPQuantizer
    n, d = 12000, 384
    rng = np.random.default_rng(45)
    docs = rng.standard_normal((n, d)).astype(np.float32)
    docs /= np.linalg.norm(docs, axis=1, keepdims=True)
    q = rng.standard_normal((8, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32)
    S = rng.normal(size=(d, d)).astype(np.float32)
    cb, s_c = datagen.turboquant_codebook(3, d)
    qz = IPQuantizer(rt, d, 3, cb, s_c, rot, S)
    codes, signs, rn, nm = qz.encode(docs)
    idx = qz.bind(codes, signs, rn, nm)
    side = F16Sidecar(rt, docs)
    ids, sc, cand = turboquant_fp16_rerank_top_k(idx, side, q, k, overfetch)
    full = oracle.tq_ip_scores(q, rot, S, d, 3, cb, s_c, codes, signs, rn, nm)
    wc = [oracle.topk_scores(r, overfetch) for r in full]
    wc_ids = np.stack([w[0] for w in wc])
    wc_sc = np.stack([w[1] for w in wc])
    assert np.array_equal(cand, wc_ids)
    wids, wsc = oracle.fp16_rerank(q, oracle.f32_to_half(docs), wc_ids, wc_sc, k, 4, overfetch)
    assert np.array_equal(ids, wids) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    idx.release()
    qz.release()
