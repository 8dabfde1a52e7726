"""GPU parity of the dense and reconstruct (mixed-width) reranks against the
CPU oracle (oracle/rerank_oracle.c). Bar: bit-exact ids and scores."""
import numpy as np
import pytest

import oracle
from eos_amd.turboquant import dense_rerank_top_k, reconstruct_rerank_top_k

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _cands(rng, q, c, n, extra_bad=True):
    cid = np.stack([rng.permutation(n)[:c] for _ in range(q)]).astype(np.int64)
    if extra_bad:
        cid[0, 3] = -1
        cid[1, 5] = n + 7            # no row: skipped, as a missing docs[ID]
    return cid


@pytest.mark.parametrize("d,c,k", [(384, 200, 100), (256, 1000, 10), (37, 64, 0), (768, 4096, 100)])
def test_dense_rerank(rt, d, c, k):
    _case(f"dense rerank d={d} c={c} k={k}")
    rng = np.random.default_rng(d + c)
    n, q = 20_000, 16
    rows = rng.normal(size=(n, d)).astype(np.float32)
    rows[11] = rows[12]                               # exact ties: id order
    queries = rng.normal(size=(q, d)).astype(np.float32)
    cid = _cands(rng, q, c, n)
    cid[2, :2] = [12, 11]
    ids, sc = dense_rerank_top_k(rt, queries, rows, cid, k)
    wid, wsc = oracle.dense_rerank(queries, rows, cid, k)
    np.testing.assert_array_equal(ids, wid)
    np.testing.assert_array_equal(sc, wsc)


def test_dense_rerank_string_id_order(rt):
    """Equal scores break by the string-ID order (id_rank), as
    retrievalScoreBetter compares IDs (runtime/retrieval_eval.go:1153-1161)."""
    _case("dense rerank id_rank ties")
    n, d = 12, 8
    rows = np.zeros((n, d), np.float32)
    rows[:, 0] = 1.0
    queries = np.ones((1, d), np.float32)
    names = [f"d{i}" for i in range(n)]
    order = sorted(range(n), key=lambda i: names[i])
    id_rank = np.empty(n, np.int64)
    id_rank[order] = np.arange(n)
    cid = np.arange(n, dtype=np.int64)[None, ::-1].copy()
    ids, _ = dense_rerank_top_k(rt, queries, rows, cid, 5, id_rank=id_rank)
    assert [names[i] for i in ids[0]] == ["d0", "d1", "d10", "d11", "d2"]
    wid, _ = oracle.dense_rerank(queries, rows, cid, 5, id_rank=id_rank)
    np.testing.assert_array_equal(ids, wid)


@pytest.mark.parametrize("bits,d,rotate", [(4, 384, True), (8, 256, True), (2, 128, False),
                                           (1, 96, True), (3, 250, True)])
def test_reconstruct_rerank(rt, bits, d, rotate):
    """Primary 4-bit codes and an 8-bit sidecar set (mixed width), with and
    without a rotation."""
    _case(f"reconstruct rerank bits={bits} d={d} rotate={rotate}")
    rng = np.random.default_rng(bits * 1000 + d)
    n, q, c, k = 5000, 8, 300, 100
    codes = rng.integers(0, 256, size=(n, (d * bits + 7) // 8)).astype(np.uint8)
    codes[21] = codes[22]
    norms = np.exp(0.25 * rng.normal(size=n)).astype(np.float32)
    norms[22] = norms[21]
    cb = np.sort(rng.normal(size=1 << bits)).astype(np.float32) / np.sqrt(d)
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32) if rotate else None
    queries = rng.normal(size=(q, d)).astype(np.float32)
    cid = _cands(rng, q, c, n)
    cid[3, :2] = [22, 21]
    ids, sc = reconstruct_rerank_top_k(rt, queries, codes, bits, norms, cb, rot, cid, k)
    wid, wsc = oracle.reconstruct_rerank(queries, rot, codes, bits, norms, cb, cid, k)
    np.testing.assert_array_equal(ids, wid)
    np.testing.assert_array_equal(sc, wsc)


@pytest.mark.parametrize("bits,d", [(3, 256), (1, 384), (4, 130)])
def test_reconstruct_rerank_inner_product_set(rt, bits, d):
    """An inner-product code set (MSE codes + QJL signs + ResNorm + Norm, as
    eoship_tq_ip_encode_device writes it) dequantized with the QJL term, then
    the f32 index-order dots: ids and scores bit-exact vs the oracle."""
    _case(f"reconstruct rerank inner-product set bits={bits} d={d}")
    rng = np.random.default_rng(bits * 7 + d)
    n, q, c, k = 3000, 6, 200, 50
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32)
    S = rng.normal(size=(d, d)).astype(np.float32)
    pts = np.sort(rng.normal(size=1 << bits))
    cbi = np.clip(np.rint(pts / np.abs(pts).max() * 127), -127, 127).astype(np.int8)
    s_c = float(np.float32(2.2 / np.sqrt(d) / 127))
    x = rng.normal(size=(n, d)).astype(np.float32)
    x[7] = x[8]
    codes, signs, rn, nm = oracle.tq_encode_ip(x, rot, S, d, bits, cbi, s_c)
    cb = (cbi.astype(np.float32) * np.float32(s_c)).astype(np.float32)
    queries = rng.normal(size=(q, d)).astype(np.float32)
    cid = _cands(rng, q, c, n)
    cid[2, :2] = [8, 7]
    ids, sc = reconstruct_rerank_top_k(rt, queries, codes, bits, nm, cb, rot, cid, k,
                                       signs=signs, resnorms=rn, sketch=S)
    wid, wsc = oracle.reconstruct_rerank(queries, rot, codes, bits, nm, cb, cid, k, signs=signs,
                                         resnorms=rn, sketch=S)
    np.testing.assert_array_equal(ids, wid)
    np.testing.assert_array_equal(sc, wsc)
