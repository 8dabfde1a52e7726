"""The rerank entry point that allocates nothing
(eoship_tq_fp16_rerank_device_noalloc, scores staged in a static device array)
against eoship_tq_fp16_rerank_device: ids and f32 scores bit-exact on two calls
in a row, the second with a smaller input, and a request beyond the static
scratch refused with an error. Collected last (test_zz_*) so that a failure
here hides no other test."""
import numpy as np
import pytest

from eos_amd._lib import EosHipError
from eos_amd.runtime import DeviceBuffer
from eos_amd.turboquant import F16Sidecar, string_id_rank, top_fp16_rerank_scores_device

pytestmark = pytest.mark.gpu


def _both(rt, side, q, cid, cs, k, overfetch, d_rank=None):
    nq, c = cid.shape
    kk = c if (k <= 0 or k > c) else k
    d_q = DeviceBuffer.from_array(rt, np.ascontiguousarray(q, np.float32))
    d_cid = DeviceBuffer.from_array(rt, np.ascontiguousarray(cid, np.int64))
    d_cs = DeviceBuffer.from_array(rt, np.ascontiguousarray(cs, np.float32))
    out = []
    for noalloc in (False, True):
        d_ids, d_sc = DeviceBuffer(rt, nq * kk * 8), DeviceBuffer(rt, nq * kk * 4)
        top_fp16_rerank_scores_device(side, d_q, nq, d_cid, d_cs, c, k, 4, overfetch, d_ids, d_sc,
                                      d_rank, noalloc=noalloc)
        out.append((d_ids.download(np.int64, (nq, kk)), d_sc.download(np.float32, (nq, kk))))
        d_ids.free()
        d_sc.free()
    for b in (d_q, d_cid, d_cs):
        b.free()
    return out


def _cands(rng, nq, n, c):
    cid = np.stack([rng.permutation(n)[:c] for _ in range(nq)]).astype(np.int64)
    cid[0, 3] = n + 5                      # a missing row: skipped by both
    cs = np.sort(rng.standard_normal(cid.shape).astype(np.float32), axis=1)[:, ::-1].copy()
    return cid, cs


def test_noalloc_rerank_matches_allocating_entry_point(rt):
    print("[case] noalloc rerank: 64 x 200 rescue, then 5 x 120 with string-id ties", flush=True)
    rng = np.random.default_rng(91)
    n, d = 5000, 384
    x = rng.standard_normal((n, d)).astype(np.float32)
    x[rng.integers(0, n, 400)] = x[11]     # exact duplicates: ties decided by the id order
    side = F16Sidecar(rt, x)
    q = rng.standard_normal((64, d)).astype(np.float32)
    # first call: the promoted profile (b4, top 100 of 200, rank-100 rescue)
    cid, cs = _cands(rng, 64, n, 200)
    (ia, sa), (ib, sb) = _both(rt, side, q, cid, cs, 100, 200)
    assert np.array_equal(ia, ib)
    assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    # second call, smaller: 5 queries x 120 candidates, every candidate kept,
    # ties ranked by string id; the scratch still holds the first call's scores
    cid, cs = _cands(rng, 5, n, 120)
    d_rank = DeviceBuffer.from_array(rt, string_id_rank([f"v{i}" for i in range(n)]))
    (ia, sa), (ib, sb) = _both(rt, side, q[:5], cid, cs, 0, 120, d_rank)
    d_rank.free()
    assert np.array_equal(ia, ib)
    assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    side.buf.free()


def test_noalloc_rerank_refuses_more_than_its_scratch(rt):
    print("[case] noalloc rerank: q * c above 2^20 refused", flush=True)
    side = F16Sidecar(rt, np.ones((8, 16), np.float32))
    nq, c = 257, 4096                       # 1052672 > 2^20 candidates
    d_q = DeviceBuffer(rt, nq * 16 * 4)
    d_cid = DeviceBuffer(rt, nq * c * 8)
    d_cs = DeviceBuffer(rt, nq * c * 4)
    d_ids, d_sc = DeviceBuffer(rt, nq * 100 * 8), DeviceBuffer(rt, nq * 100 * 4)
    with pytest.raises(EosHipError, match="static scratch"):
        top_fp16_rerank_scores_device(side, d_q, nq, d_cid, d_cs, c, 100, 4, c, d_ids, d_sc,
                                      noalloc=True)
    for b in (d_q, d_cid, d_cs, d_ids, d_sc):
        b.free()
    side.buf.free()


def test_noalloc_rerank_two_runtimes_interleaved(rt):
    """Two runtimes (two streams) on one GPU call the no-allocation rerank
    back to back without a synchronisation between them: the per-device
    event chain orders them on the shared static scratch, so each result
    equals the allocating entry point's bit for bit."""
    print("[case] noalloc rerank: two runtimes interleaved on one GPU", flush=True)
    from eos_amd.runtime import Runtime
    rng = np.random.default_rng(93)
    n, d = 4000, 256
    x = rng.standard_normal((n, d)).astype(np.float32)
    rt2 = Runtime(0)
    sides = (F16Sidecar(rt, x), F16Sidecar(rt2, x))
    runs = []
    for r, side, nq, c in ((rt, sides[0], 64, 200), (rt2, sides[1], 48, 160)):
        q = rng.standard_normal((nq, d)).astype(np.float32)
        cid, cs = _cands(rng, nq, n, c)
        d_q = DeviceBuffer.from_array(r, q)
        d_cid = DeviceBuffer.from_array(r, cid)
        d_cs = DeviceBuffer.from_array(r, cs)
        runs.append((r, side, nq, c, d_q, d_cid, d_cs, q, cid, cs))
    rt.sync()
    rt2.sync()
    # Outputs allocated first, so nothing between the calls synchronises.
    outs = [(r, DeviceBuffer(r, nq * 100 * 8), DeviceBuffer(r, nq * 100 * 4), nq)
            for rep in range(4) for r, side, nq, *_ in runs]
    for j, (r, d_ids, d_sc, nq) in enumerate(outs):
        _, side, _, c, d_q, d_cid, d_cs, *_ = runs[j % 2]
        top_fp16_rerank_scores_device(side, d_q, nq, d_cid, d_cs, c, 100, 4, c, d_ids, d_sc,
                                      noalloc=True)
    got = [(i.download(np.int64, (nq, 100)), s.download(np.float32, (nq, 100)))
           for r, i, s, nq in outs]
    for r, i, s, nq in outs:
        i.free()
        s.free()
    for j, (r, side, nq, c, d_q, d_cid, d_cs, q, cid, cs) in enumerate(runs):
        (ia, sa), _ = _both(r, side, q, cid, cs, 100, c)
        for rep in range(4):
            ib, sb = got[2 * rep + j]
            assert np.array_equal(ia, ib)
            assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
        for b in (d_q, d_cid, d_cs):
            b.free()
    for side in sides:
        side.buf.free()
    rt2.close()
