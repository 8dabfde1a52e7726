"""TurboQuant retrieval scoring on the MI355X backend.

Host-side mirror of the reference's scoring entry points, with the same names,
argument meaning and error behaviour:

* ``TurboQuantIndex``  -- the bound corpus; the device-resident counterpart of
  ``[]turboQuantRetrievalDoc`` + ``*turboquant.IPQuantizer``
  (runtime/retrieval_turboquant.go:699-711).
* ``top_turboquant_retrieval_scores_with_stats`` --
  ``topTurboQuantRetrievalScoresWithStats`` (runtime/retrieval_turboquant.go:1853-1887):
  top-k by score descending, ties by id ascending (runtime/retrieval_eval.go:1153-1161);
  ``top_k <= 0`` or ``top_k > len(docs)`` means all documents (:1854-1856).
* ``TurboQuantIndex.inner_product_prepared`` -- ``InnerProductPrepared`` over a
  slice of documents (runtime/retrieval_turboquant.go:1874), with the exact
  integer code dot products.
* ``TurboQuantMultiVectorIndex`` -- MaxSim over fixed-size documents.
* ``TurboQuantParents`` / ``top_turboquant_multivector_parent_scores`` --
  ``topTurboQuantMultiVectorParentScores`` over ragged parents with the
  max / topN-mean aggregations and the child-count penalty
  (runtime/retrieval_multivector_turboquant.go:746-908).

All arithmetic runs in libeoship's gfx950 kernels; nothing here computes scores.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, Runtime


def string_id_rank(ids) -> np.ndarray:
    """Position of each ID among the IDs sorted ascending by Go string order
    (bytewise UTF-8), as int64 [n]; IDs must be distinct."""
    keys = [str(x).encode("utf-8") for x in ids]
    order = sorted(range(len(keys)), key=lambda i: keys[i])
    rank = np.empty(len(keys), np.int64)
    rank[np.asarray(order, dtype=np.int64)] = np.arange(len(keys), dtype=np.int64)
    if len(set(keys)) != len(keys):
        raise ValueError("document IDs must be distinct")
    return rank


def turboquant_vector_bytes(dim: int, bit_width: int) -> int:
    """turboquantVectorBytes (runtime/turboquant_bytes.go:14-25): MSE codes at
    bit_width - 1 bits, QJL signs at one bit per coordinate, plus Norm and
    ResNorm (8 bytes)."""
    out = C.c_int64()
    _lib.call("eoship_tq_vector_bytes", C.c_int32(dim), C.c_int32(bit_width), C.byref(out))
    return int(out.value)


def turboquant_mse_vector_bytes(dim: int, bits: int) -> int:
    """Bytes per vector of the MSE-stage layout bound here: codes + one f32 Norm."""
    out = C.c_int64()
    _lib.call("eoship_tq_mse_vector_bytes", C.c_int32(dim), C.c_int32(bits), C.byref(out))
    return int(out.value)


@dataclass
class RetrievalScoredDoc:
    """One ranked result (runtime/retrieval_eval.go retrievalScoredDoc): ID is the vector index."""
    id: int
    score: float


@dataclass
class TurboQuantRetrievalScoreStats:
    """Counterpart of turboQuantRetrievalScoreStats (runtime/retrieval_turboquant.go:1857-1887)."""
    candidate_count: int = 0
    candidates_scored: int = 0
    candidates_kept: int = 0
    fallback_queries: int = 0
    batches: int = 0
    pruning_supported: bool = False
    pruning_used: bool = False


class TurboQuantIndex:
    """A TurboQuant corpus bound on the device.

    codes: uint8 [n, ceil(dim*bits/8)] (coordinate j at bit (j*bits)%8 of byte
    (j*bits)//8, low bits first); norms: float32 [n], finite and > 0 (the
    Norm policy of validateEosQuantizedVectorNorm,
    runtime/turboquant_quantized_vector.go:25-34); codebook: int8 [2^bits]
    grid values with f32 scale; rotation: float32 [dim, dim] orthogonal (None =
    identity).

    zero_vector_allowed: None, True (every vector of Norm 0 is a confirmed
    genuine zero vector) or a bool array [n] (zeroVectorAllowed per vector).
    ids: None (IDs order like the indices) or the documents' string IDs [n];
    equal scores then rank by string ID ascending (retrievalScoreBetter,
    runtime/retrieval_eval.go:1153-1161), and results still report indices.
    """

    def __init__(self, rt: Runtime, codes: np.ndarray, norms: np.ndarray, dim: int, bits: int,
                 codebook: np.ndarray, codebook_scale: float, rotation: np.ndarray | None = None,
                 zero_vector_allowed=None, ids=None):
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        norms = np.ascontiguousarray(norms, dtype=np.float32)
        n = int(norms.shape[0])
        row_bytes = (dim * bits + 7) // 8
        if codes.shape != (n, row_bytes):
            raise ValueError(f"codes must have shape ({n}, {row_bytes}), got {codes.shape}")
        cb = np.ascontiguousarray(codebook, dtype=np.int8)
        if cb.shape != (1 << bits,):
            raise ValueError(f"codebook must have {1 << bits} entries")
        rot = None if rotation is None else np.ascontiguousarray(rotation, dtype=np.float32)
        if rot is not None and rot.shape != (dim, dim):
            raise ValueError("rotation must be dim x dim")
        self.rt, self.n, self.dim, self.bits = rt, n, dim, bits
        desc = _lib.EosHipTQDesc(
            dim=dim, bits=bits, codebook_scale=float(codebook_scale),
            codebook=cb.ctypes.data_as(C.POINTER(C.c_int8)),
            rotation=rot.ctypes.data_as(C.POINTER(C.c_float)) if rot is not None else None)
        self.handle = C.c_void_p()
        self.id_rank = None
        opts = _lib.EosHipTQBindOptions()
        keep = []
        if zero_vector_allowed is not None:
            z = np.broadcast_to(np.asarray(zero_vector_allowed, dtype=bool), (n,))
            z = np.ascontiguousarray(z, dtype=np.uint8)
            keep.append(z)
            opts.zero_vector_allowed = z.ctypes.data_as(C.POINTER(C.c_uint8))
        if ids is not None:
            self.id_rank = string_id_rank(ids)
            if self.id_rank.shape != (n,):
                raise ValueError(f"ids must hold {n} entries")
            opts.id_rank = self.id_rank.ctypes.data_as(C.POINTER(C.c_int64))
        _lib.call("eoship_tq_bind_corpus_opts", rt.handle, C.byref(desc),
                  codes.ctypes.data_as(C.c_void_p), norms.ctypes.data_as(C.c_void_p), C.c_int64(n),
                  C.byref(opts), C.byref(self.handle))
        del keep

    def share(self, rt: Runtime) -> "TurboQuantIndex":
        """A handle on the same resident corpus for another runtime (stream)
        of the device, with its own scratch: batches on the two runtimes may
        run concurrently."""
        h = C.c_void_p()
        _lib.call("eoship_tq_share", rt.handle, self.handle, C.byref(h))
        other = TurboQuantIndex.__new__(TurboQuantIndex)
        other.rt, other.n, other.dim, other.bits, other.handle = rt, self.n, self.dim, self.bits, h
        other.id_rank = self.id_rank
        return other

    def release(self) -> None:
        # After the runtime is closed the object cannot be released any more
        # (its stream is gone); the handle is only dropped.
        if self.handle and self.rt.handle:
            _lib.call("eoship_tq_release", self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def encode(self, vectors: np.ndarray):
        """Quantizes rows of vectors [n, dim] on the device with this index's
        rotation, codebook and bits: (codes uint8 [n, row_bytes], norms f32 [n]),
        ready to bind as a TurboQuantIndex corpus (the corpus-side Quantize of
        runtime/retrieval_turboquant.go:700,708). An index bound with no vectors
        serves as a pure quantizer."""
        x = np.ascontiguousarray(vectors, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != self.dim:
            raise ValueError(f"vectors must be [n, {self.dim}]")
        row_bytes = (self.dim * self.bits + 7) // 8
        codes = np.zeros((x.shape[0], row_bytes), np.uint8)
        norms = np.zeros(x.shape[0], np.float32)
        _lib.call("eoship_tq_encode", self.rt.handle, self.handle, x.ctypes.data_as(C.c_void_p),
                  C.c_int64(x.shape[0]), codes.ctypes.data_as(C.c_void_p),
                  norms.ctypes.data_as(C.c_void_p))
        return codes, norms

    def encode_device(self, d_x: DeviceBuffer, n: int, d_codes: DeviceBuffer,
                      d_norms: DeviceBuffer) -> None:
        """Enqueues encode on device buffers (x f32 [n, dim] -> codes
        [n, row_bytes], norms f32 [n]); no wait."""
        _lib.call("eoship_tq_encode_device", self.rt.handle, self.handle, d_x.ptr, C.c_int64(n),
                  d_codes.ptr, d_norms.ptr)

    def _queries(self, queries: np.ndarray) -> np.ndarray:
        q = np.ascontiguousarray(queries, dtype=np.float32)
        if q.ndim == 1:
            q = q[None, :]
        if q.ndim != 2 or q.shape[1] != self.dim:
            raise ValueError(f"queries must be [Q, {self.dim}]")
        return q

    def effective_k(self, top_k: int) -> int:
        return self.n if (top_k <= 0 or top_k > self.n) else int(top_k)

    def top_k(self, queries: np.ndarray, top_k: int):
        """Returns (ids int64 [Q, kk], scores float32 [Q, kk], stats)."""
        q = self._queries(queries)
        kk = self.effective_k(top_k)
        ids = np.zeros((q.shape[0], kk), np.int64)
        scores = np.zeros((q.shape[0], kk), np.float32)
        st = _lib.EosHipTQStats()
        _lib.call("eoship_tq_topk", self.rt.handle, self.handle, q.ctypes.data_as(C.c_void_p),
                  C.c_int32(q.shape[0]), C.c_int32(int(top_k)), ids.ctypes.data_as(C.c_void_p),
                  scores.ctypes.data_as(C.c_void_p), C.byref(st))
        stats = TurboQuantRetrievalScoreStats(
            candidate_count=st.candidate_count, candidates_scored=st.candidate_count,
            candidates_kept=st.candidates_kept, fallback_queries=st.fallback_queries,
            batches=st.batches)
        return ids, scores, stats

    def top_k_device(self, d_queries: DeviceBuffer, nq: int, top_k: int, d_ids: DeviceBuffer,
                     d_scores: DeviceBuffer, with_stats: bool = True):
        """Enqueue a top-k on device buffers. Without stats the call does not
        wait for the device; results are complete after Runtime.sync()."""
        st = _lib.EosHipTQStats() if with_stats else None
        _lib.call("eoship_tq_topk_device", self.rt.handle, self.handle, d_queries.ptr,
                  C.c_int32(nq), C.c_int32(int(top_k)), d_ids.ptr, d_scores.ptr,
                  C.byref(st) if st is not None else None)
        return st

    def top_k_device_deferred(self, d_queries: DeviceBuffer, nq: int, top_k: int,
                              d_ids: DeviceBuffer, d_scores: DeviceBuffer,
                              d_status: DeviceBuffer) -> None:
        """Enqueue a top-k without the exhaustive fallback: int32 d_status[nq]
        receives 0 for final rows, nonzero for rows repair_device must redo."""
        _lib.call("eoship_tq_topk_device_deferred", self.rt.handle, self.handle, d_queries.ptr,
                  C.c_int32(nq), C.c_int32(int(top_k)), d_ids.ptr, d_scores.ptr, d_status.ptr)

    def repair_device(self, d_queries: DeviceBuffer, nq: int, top_k: int, d_ids: DeviceBuffer,
                      d_scores: DeviceBuffer, d_status: DeviceBuffer) -> None:
        """Exhaustively recompute the rows a deferred top-k flagged."""
        _lib.call("eoship_tq_topk_repair_device", self.rt.handle, self.handle, d_queries.ptr,
                  C.c_int32(nq), C.c_int32(int(top_k)), d_ids.ptr, d_scores.ptr, d_status.ptr)

    def inner_product_prepared(self, queries: np.ndarray, begin: int = 0, count: int | None = None):
        """Exhaustive (dots int32 [Q, count], scores float32 [Q, count]) for vectors [begin, begin+count)."""
        q = self._queries(queries)
        count = self.n - begin if count is None else int(count)
        dots = np.zeros((q.shape[0], count), np.int32)
        scores = np.zeros((q.shape[0], count), np.float32)
        _lib.call("eoship_tq_scores", self.rt.handle, self.handle, q.ctypes.data_as(C.c_void_p),
                  C.c_int32(q.shape[0]), C.c_int64(begin), C.c_int64(count),
                  dots.ctypes.data_as(C.c_void_p), scores.ctypes.data_as(C.c_void_p))
        return dots, scores

    def prepare_query(self, queries: np.ndarray):
        """Device PrepareQuery: (int16 [Q, dim] rotated-rounded query, float32 [Q] alpha)."""
        q = self._queries(queries)
        qs = np.zeros((q.shape[0], self.dim), np.int16)
        alpha = np.zeros(q.shape[0], np.float32)
        _lib.call("eoship_tq_prepare", self.rt.handle, self.handle, q.ctypes.data_as(C.c_void_p),
                  C.c_int32(q.shape[0]), qs.ctypes.data_as(C.c_void_p),
                  alpha.ctypes.data_as(C.c_void_p))
        return qs, alpha


class TurboQuantMultiVectorIndex:
    """A bound corpus viewed as documents of doc_len consecutive vectors
    (the multivector children of runtime/retrieval_multivector_turboquant.go:
    546-605), scored by MaxSim: sum over query tokens of the best child score."""

    def __init__(self, index: TurboQuantIndex, doc_len: int):
        if doc_len <= 0 or doc_len % 32 or index.n % doc_len:
            raise ValueError("doc_len must be a multiple of 32 dividing the corpus size")
        self.index, self.doc_len = index, doc_len
        self.ndocs = index.n // doc_len

    def _queries(self, queries: np.ndarray) -> np.ndarray:
        q = np.ascontiguousarray(queries, dtype=np.float32)
        if q.ndim == 2:
            q = q[:, None, :]
        if q.ndim != 3 or q.shape[2] != self.index.dim or not 1 <= q.shape[1] <= 32:
            raise ValueError(f"queries must be [Q, tokens<=32, {self.index.dim}]")
        return q

    def top_k(self, queries: np.ndarray, top_k: int):
        q = self._queries(queries)
        kk = self.ndocs if (top_k <= 0 or top_k > self.ndocs) else int(top_k)
        ids = np.zeros((q.shape[0], kk), np.int64)
        scores = np.zeros((q.shape[0], kk), np.float32)
        _lib.call("eoship_tq_maxsim_topk", self.index.rt.handle, self.index.handle,
                  C.c_int32(self.doc_len), q.ctypes.data_as(C.c_void_p), C.c_int32(q.shape[0]),
                  C.c_int32(q.shape[1]), C.c_int32(int(top_k)), ids.ctypes.data_as(C.c_void_p),
                  scores.ctypes.data_as(C.c_void_p))
        return ids, scores

    def top_k_device(self, d_queries: DeviceBuffer, nq: int, tokens: int, top_k: int,
                     d_ids: DeviceBuffer, d_scores: DeviceBuffer) -> None:
        _lib.call("eoship_tq_maxsim_topk_device", self.index.rt.handle, self.index.handle,
                  C.c_int32(self.doc_len), d_queries.ptr, C.c_int32(nq), C.c_int32(tokens),
                  C.c_int32(int(top_k)), d_ids.ptr, d_scores.ptr)

    def scores(self, queries: np.ndarray, doc_begin: int = 0, doc_count: int | None = None):
        q = self._queries(queries)
        doc_count = self.ndocs - doc_begin if doc_count is None else int(doc_count)
        out = np.zeros((q.shape[0], doc_count), np.float32)
        _lib.call("eoship_tq_maxsim_scores", self.index.rt.handle, self.index.handle,
                  C.c_int32(self.doc_len), q.ctypes.data_as(C.c_void_p), C.c_int32(q.shape[0]),
                  C.c_int32(q.shape[1]), C.c_int64(doc_begin), C.c_int64(doc_count),
                  out.ctypes.data_as(C.c_void_p))
        return out


_AGGREGATION_TOP_N = {"max": 1, "top2-mean": 2, "top3-mean": 3, "top5-mean": 5}


@dataclass
class ParentScoredDoc:
    """A ranked parent with its best child (retrievalScoredDoc's ID, Score,
    ChildID and ChildScore, runtime/retrieval_multivector_turboquant.go:
    800-806); ids are integer parent and corpus-vector indices."""
    id: int
    score: float
    child_id: int
    child_score: float


class TurboQuantParents:
    """Children grouped by parent over a bound corpus: parent p owns vectors
    [offsets[p], offsets[p+1]). ``top_k`` is topTurboQuantMultiVectorParentScores
    (runtime/retrieval_multivector_turboquant.go:746-758) for each query vector,
    with aggregation "max" | "top2-mean" | "top3-mean" | "top5-mean" and a
    non-negative child_count_penalty (validated as :826-837 does)."""

    def __init__(self, index: TurboQuantIndex, offsets: np.ndarray):
        off = np.ascontiguousarray(offsets, dtype=np.int64)
        if off.ndim != 1 or off.shape[0] < 2:
            raise ValueError("offsets must be [nparents + 1]")
        self.index, self.offsets = index, off
        self.nparents = off.shape[0] - 1
        self.live = int(np.sum(off[1:] > off[:-1]))
        self.handle = C.c_void_p()
        _lib.call("eoship_tq_parents_bind", index.rt.handle, index.handle,
                  off.ctypes.data_as(C.c_void_p), C.c_int64(self.nparents), C.byref(self.handle))

    def release(self) -> None:
        # After the runtime is closed the object cannot be released any more
        # (its stream is gone); the handle is only dropped.
        if self.handle and self.index.rt.handle:
            _lib.call("eoship_tq_parents_release", self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    @staticmethod
    def _top_n(aggregation: str) -> int:
        if aggregation not in _AGGREGATION_TOP_N:
            raise ValueError("aggregation must be one of max, top2-mean, top3-mean, top5-mean")
        return _AGGREGATION_TOP_N[aggregation]

    def top_k(self, queries: np.ndarray, top_k: int, aggregation: str = "max",
              child_count_penalty: float = 0.0):
        """Returns (parent_ids, scores, best_child, best_child_score), each [Q, kk]."""
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.index.dim)
        kk = self.live if (top_k <= 0 or top_k > self.live) else int(top_k)
        ids = np.zeros((q.shape[0], kk), np.int64)
        sc = np.zeros((q.shape[0], kk), np.float32)
        bc = np.zeros((q.shape[0], kk), np.int64)
        bs = np.zeros((q.shape[0], kk), np.float32)
        _lib.call("eoship_tq_parent_topk", self.index.rt.handle, self.handle,
                  q.ctypes.data_as(C.c_void_p), C.c_int32(q.shape[0]), C.c_int32(int(top_k)),
                  C.c_int32(self._top_n(aggregation)), C.c_double(child_count_penalty),
                  ids.ctypes.data_as(C.c_void_p), sc.ctypes.data_as(C.c_void_p),
                  bc.ctypes.data_as(C.c_void_p), bs.ctypes.data_as(C.c_void_p))
        return ids, sc, bc, bs

    def top_k_device(self, d_queries: DeviceBuffer, nq: int, top_k: int, d_ids: DeviceBuffer,
                     d_scores: DeviceBuffer, d_best: DeviceBuffer, d_best_scores: DeviceBuffer,
                     aggregation: str = "max", child_count_penalty: float = 0.0) -> None:
        _lib.call("eoship_tq_parent_topk_device", self.index.rt.handle, self.handle, d_queries.ptr,
                  C.c_int32(nq), C.c_int32(int(top_k)), C.c_int32(self._top_n(aggregation)),
                  C.c_double(child_count_penalty), d_ids.ptr, d_scores.ptr, d_best.ptr,
                  d_best_scores.ptr)


def top_turboquant_multivector_parent_scores(parents: TurboQuantParents, query: np.ndarray,
                                             top_k: int, aggregation: str = "max",
                                             child_count_penalty: float = 0.0):
    """topTurboQuantMultiVectorParentScores for one query vector: the ranked
    [ParentScoredDoc] list."""
    ids, sc, bc, bs = parents.top_k(np.asarray(query)[None, :], top_k, aggregation,
                                    child_count_penalty)
    return [ParentScoredDoc(int(i), float(s), int(c), float(cs))
            for i, s, c, cs in zip(ids[0], sc[0], bc[0], bs[0])]


def top_turboquant_retrieval_scores_with_stats(index: TurboQuantIndex, queries: np.ndarray,
                                               top_k: int):
    """Per query, the ranked [RetrievalScoredDoc] list and the run's stats."""
    ids, scores, stats = index.top_k(queries, top_k)
    out = [[RetrievalScoredDoc(int(i), float(s)) for i, s in zip(ids[r], scores[r])]
           for r in range(ids.shape[0])]
    return out, stats


class F16Sidecar:
    """f16 rerank rows on the device: the counterpart of halfByID in
    computeTurboQuantFP16RerankRetrievalQuality (runtime/retrieval_turboquant.go:1503-1511),
    each f32 converted by float32ToHalf (runtime/mll_export.go:1007-1041) in a
    gfx950 kernel. vectors: float32 [n, dim]; row i is the document with id i."""

    def __init__(self, rt: Runtime, vectors: np.ndarray):
        v = np.ascontiguousarray(vectors, np.float32)
        if v.ndim != 2:
            raise ValueError("sidecar vectors must be [n, dim]")
        self.rt, self.n, self.dim = rt, int(v.shape[0]), int(v.shape[1])
        self.buf = DeviceBuffer(rt, max(2, v.size * 2))
        src = DeviceBuffer.from_array(rt, v) if v.size else None
        if src is not None:
            _lib.call("eoship_f16_sidecar_device", rt.handle, src.ptr, C.c_int64(v.size),
                      self.buf.ptr)
            src.free()

    @classmethod
    def allocate(cls, rt: Runtime, n: int, dim: int) -> "F16Sidecar":
        """An n x dim sidecar whose rows are filled later with fill_device."""
        obj = cls.__new__(cls)
        obj.rt, obj.n, obj.dim = rt, int(n), int(dim)
        obj.buf = DeviceBuffer(rt, max(2, obj.n * obj.dim * 2))
        return obj

    def fill_device(self, d_x: DeviceBuffer, row0: int, rows: int) -> None:
        """Rows [row0, row0 + rows) from f32 vectors already on the device."""
        if row0 < 0 or rows < 0 or row0 + rows > self.n:
            raise ValueError("rows outside the sidecar")
        if rows:
            _lib.call("eoship_f16_sidecar_device", self.rt.handle, d_x.ptr,
                      C.c_int64(rows * self.dim),
                      self.buf.view(row0 * self.dim * 2, rows * self.dim * 2).ptr)

    def halves(self) -> np.ndarray:
        return self.buf.download(np.uint16, (self.n, self.dim))


def top_fp16_rerank_scores_device(sidecar: F16Sidecar, d_queries: DeviceBuffer, nq: int,
                                  d_cand_ids: DeviceBuffer, d_cand_scores: DeviceBuffer, c: int,
                                  top_k: int, bit_width: int, overfetch: int,
                                  d_ids: DeviceBuffer, d_scores: DeviceBuffer,
                                  d_id_rank: DeviceBuffer | None = None,
                                  noalloc: bool = False) -> int:
    """topFP16RerankScores / topFP16RerankRescueScores for nq queries on device
    buffers (runtime/retrieval_turboquant.go:1551-1556, :1635-1786). c is the
    first stage's output width, min(overfetch, n). d_id_rank (int64 [n], the
    string-ID order) breaks equal scores by string ID. noalloc selects the entry
    point that allocates no device memory (nq * c <= 2^20). Returns kk."""
    entry = "eoship_tq_fp16_rerank_device_noalloc" if noalloc else "eoship_tq_fp16_rerank_device"
    _lib.call(entry, sidecar.rt.handle, d_queries.ptr, C.c_int32(nq),
              C.c_int32(sidecar.dim), sidecar.buf.ptr, C.c_int64(sidecar.n), d_cand_ids.ptr,
              d_cand_scores.ptr, C.c_int32(c), C.c_int32(int(top_k)), C.c_int32(int(bit_width)),
              C.c_int32(int(overfetch)), d_id_rank.ptr if d_id_rank is not None else None,
              d_ids.ptr, d_scores.ptr)
    return c if (top_k <= 0 or top_k > c) else int(top_k)


def turboquant_fp16_rerank_top_k(index, sidecar: F16Sidecar, queries: np.ndarray, top_k: int,
                                 overfetch: int, bit_width: int | None = None):
    """Two-stage retrieval per query as computeTurboQuantFP16RerankRetrievalQuality
    runs it (runtime/retrieval_turboquant.go:1512-1556): top_k < 100 -> 100,
    overfetch < top_k -> top_k, TurboQuant top-overfetch candidates, then the f16
    rerank (with the rank-100 rescue for the b4 / overfetch 200 / top 100
    profile). index: an IPIndex (the reference's IPQuantized first stage; the
    rescue gate gets its bit width, MSE bits + 1, as the reference passes the
    IP quantizer's bitWidth) or a TurboQuantIndex over the MSE-stage layout,
    for which bit_width must be given. Returns (ids int64 [Q, kk], scores
    float32 [Q, kk], candidate ids [Q, c])."""
    top_k = max(int(top_k), 100)
    overfetch = max(int(overfetch), top_k)
    is_ip = isinstance(index, IPIndex)
    dim = index.qz.dim if is_ip else index.dim
    if bit_width is None:
        if not is_ip:
            raise ValueError("bit_width is required for an MSE-layout index")
        bit_width = index.qz.bits + 1
    if sidecar.n != index.n or sidecar.dim != dim:
        raise ValueError("sidecar rows must match the bound corpus")
    q = np.ascontiguousarray(queries, np.float32).reshape(-1, dim) if is_ip else index._queries(queries)
    nq = q.shape[0]
    c = index.effective_k(overfetch)
    rt = index.rt
    d_q = DeviceBuffer.from_array(rt, q)
    d_cid = DeviceBuffer(rt, max(8, nq * c * 8))
    d_cs = DeviceBuffer(rt, max(4, nq * c * 4))
    index.top_k_device(d_q, nq, overfetch, d_cid, d_cs)
    kk = c if top_k > c else top_k
    d_ids = DeviceBuffer(rt, max(8, nq * kk * 8))
    d_sc = DeviceBuffer(rt, max(4, nq * kk * 4))
    rank = None if is_ip else index.id_rank
    d_rank = DeviceBuffer.from_array(rt, rank) if rank is not None else None
    top_fp16_rerank_scores_device(sidecar, d_q, nq, d_cid, d_cs, c, top_k, bit_width, overfetch,
                                  d_ids, d_sc, d_rank)
    ids = d_ids.download(np.int64, (nq, kk))
    scores = d_sc.download(np.float32, (nq, kk))
    cand = d_cid.download(np.int64, (nq, c))
    for b in (d_q, d_cid, d_cs, d_ids, d_sc) + ((d_rank,) if d_rank is not None else ()):
        b.free()
    return ids, scores, cand


def _rerank_out(rt, nq, c, top_k):
    kk = c if (top_k <= 0 or top_k > c) else int(top_k)
    return kk, DeviceBuffer(rt, max(8, nq * kk * 8)), DeviceBuffer(rt, max(4, nq * kk * 4))


def dense_rerank_top_k(rt: Runtime, queries: np.ndarray, rows: np.ndarray,
                       cand_ids: np.ndarray, top_k: int, id_rank: np.ndarray | None = None):
    """topDenseRerankScores (runtime/retrieval_turboquant.go:1610-1633) for each
    query over f32 corpus rows [n, d]: (ids int64 [Q, kk], scores float32)."""
    q = np.ascontiguousarray(queries, np.float32)
    cid = np.ascontiguousarray(cand_ids, np.int64)
    nq, c = cid.shape
    rows = np.ascontiguousarray(rows, np.float32)
    bufs = [DeviceBuffer.from_array(rt, q), DeviceBuffer.from_array(rt, rows),
            DeviceBuffer.from_array(rt, cid)]
    rank = DeviceBuffer.from_array(rt, np.ascontiguousarray(id_rank, np.int64)) \
        if id_rank is not None else None
    kk, d_ids, d_sc = _rerank_out(rt, nq, c, top_k)
    try:
        _lib.call("eoship_tq_dense_rerank_device", rt.handle, bufs[0].ptr, C.c_int32(nq),
                  C.c_int32(q.shape[1]), bufs[1].ptr, C.c_int64(rows.shape[0]), bufs[2].ptr,
                  C.c_int32(c), C.c_int32(int(top_k)), rank.ptr if rank is not None else None,
                  d_ids.ptr, d_sc.ptr)
        return d_ids.download(np.int64, (nq, kk)), d_sc.download(np.float32, (nq, kk))
    finally:
        for b in bufs + [d_ids, d_sc] + ([rank] if rank is not None else []):
            b.free()


def reconstruct_rerank_top_k(rt: Runtime, queries: np.ndarray, codes: np.ndarray, bits: int,
                             norms: np.ndarray, codebook: np.ndarray, rotation: np.ndarray | None,
                             cand_ids: np.ndarray, top_k: int,
                             id_rank: np.ndarray | None = None, signs: np.ndarray | None = None,
                             resnorms: np.ndarray | None = None, sketch: np.ndarray | None = None):
    """Reconstruct rerank over a code set in the reference row layout (the
    primary codes: topTurboQuantReconstructRerankScores; a wider sidecar set:
    topTurboQuantMixedWidthRerankScores, runtime/retrieval_turboquant.go:
    1788-1846): each candidate dequantized (with the QJL term when signs,
    resnorms and the sketch S [d, d] are given: an inner-product set), then
    the f32 index-order dot. rotation is R [d, d] (None: identity), codebook
    the f32 centroids [2^bits]. Returns (ids int64 [Q, kk], scores float32)."""
    q = np.ascontiguousarray(queries, np.float32)
    cid = np.ascontiguousarray(cand_ids, np.int64)
    nq, c = cid.shape
    d = q.shape[1]
    codes = np.ascontiguousarray(codes, np.uint8)
    norms = np.ascontiguousarray(norms, np.float32)
    cb = np.ascontiguousarray(codebook, np.float32)
    if cb.shape != (1 << bits,):
        raise ValueError(f"codebook must hold 2^{bits} values")
    bufs = [DeviceBuffer.from_array(rt, q), DeviceBuffer.from_array(rt, codes),
            DeviceBuffer.from_array(rt, norms), DeviceBuffer.from_array(rt, cb),
            DeviceBuffer.from_array(rt, cid)]
    rot = None
    if rotation is not None:
        rot = DeviceBuffer.from_array(rt, np.ascontiguousarray(np.asarray(rotation, np.float32).T))
        bufs.append(rot)
    rank = None
    if id_rank is not None:
        rank = DeviceBuffer.from_array(rt, np.ascontiguousarray(id_rank, np.int64))
        bufs.append(rank)
    ipb = [None, None, None]
    if signs is not None:
        ipb = [DeviceBuffer.from_array(rt, np.ascontiguousarray(signs, np.uint8)),
               DeviceBuffer.from_array(rt, np.ascontiguousarray(resnorms, np.float32)),
               DeviceBuffer.from_array(rt, np.ascontiguousarray(np.asarray(sketch, np.float32).T))]
        bufs += ipb
    spec = _lib.EosHipTQCodes(bits=bits, dim=d, n=norms.shape[0], codes=bufs[1].ptr.value,
                              norms=bufs[2].ptr.value, codebook=bufs[3].ptr.value,
                              rotation_t=rot.ptr.value if rot is not None else None,
                              signs=ipb[0].ptr.value if ipb[0] is not None else None,
                              resnorms=ipb[1].ptr.value if ipb[1] is not None else None,
                              qjl_t=ipb[2].ptr.value if ipb[2] is not None else None)
    kk, d_ids, d_sc = _rerank_out(rt, nq, c, top_k)
    try:
        _lib.call("eoship_tq_reconstruct_rerank_device", rt.handle, C.byref(spec), bufs[0].ptr,
                  C.c_int32(nq), bufs[4].ptr, C.c_int32(c), C.c_int32(int(top_k)),
                  rank.ptr if rank is not None else None, d_ids.ptr, d_sc.ptr)
        return d_ids.download(np.int64, (nq, kk)), d_sc.download(np.float32, (nq, kk))
    finally:
        for b in bufs + [d_ids, d_sc]:
            b.free()


class IPQuantizer:
    """The inner-product layout (MSE codes + QJL signs + ResNorm + Norm) on
    the device: ``encode`` (eoship_tq_ip_encode_device) and exhaustive
    ``scores`` / top-k (eoship_tq_ip_scores_device). rotation R and sketch S
    are [d, d] f32; codebook the int8 grid with its scale."""

    def __init__(self, rt: Runtime, dim: int, bits: int, codebook: np.ndarray,
                 codebook_scale: float, rotation: np.ndarray | None, sketch: np.ndarray):
        self.rt, self.dim, self.bits = rt, int(dim), int(bits)
        self._cb = np.ascontiguousarray(codebook, np.int8)
        if self._cb.shape != (1 << self.bits,):
            raise ValueError("codebook must hold 2^bits entries")
        self._rot = None
        if rotation is not None:
            self._rot = DeviceBuffer.from_array(rt, np.ascontiguousarray(
                np.asarray(rotation, np.float32).T))
        self._qjl = DeviceBuffer.from_array(rt, np.ascontiguousarray(np.asarray(sketch, np.float32).T))
        self.spec = _lib.EosHipTQIPSpec(self.dim, self.bits, float(codebook_scale),
                                        self._cb.ctypes.data_as(C.c_void_p).value,
                                        self._rot.ptr.value if self._rot is not None else None,
                                        self._qjl.ptr.value)
        self.row_bytes = (self.dim * self.bits + 7) // 8
        self.sign_bytes = (self.dim + 7) // 8

    def vector_bytes(self) -> int:
        """MSE + signs + 8 bytes per vector (runtime/turboquant_bytes.go:14-25)."""
        return self.row_bytes + self.sign_bytes + 8

    def encode(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.dim)
        n = x.shape[0]
        bufs = [DeviceBuffer.from_array(self.rt, x), DeviceBuffer(self.rt, max(1, n * self.row_bytes)),
                DeviceBuffer(self.rt, max(1, n * self.sign_bytes)), DeviceBuffer(self.rt, max(4, n * 4)),
                DeviceBuffer(self.rt, max(4, n * 4))]
        try:
            _lib.call("eoship_tq_ip_encode_device", self.rt.handle, C.byref(self.spec), bufs[0].ptr,
                      C.c_int64(n), bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, bufs[4].ptr)
            return (bufs[1].download(np.uint8, (n, self.row_bytes)),
                    bufs[2].download(np.uint8, (n, self.sign_bytes)),
                    bufs[3].download(np.float32, (n,)), bufs[4].download(np.float32, (n,)))
        finally:
            for b in bufs:
                b.free()

    def scores(self, queries, codes, signs, resnorms, norms, k: int = 0):
        """scores [q, n], and with k > 0 also (top ids [q, kk], top scores)."""
        q = np.ascontiguousarray(queries, np.float32).reshape(-1, self.dim)
        nq, n = q.shape[0], int(np.asarray(norms).shape[0])
        kk = min(k, n)
        ins = [DeviceBuffer.from_array(self.rt, a) for a in (
            q, np.ascontiguousarray(codes, np.uint8), np.ascontiguousarray(signs, np.uint8),
            np.ascontiguousarray(resnorms, np.float32), np.ascontiguousarray(norms, np.float32))]
        out = DeviceBuffer(self.rt, max(4, nq * n * 4))
        tid = DeviceBuffer(self.rt, max(8, nq * kk * 8)) if k > 0 else None
        tsc = DeviceBuffer(self.rt, max(4, nq * kk * 4)) if k > 0 else None
        try:
            _lib.call("eoship_tq_ip_scores_device", self.rt.handle, C.byref(self.spec), ins[0].ptr,
                      C.c_int32(nq), ins[1].ptr, ins[2].ptr, ins[3].ptr, ins[4].ptr, C.c_int64(n),
                      out.ptr, C.c_int32(k), tid.ptr if tid else None, tsc.ptr if tsc else None)
            s = out.download(np.float32, (nq, n))
            if k > 0:
                return s, tid.download(np.int64, (nq, kk)), tsc.download(np.float32, (nq, kk))
            return s
        finally:
            for b in ins + [out] + ([tid, tsc] if k > 0 else []):
                b.free()

    def bind(self, codes, signs, resnorms, norms, zero_vector_allowed=None) -> "IPIndex":
        """Binds an encoded corpus for top-k search (eoship_tq_ip_bind_corpus):
        host arrays or DeviceBuffers of codes [n, row_bytes], signs [n,
        sign_bytes], resnorms and norms [n]."""
        return IPIndex(self, codes, signs, resnorms, norms, zero_vector_allowed)

    def release(self) -> None:
        for b in (self._rot, self._qjl):
            if b is not None:
                b.free()
        self._rot = self._qjl = None


class IPIndex:
    """An inner-product corpus bound for top-k (the promoted profile's first
    stage): ``top_k_device`` on device queries, ``top_k`` on host arrays."""

    def __init__(self, quantizer: IPQuantizer, codes, signs, resnorms, norms,
                 zero_vector_allowed=None):
        self.qz, self.rt = quantizer, quantizer.rt
        tmp = []

        def dev(x, dtype):
            if isinstance(x, DeviceBuffer):
                return x
            b = DeviceBuffer.from_array(self.rt, np.ascontiguousarray(x, dtype))
            tmp.append(b)
            return b

        n = int(norms.nbytes // 4) if isinstance(norms, DeviceBuffer) else int(np.asarray(norms).shape[0])
        bufs = [dev(codes, np.uint8), dev(signs, np.uint8), dev(resnorms, np.float32),
                dev(norms, np.float32)]
        zv = None
        opts = None
        if zero_vector_allowed is not None:
            zv = np.ascontiguousarray(zero_vector_allowed, np.uint8)
            opts = _lib.EosHipTQBindOptions(zero_vector_allowed=zv.ctypes.data_as(C.POINTER(C.c_uint8)),
                                            id_rank=None)
        self.handle = C.c_void_p()
        try:
            _lib.call("eoship_tq_ip_bind_corpus", self.rt.handle, C.byref(quantizer.spec),
                      bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, C.c_int64(n),
                      C.byref(opts) if opts is not None else None, C.byref(self.handle))
        finally:
            for b in tmp:
                b.free()
        self.n = n

    def effective_k(self, k: int) -> int:
        return self.n if (k <= 0 or k > self.n) else k

    def top_k_device(self, d_queries: DeviceBuffer, nq: int, k: int, d_ids: DeviceBuffer,
                     d_scores: DeviceBuffer) -> None:
        _lib.call("eoship_tq_ip_topk_device", self.rt.handle, self.handle, d_queries.ptr,
                  C.c_int32(nq), C.c_int32(int(k)), d_ids.ptr, d_scores.ptr)

    def top_k(self, queries: np.ndarray, k: int):
        q = np.ascontiguousarray(queries, np.float32).reshape(-1, self.qz.dim)
        nq, kk = q.shape[0], self.effective_k(k)
        dq = DeviceBuffer.from_array(self.rt, q)
        di, ds = DeviceBuffer(self.rt, max(8, nq * kk * 8)), DeviceBuffer(self.rt, max(4, nq * kk * 4))
        try:
            self.top_k_device(dq, nq, k, di, ds)
            return di.download(np.int64, (nq, kk)), ds.download(np.float32, (nq, kk))
        finally:
            for b in (dq, di, ds):
                b.free()

    def release(self) -> None:
        if self.handle and self.rt.handle:
            _lib.call("eoship_tq_ip_release", self.handle)
        self.handle = C.c_void_p()
