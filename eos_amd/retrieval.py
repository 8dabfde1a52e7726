"""Host side of the retrieval plans (libeoship): a dot / cosine /
l2_distance score step, topk and the gathers of candidate ids, scores and
document rows (runtime/retrieval.go:51-112; examples/retrieve.eos,
candidates.eos, packed_candidates.eos, batch_candidates.eos).

``score_topk`` runs the fused path on host arrays; ``MllRetrieval`` binds a
retrieval entry of an MLL package (``eoship_retrieval_bind_mll``) and returns
the entry's outputs by name."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, Runtime

OPS = {"dot": 1, "cosine": 2, "l2_distance": 3}
OUT_NAMES = {1: "scores", 2: "top_index", 3: "top_ids", 4: "top_scores", 5: "top_docs",
             6: "pack"}


def _run(rt: Runtime, fn, k: int, q: int, n: int, d: int, want_docs: bool, call_args):
    """Allocate outputs, call fn(*call_args, scores, index, ids, top_scores,
    top_docs) and download them."""
    bufs = {"scores": DeviceBuffer(rt, max(1, q * n * 4))}
    if k > 0:
        bufs["top_index"] = DeviceBuffer(rt, q * k * 4)
        bufs["top_ids"] = DeviceBuffer(rt, q * k * 8)
        bufs["top_scores"] = DeviceBuffer(rt, q * k * 4)
        if want_docs:
            bufs["top_docs"] = DeviceBuffer(rt, q * k * d * 4)
    ptr = lambda name: bufs[name].ptr if name in bufs else None
    _lib.call(fn, *call_args, ptr("scores"), ptr("top_index"), ptr("top_ids"),
              ptr("top_scores"), ptr("top_docs"))
    out = {"scores": bufs["scores"].download(np.float32, (q, n))}
    if k > 0:
        out["top_index"] = bufs["top_index"].download(np.int32, (q, k))
        out["top_ids"] = bufs["top_ids"].download(np.int64, (q, k))
        out["top_scores"] = bufs["top_scores"].download(np.float32, (q, k))
        if want_docs:
            out["top_docs"] = bufs["top_docs"].download(np.float32, (q, k, d))
    for b in bufs.values():
        b.free()
    return out


def score_topk(rt: Runtime, op: str, queries: np.ndarray, docs: np.ndarray, k: int = 0,
               candidate_ids: np.ndarray | None = None, batched: bool = False,
               q4_scale: float | None = None, q4_shape: tuple | None = None) -> dict:
    """Scores [Q, N] and (k > 0) top_index, top_ids, top_scores, top_docs.
    docs: f32 [N, D] (batched: [Q, N, D]), or packed q4 bytes with q4_scale
    and q4_shape."""
    qs = np.ascontiguousarray(np.atleast_2d(queries), np.float32)
    q, d = qs.shape
    if q4_scale is None:
        x = np.ascontiguousarray(docs, np.float32)
        n = x.shape[-2]
        spec = _lib.EosHipScoreSpec(op=OPS[op], k=k, docs_q4=0, docs_scale=0.0,
                                    batched=int(batched))
    else:
        x = np.ascontiguousarray(np.frombuffer(bytes(docs), np.uint8))
        n = q4_shape[-2]
        spec = _lib.EosHipScoreSpec(op=OPS[op], k=k, docs_q4=1, docs_scale=float(q4_scale),
                                    batched=int(batched))
    dq = DeviceBuffer.from_array(rt, qs)
    dx = DeviceBuffer.from_array(rt, x)
    di = None
    if candidate_ids is not None:
        di = DeviceBuffer.from_array(rt, np.ascontiguousarray(candidate_ids, np.int64))
    try:
        return _run(rt, "eoship_score_topk_device", k, q, n, d, True,
                    (rt.handle, C.byref(spec), dq.ptr, C.c_int32(q), C.c_int32(d), dx.ptr,
                     C.c_int64(n), di.ptr if di is not None else None))
    finally:
        dq.free()
        dx.free()
        if di is not None:
            di.free()


def plan_dict(p) -> dict:
    return {
        "op": {1: "dot", 2: "cosine", 3: "l2_distance"}[p.op], "k": p.k,
        "batched": bool(p.batched), "docs_param": bool(p.docs_param),
        "has_candidate_ids": bool(p.has_candidate_ids), "docs_q4": bool(p.docs_q4),
        "docs_rows": p.docs_rows, "dim": p.dim,
        "outputs": [OUT_NAMES[p.outputs[i]] for i in range(p.n_outputs)], "steps": p.steps,
        "entry": p.entry.decode(), "query_input": p.query_input.decode(),
        "docs_input": p.docs_input.decode(), "ids_input": p.ids_input.decode(),
    }


class MllRetrieval:
    """A retrieval entry of an MLL package bound on the device. ``run``
    returns the entry's return values in order (pack_candidates as the
    (ids, scores, docs) triple)."""

    def __init__(self, rt: Runtime, pkg, entry: str | None = None):
        self.rt = rt
        self.handle = C.c_void_p()
        plan = _lib.EosHipRetrievalPlan()
        _lib.call("eoship_retrieval_bind_mll", rt.handle, pkg.handle,
                  entry.encode() if entry else None, C.byref(self.handle), C.byref(plan))
        self.plan = plan_dict(plan)

    def release(self) -> None:
        if self.handle and self.rt.handle:
            _lib.call("eoship_retrieval_release", self.rt.handle, self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def run(self, queries: np.ndarray, docs: np.ndarray | None = None,
            candidate_ids: np.ndarray | None = None) -> list:
        p = self.plan
        qs = np.ascontiguousarray(np.atleast_2d(queries), np.float32)
        q, d = qs.shape
        dx = di = None
        if p["docs_param"]:
            n = p["docs_rows"]
        else:
            x = np.ascontiguousarray(docs, np.float32)
            n = x.shape[-2]
            dx = DeviceBuffer.from_array(self.rt, x)
        if candidate_ids is not None:
            di = DeviceBuffer.from_array(self.rt, np.ascontiguousarray(candidate_ids, np.int64))
        dq = DeviceBuffer.from_array(self.rt, qs)
        try:
            res = _run(self.rt, "eoship_retrieval_run_device", p["k"], q, n, d, True,
                       (self.rt.handle, self.handle, dq.ptr, C.c_int32(q), C.c_int32(d),
                        dx.ptr if dx is not None else None, C.c_int64(n),
                        di.ptr if di is not None else None))
        finally:
            for b in (dq, dx, di):
                if b is not None:
                    b.free()
        single = np.asarray(queries).ndim == 1
        outs = []
        for name in p["outputs"]:
            if name == "pack":
                v = tuple(res[k][0] if single else res[k]
                          for k in ("top_ids", "top_scores", "top_docs"))
            else:
                v = res[name][0] if single else res[name]
            outs.append(v)
        return outs
