"""TEST INFRASTRUCTURE ONLY: the CPU oracle (plain C restatement of the
reference's host path, see the headers of the C sources for the file:line each
function follows). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    P = C.c_void_p
    lib.tq_qmax.argtypes = [P, C.c_int, C.c_int]
    lib.tq_qmax.restype = C.c_int
    lib.tq_prepare.argtypes = [P, P, C.c_int, C.c_int, C.c_float, P, P]
    lib.tq_prepare.restype = None
    lib.tq_dots.argtypes = [P, C.c_int, P, C.c_int64, C.c_int, P, P]
    lib.tq_dots.restype = None
    lib.tq_scores.argtypes = [P, C.c_int, P, C.c_int, C.c_int, P, C.c_float, P, P, C.c_int64,
                              C.c_int64, P, P]
    lib.tq_scores.restype = None
    lib.tq_scores_f64.argtypes = [P, C.c_int, P, C.c_int, C.c_int, P, C.c_float, P, P, C.c_int64, P]
    lib.tq_scores_f64.restype = None
    lib.tq_topk.argtypes = [P, C.c_int, P, C.c_int, C.c_int, P, C.c_float, P, P, C.c_int64, C.c_int,
                            P, P]
    lib.tq_topk.restype = C.c_int64
    lib.topk_scores.argtypes = [P, C.c_int64, C.c_int, P, P]
    lib.topk_scores.restype = C.c_int64
    lib.tq_maxsim_scores.argtypes = [P, C.c_int, C.c_int, P, C.c_int, C.c_int, P, C.c_float, P, P,
                                     C.c_int64, C.c_int, P]
    lib.tq_maxsim_scores.restype = None
    lib.tq_parent_topk.argtypes = [P, C.c_int, P, C.c_int, C.c_int, P, C.c_float, P, P, P,
                                   C.c_int64, C.c_int, C.c_double, C.c_int, P, P, P, P]
    lib.tq_parent_topk.restype = C.c_int64
    lib.tq_encode.argtypes = [P, C.c_int64, P, C.c_int, C.c_int, P, C.c_float, P, P]
    lib.tq_encode.restype = None
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def tq_qmax(codebook: np.ndarray, dim: int) -> int:
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    return load().tq_qmax(_p(cb), int(cb.shape[0]), int(dim))


def tq_prepare(query: np.ndarray, rotation, codebook, codebook_scale: float):
    q = _f32(query)
    d = q.shape[0]
    rot = None if rotation is None else _f32(rotation)
    qs = np.zeros(d, np.int16)
    alpha = C.c_float()
    load().tq_prepare(_p(q), _p(rot), d, tq_qmax(codebook, d), C.c_float(codebook_scale), _p(qs),
                      C.byref(alpha))
    return qs, np.float32(alpha.value)


def tq_dots(qs: np.ndarray, codes: np.ndarray, bits: int, codebook: np.ndarray) -> np.ndarray:
    qs = np.ascontiguousarray(qs, dtype=np.int16)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    out = np.zeros(codes.shape[0], np.int32)
    load().tq_dots(_p(qs), qs.shape[0], _p(codes), codes.shape[0], bits, _p(cb), _p(out))
    return out


def tq_scores(queries, rotation, dim, bits, codebook, codebook_scale, codes, norms, begin=0,
              count=None):
    q = _f32(queries).reshape(-1, dim)
    rot = None if rotation is None else _f32(rotation)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    norms = _f32(norms)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    count = codes.shape[0] - begin if count is None else count
    dots = np.zeros((q.shape[0], count), np.int32)
    scores = np.zeros((q.shape[0], count), np.float32)
    load().tq_scores(_p(q), q.shape[0], _p(rot), dim, bits, _p(cb), C.c_float(codebook_scale),
                     _p(codes), _p(norms), begin, count, _p(dots), _p(scores))
    return dots, scores


def tq_scores_f64(queries, rotation, dim, bits, codebook, codebook_scale, codes, norms):
    q = _f32(queries).reshape(-1, dim)
    rot = None if rotation is None else _f32(rotation)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    norms = _f32(norms)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    out = np.zeros((q.shape[0], codes.shape[0]), np.float64)
    load().tq_scores_f64(_p(q), q.shape[0], _p(rot), dim, bits, _p(cb), C.c_float(codebook_scale),
                         _p(codes), _p(norms), codes.shape[0], _p(out))
    return out


def tq_topk(queries, rotation, dim, bits, codebook, codebook_scale, codes, norms, k):
    q = _f32(queries).reshape(-1, dim)
    rot = None if rotation is None else _f32(rotation)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    norms = _f32(norms)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    n = codes.shape[0]
    kk = n if (k <= 0 or k > n) else k
    ids = np.zeros((q.shape[0], kk), np.int64)
    scores = np.zeros((q.shape[0], kk), np.float32)
    load().tq_topk(_p(q), q.shape[0], _p(rot), dim, bits, _p(cb), C.c_float(codebook_scale),
                   _p(codes), _p(norms), n, int(k), _p(ids), _p(scores))
    return ids, scores


def topk_scores(scores: np.ndarray, k: int):
    s = _f32(scores)
    n = s.shape[0]
    kk = n if (k <= 0 or k > n) else k
    ids = np.zeros(kk, np.int64)
    out = np.zeros(kk, np.float32)
    load().topk_scores(_p(s), n, int(k), _p(ids), _p(out))
    return ids, out


SCORE_OPS = {"dot": 1, "cosine": 2, "l2_distance": 3}


def score_rows(op, query, docs) -> np.ndarray:
    """dotRows / cosineRows / l2DistanceRows of one query [D] against docs
    [N, D] (retrieval_oracle.c), f32 [N]."""
    lib = load()
    fn = lib.ret_score_rows
    fn.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_void_p]
    fn.restype = None
    q, x = _f32(query), _f32(docs)
    n, d = x.shape
    assert q.shape == (d,)
    out = np.zeros(n, np.float32)
    fn(SCORE_OPS[op] if isinstance(op, str) else int(op), _p(q), _p(x), n, d, _p(out))
    return out


def tq_maxsim_scores(queries, rotation, dim, bits, codebook, codebook_scale, codes, norms,
                     doc_len):
    """queries [Q, tokens, dim] -> doc scores [Q, ndocs]."""
    q = _f32(queries)
    if q.ndim == 2:
        q = q[:, None, :]
    rot = None if rotation is None else _f32(rotation)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    norms = _f32(norms)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    ndocs = codes.shape[0] // doc_len
    out = np.zeros((q.shape[0], ndocs), np.float32)
    load().tq_maxsim_scores(_p(q), q.shape[0], q.shape[1], _p(rot), dim, bits, _p(cb),
                            C.c_float(codebook_scale), _p(codes), _p(norms), ndocs, doc_len,
                            _p(out))
    return out


def tq_encode(vectors, rotation, dim, bits, codebook, codebook_scale):
    """Build-defined MSE-stage encoder: (codes uint8 [n, row_bytes], norms f32 [n])."""
    x = _f32(vectors).reshape(-1, dim)
    rot = None if rotation is None else _f32(rotation)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    row_bytes = (dim * bits + 7) // 8
    codes = np.zeros((x.shape[0], row_bytes), np.uint8)
    norms = np.zeros(x.shape[0], np.float32)
    load().tq_encode(_p(x), x.shape[0], _p(rot), dim, bits, _p(cb), C.c_float(codebook_scale),
                     _p(codes), _p(norms))
    return codes, norms


def tq_parent_topk(queries, rotation, dim, bits, codebook, codebook_scale, codes, norms,
                   offsets, k, top_n=1, penalty=0.0):
    """Parent (multivector child) aggregation top-k, one query vector each.
    offsets [nparents + 1] (parent p owns vectors [off[p], off[p+1])).
    Returns (ids, scores, best_child, best_child_score), each [Q, kk]."""
    q = _f32(queries).reshape(-1, dim)
    rot = None if rotation is None else _f32(rotation)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    norms = _f32(norms)
    cb = np.ascontiguousarray(codebook, dtype=np.int8)
    off = np.ascontiguousarray(offsets, dtype=np.int64)
    npar = off.shape[0] - 1
    live = int(np.sum(off[1:] > off[:-1]))
    kk = live if (k <= 0 or k > live) else k
    ids = np.zeros((q.shape[0], kk), np.int64)
    sc = np.zeros((q.shape[0], kk), np.float32)
    bc = np.zeros((q.shape[0], kk), np.int64)
    bs = np.zeros((q.shape[0], kk), np.float32)
    got = load().tq_parent_topk(_p(q), q.shape[0], _p(rot), dim, bits, _p(cb),
                                C.c_float(codebook_scale), _p(codes), _p(norms), _p(off), npar,
                                top_n, C.c_double(penalty), k, _p(ids), _p(sc), _p(bc), _p(bs))
    assert got == kk
    return ids, sc, bc, bs


# ------------------------------------------------------------------ encoder

def _enc():
    lib = load()
    if getattr(lib, "_enc_ready", False):
        return lib
    P = C.c_void_p
    lib.dense_hf.argtypes = [P, C.c_int, C.c_int, P, P, C.c_int, P]
    lib.dense_hf.restype = None
    lib.bert_attention.argtypes = [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]
    lib.bert_attention.restype = None
    lib.bert_embed.argtypes = [P, C.c_int, P, C.c_int, P, C.c_int, P, P, P, C.c_int, P, P, P,
                               C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, P]
    lib.bert_embed.restype = None
    lib.bert_embed_pool.argtypes = [P, C.c_int, P, C.c_int, P, C.c_int, P, P, P, C.c_int, P, P,
                                    P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double,
                                    C.c_int, P]
    lib.bert_embed_pool.restype = None
    lib.bert_hidden.argtypes = lib.bert_embed.argtypes
    lib.bert_hidden.restype = None
    lib.mean_pool_masked.argtypes = [P, P, C.c_int, C.c_int, C.c_int, P]
    lib.mean_pool_masked.restype = None
    lib.normalize_rows.argtypes = [P, C.c_int, C.c_int]
    lib.normalize_rows.restype = None
    lib.tiny_embed.argtypes = [P, C.c_int, C.c_int, P, C.c_int, P, C.c_int, P]
    lib.tiny_embed.restype = None
    lib.rope_rows.argtypes = [P, C.c_int, C.c_int, C.c_int]
    lib.rope_rows.restype = None
    lib.matmul_f32.argtypes = [P, C.c_int, C.c_int, P, C.c_int, P]
    lib.matmul_f32.restype = None
    lib.layer_norm_rows.argtypes = [P, C.c_int, C.c_int]
    lib.layer_norm_rows.restype = None
    lib.compact_single_head_attention.argtypes = [P, P, P, P, C.c_int, C.c_int, C.c_int, P]
    lib.compact_single_head_attention.restype = None
    lib.compact_embed.argtypes = [P, C.c_int, P, C.c_int, P, C.c_int, P, C.c_int, P, P, P,
                                  C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]
    lib.compact_embed.restype = None
    lib.compact_embed_opts.argtypes = [P, C.c_int, P, C.c_int, P, C.c_int, P, C.c_int, P, P, P,
                                       C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]
    lib.compact_embed_opts.restype = None
    lib.gelu_tanh_inplace.argtypes = [P, C.c_long]
    lib.gelu_tanh_inplace.restype = None
    lib._enc_ready = True
    return lib


def bert_embed(tok, pos, typ, emb_gamma, emb_beta, layers, ids, mask, type_ids, heads, eps,
               pooling: str = "masked_mean"):
    """layers: list of 16-tensor lists (reference order, f32, HF [out, in]).
    pooling: "masked_mean" or "cls" (bert_embedder_ops.go:179-196)."""
    lib = _enc()
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    types = np.zeros_like(ids) if type_ids is None else np.ascontiguousarray(type_ids, np.int32)
    batch, tokens = ids.shape
    hidden = tok.shape[1]
    inter = layers[0][10].shape[0] if layers else hidden
    keep = [_f32(x) for L in layers for x in L]
    ptrs = (C.c_void_p * max(len(keep), 1))(*[k.ctypes.data for k in keep])
    tok, pos, typ = _f32(tok), _f32(pos), _f32(typ)
    g, b = _f32(emb_gamma), _f32(emb_beta)
    out = np.zeros((batch, hidden), np.float32)
    mode = {"masked_mean": 0, "cls": 1}[pooling]
    lib.bert_embed_pool(_p(tok), tok.shape[0], _p(pos), pos.shape[0], _p(typ), typ.shape[0],
                        _p(g), _p(b), ptrs, len(layers), _p(ids), _p(types), _p(mask), batch,
                        tokens, hidden, heads, inter, C.c_double(eps), mode, _p(out))
    return out


def bert_hidden(tok, pos, typ, emb_gamma, emb_beta, layers, ids, mask, type_ids, heads, eps):
    """Hidden states [batch, tokens, hidden] after every layer (the state the
    pooling reads), every position computed."""
    lib = _enc()
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    types = np.zeros_like(ids) if type_ids is None else np.ascontiguousarray(type_ids, np.int32)
    batch, tokens = ids.shape
    hidden = tok.shape[1]
    inter = layers[0][10].shape[0] if layers else hidden
    keep = [_f32(x) for L in layers for x in L]
    ptrs = (C.c_void_p * max(len(keep), 1))(*[k.ctypes.data for k in keep])
    tok, pos, typ = _f32(tok), _f32(pos), _f32(typ)
    g, b = _f32(emb_gamma), _f32(emb_beta)
    h = np.zeros((batch, tokens, hidden), np.float32)
    lib.bert_hidden(_p(tok), tok.shape[0], _p(pos), pos.shape[0], _p(typ), typ.shape[0], _p(g),
                    _p(b), ptrs, len(layers), _p(ids), _p(types), _p(mask), batch, tokens, hidden,
                    heads, inter, C.c_double(eps), _p(h))
    return h


def dense_hf(x, w, b):
    lib = _enc()
    x, w, b = _f32(x), _f32(w), _f32(b)
    y = np.zeros((x.shape[0], w.shape[0]), np.float32)
    lib.dense_hf(_p(x), x.shape[0], x.shape[1], _p(w), _p(b), w.shape[0], _p(y))
    return y


def bert_attention(q, k, v, mask, heads):
    lib = _enc()
    q, k, v = _f32(q), _f32(k), _f32(v)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    batch, tokens = mask.shape
    ctx = np.zeros_like(q)
    lib.bert_attention(_p(q), _p(k), _p(v), _p(mask), batch, tokens, q.shape[1], heads, _p(ctx))
    return ctx


def mean_pool_masked(h, mask):
    lib = _enc()
    h = _f32(h)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    batch, tokens, hidden = h.shape
    out = np.zeros((batch, hidden), np.float32)
    lib.mean_pool_masked(_p(h), _p(mask), batch, tokens, hidden, _p(out))
    return out


def normalize_rows(x):
    lib = _enc()
    x = _f32(x).copy()
    lib.normalize_rows(_p(x), x.shape[0], x.shape[1])
    return x


def tiny_embed(table, proj, ids):
    lib = _enc()
    table, proj = _f32(table), _f32(proj)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.zeros((ids.shape[0], proj.shape[1]), np.float32)
    lib.tiny_embed(_p(table), table.shape[0], table.shape[1], _p(proj), proj.shape[1], _p(ids),
                   ids.shape[0], _p(out))
    return out


# ------------------------------------------------- compact (family (a)) embedder

def rope_rows(x, seq):
    """ropeRows on [rows][cols] with pos = row % seq."""
    lib = _enc()
    x = _f32(x).copy()
    lib.rope_rows(_p(x), x.shape[0], seq, x.shape[1])
    return x


def matmul_f32(x, w):
    """matmulTensor: x [rows][in] @ w [in][out], f32 in k order."""
    lib = _enc()
    x, w = _f32(x), _f32(w)
    y = np.zeros((x.shape[0], w.shape[1]), np.float32)
    lib.matmul_f32(_p(x), x.shape[0], x.shape[1], _p(w), w.shape[1], _p(y))
    return y


def layer_norm_rows(x):
    lib = _enc()
    x = _f32(x).copy()
    lib.layer_norm_rows(_p(x), x.shape[0], x.shape[1])
    return x


def gelu_tanh(x):
    """geluTensor (tanh form) elementwise."""
    lib = _enc()
    x = _f32(x).copy()
    lib.gelu_tanh_inplace(_p(x), x.size)
    return x


def compact_single_head_attention(q, k, v, mask):
    """q, k, v: [batch*tokens][dim]; mask [batch][tokens]."""
    lib = _enc()
    q, k, v = _f32(q), _f32(k), _f32(v)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    batch, tokens = mask.shape
    out = np.zeros_like(q)
    lib.compact_single_head_attention(_p(q), _p(k), _p(v), _p(mask), batch, tokens, q.shape[1],
                                      _p(out))
    return out


COMPACT_NO_ROPE, COMPACT_UNSCALED, COMPACT_ATTEND_ALL = 1, 2, 4


def compact_embed(tok, role, layers, ids, mask, role_ids, heads, wout=None, flags=0):
    """Family (a) embedder. tok [V][D], role [R][D] dequantized f32 (None: no
    role rows); layers: list of (wq, wk, wv, wo, wup, wdown) in [in, out]
    layout; wout [D][O] or None. flags: COMPACT_NO_ROPE, COMPACT_UNSCALED (one
    head's plain q kT), COMPACT_ATTEND_ALL (softmax over every position, the
    mask only pools)."""
    lib = _enc()
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    roles = np.zeros_like(ids) if role_ids is None else np.ascontiguousarray(role_ids, np.int32)
    batch, tokens = ids.shape
    dim = tok.shape[1]
    ffn = layers[0][4].shape[1] if layers else dim
    keep = [_f32(x) for L in layers for x in L]
    ptrs = (C.c_void_p * max(len(keep), 1))(*[k.ctypes.data for k in keep])
    if role is None:
        role = np.zeros((1, tok.shape[1]), np.float32)
        roles = np.zeros_like(ids)
    tok, role = _f32(tok), _f32(role)
    wo = None if wout is None else _f32(wout)
    odim = dim if wo is None else wo.shape[1]
    out = np.zeros((batch, odim), np.float32)
    lib.compact_embed_opts(_p(tok), tok.shape[0], _p(role), role.shape[0], ptrs, len(layers),
                           None if wo is None else _p(wo), odim, _p(ids), _p(roles), _p(mask),
                           batch, tokens, dim, heads, ffn, int(flags), _p(out))
    return out


# ------------------------------------------------ two-stage retrieval (f16)
class _Scored(C.Structure):
    _fields_ = [("id", C.c_int64), ("score", C.c_float), ("rank", C.c_int), ("compact", C.c_float)]


def f32_to_half(x) -> np.ndarray:
    """float32ToHalf (runtime/mll_export.go:1007-1041) elementwise -> uint16."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    load().oracle_f32_to_half_n(x.ctypes.data_as(C.c_void_p), C.c_int64(x.size),
                                out.ctypes.data_as(C.c_void_p))
    return out


def half_to_f32(h) -> np.ndarray:
    """halfToFloat32 (runtime/weight_file.go:461-483) elementwise."""
    fn = load().oracle_half_to_f32
    fn.restype, fn.argtypes = C.c_float, [C.c_uint16]
    h = np.asarray(h, np.uint16)
    return np.array([fn(int(v)) for v in h.ravel()], np.float32).reshape(h.shape)


def fp16_rerank_should_rescue(bit_width: int, k: int, overfetch: int, c: int) -> bool:
    """shouldApplyTurboQuantFP16RerankRescue (runtime/retrieval_turboquant.go:1664-1669)."""
    return bit_width == 4 and k == 100 and overfetch == 200 and c >= 120


def apply_rescue(ids, scores, ranks, compact) -> np.ndarray:
    """applyTurboQuantFP16RerankRescue over an already fp16-ranked list; returns the ids."""
    m = len(ids)
    arr = (_Scored * max(m, 1))()
    for i in range(m):
        arr[i] = _Scored(int(ids[i]), float(scores[i]), int(ranks[i]), float(compact[i]))
    out = (_Scored * max(m, 1))()
    load().oracle_apply_rescue(arr, C.c_int(m), out)
    return np.array([out[i].id for i in range(m)], np.int64)


def fp16_rerank(queries, rows, cand_ids, cand_scores, k, bit_width=0, overfetch=0, rescue=None):
    """Second stage for each query: (ids int64 [Q, kk], scores float32 [Q, kk]),
    rows past a query's result count hold id -1 and score 0."""
    q = np.ascontiguousarray(queries, np.float32)
    rows = np.ascontiguousarray(rows, np.uint16)
    cid = np.ascontiguousarray(cand_ids, np.int64)
    cs = np.ascontiguousarray(cand_scores, np.float32)
    nq, d = q.shape
    c = cid.shape[1]
    kk = c if (k <= 0 or k > c) else k
    if rescue is None:
        rescue = fp16_rerank_should_rescue(bit_width, k, overfetch, c)
    ids = np.full((nq, kk), -1, np.int64)
    scores = np.zeros((nq, kk), np.float32)
    lib = load()
    for i in range(nq):
        lib.oracle_fp16_rerank(q[i].ctypes.data_as(C.c_void_p), C.c_int(d),
                               rows.ctypes.data_as(C.c_void_p), C.c_int64(rows.shape[0]),
                               cid[i].ctypes.data_as(C.c_void_p), cs[i].ctypes.data_as(C.c_void_p),
                               C.c_int(c), C.c_int(int(k)), C.c_int(1 if rescue else 0),
                               ids[i].ctypes.data_as(C.c_void_p), scores[i].ctypes.data_as(C.c_void_p))
    return ids, scores


def _rerank_finish(scores, cid, n, k, id_rank):
    lib = load()
    nq, c = cid.shape
    kk = c if (k <= 0 or k > c) else k
    ids = np.full((nq, kk), -1, np.int64)
    out = np.zeros((nq, kk), np.float32)
    rank = None if id_rank is None else np.ascontiguousarray(id_rank, np.int64)
    for i in range(nq):
        lib.oracle_rerank_order(scores[i].ctypes.data_as(C.c_void_p),
                                cid[i].ctypes.data_as(C.c_void_p), C.c_int64(n), C.c_int(c),
                                C.c_int(int(k)),
                                None if rank is None else rank.ctypes.data_as(C.c_void_p),
                                ids[i].ctypes.data_as(C.c_void_p),
                                out[i].ctypes.data_as(C.c_void_p))
    return ids, out


def dense_rerank(queries, rows, cand_ids, k, id_rank=None):
    """topDenseRerankScores per query over f32 rows: (ids [Q, kk], scores)."""
    q = np.ascontiguousarray(queries, np.float32)
    rows = np.ascontiguousarray(rows, np.float32)
    cid = np.ascontiguousarray(cand_ids, np.int64)
    nq, d = q.shape
    c = cid.shape[1]
    sc = np.zeros((nq, c), np.float32)
    lib = load()
    for i in range(nq):
        lib.oracle_dense_scores(q[i].ctypes.data_as(C.c_void_p), C.c_int(d),
                                rows.ctypes.data_as(C.c_void_p), C.c_int64(rows.shape[0]),
                                cid[i].ctypes.data_as(C.c_void_p), C.c_int(c),
                                sc[i].ctypes.data_as(C.c_void_p))
    return _rerank_finish(sc, cid, rows.shape[0], k, id_rank)


def reconstruct_rerank(queries, rotation, codes, bits, norms, codebook, cand_ids, k,
                       id_rank=None, signs=None, resnorms=None, sketch=None):
    """Reconstruct / mixed-width rerank per query (rerank_oracle.c): each
    candidate dequantized to the original frame (with the QJL term when
    signs, resnorms and sketch S [d, d] are given: an inner-product code
    set), then the f32 index-order dot. (ids [Q, kk], scores)."""
    q = np.ascontiguousarray(queries, np.float32)
    rot = None if rotation is None else np.ascontiguousarray(rotation, np.float32)
    codes = np.ascontiguousarray(codes, np.uint8)
    norms = np.ascontiguousarray(norms, np.float32)
    cb = np.ascontiguousarray(codebook, np.float32)
    cid = np.ascontiguousarray(cand_ids, np.int64)
    ip = signs is not None
    if ip:
        signs = np.ascontiguousarray(signs, np.uint8)
        resnorms = np.ascontiguousarray(resnorms, np.float32)
        sketch = np.ascontiguousarray(sketch, np.float32)
    nq, d = q.shape
    c = cid.shape[1]
    n = norms.shape[0]
    sc = np.zeros((nq, c), np.float32)
    lib = load()
    fn = lib.oracle_recon_scores_ip
    fn.restype = None
    vp = lambda a: None if a is None else a.ctypes.data_as(C.c_void_p)
    for i in range(nq):
        fn(vp(q[i]), C.c_int(d), vp(rot), vp(codes), C.c_int(bits), vp(norms), vp(cb),
           vp(signs) if ip else None, vp(resnorms) if ip else None, vp(sketch) if ip else None,
           C.c_int64(n), vp(cid[i]), C.c_int(c), vp(sc[i]))
    return _rerank_finish(sc, cid, n, k, id_rank)


def tq_dequantize(rotation, code_row, bits, norm, codebook, sign_row=None, resnorm=0.0,
                  sketch=None):
    """One entry's dequantized vector (rerank_oracle.c oracle_tq_dequantize)."""
    cb = np.ascontiguousarray(codebook, np.float32)
    row = np.ascontiguousarray(code_row, np.uint8)
    d = None
    rot = None if rotation is None else np.ascontiguousarray(rotation, np.float32)
    sk = None if sketch is None else np.ascontiguousarray(sketch, np.float32)
    if rot is not None:
        d = rot.shape[0]
    elif sk is not None:
        d = sk.shape[0]
    else:
        d = row.size * 8 // bits
    out = np.zeros(d, np.float32)
    sg = None if sign_row is None else np.ascontiguousarray(sign_row, np.uint8)
    vp = lambda a: None if a is None else a.ctypes.data_as(C.c_void_p)
    fn = load().oracle_tq_dequantize
    fn.restype = None
    fn(C.c_int(d), vp(rot), vp(row), C.c_int(bits), C.c_float(norm), vp(cb), vp(sg),
       C.c_float(resnorm), vp(sk), vp(out))
    return out


# ------------------------------------------------ Hadamard TurboQuant codec
def hq_fwht(v):
    """Normalized FWHT on power-of-two blocks (retrieval_oracle.c)."""
    x = np.array(v, np.float32)
    fn = load().hq_fwht
    fn.argtypes = [C.c_void_p, C.c_int]
    fn.restype = None
    fn(_p(x), x.shape[0])
    return x


def hq_norm_code(norm: float) -> int:
    fn = load().hq_norm_code
    fn.argtypes = [C.c_float]
    fn.restype = C.c_int
    return fn(C.c_float(norm))


def hq_norm_value(code: int) -> float:
    fn = load().hq_norm_value
    fn.argtypes = [C.c_int]
    fn.restype = C.c_float
    return fn(int(code))


def hq_encode(x, perm, s1, s2, boundaries, levels):
    """x f32 [n, C, H, W] -> (coords u8 [n, C, H, W], norm codes u8 [n, H, W])."""
    x = _f32(x)
    n, c, h, w = x.shape
    coords = np.zeros(x.shape, np.uint8)
    norms = np.zeros((n, h, w), np.uint8)
    fn = load().hq_encode
    fn.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int] + [C.c_void_p] * 4 + [C.c_int] + \
        [C.c_void_p] * 2
    fn.restype = None
    perm = np.ascontiguousarray(perm, np.int32)
    s1, s2, b = _f32(s1), _f32(s2), _f32(boundaries)
    fn(_p(x), n, c, h * w, _p(perm), _p(s1), _p(s2), _p(b), levels, _p(coords), _p(norms))
    return coords, norms


def hq_decode(coords, norms, perm, s1, s2, centroids, levels):
    coords = np.ascontiguousarray(coords, np.uint8)
    norms = np.ascontiguousarray(norms, np.uint8)
    n, c, h, w = coords.shape
    out = np.zeros(coords.shape, np.float32)
    fn = load().hq_decode
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int] + [C.c_void_p] * 4 + \
        [C.c_int, C.c_void_p]
    fn.restype = None
    perm = np.ascontiguousarray(perm, np.int32)
    s1, s2, cb = _f32(s1), _f32(s2), _f32(centroids)
    fn(_p(coords), _p(norms), n, c, h * w, _p(perm), _p(s1), _p(s2), _p(cb), levels, _p(out))
    return out


# ------------------------------------------------ inner-product layout (QJL)
def tq_encode_ip(vectors, rotation, qjl, dim, bits, codebook, codebook_scale):
    """(codes [n, row_bytes], signs [n, (d + 7) // 8], resnorms [n], norms [n])."""
    x = _f32(vectors).reshape(-1, dim)
    n = x.shape[0]
    rot = None if rotation is None else _f32(rotation)
    s = _f32(qjl)
    cb = np.ascontiguousarray(codebook, np.int8)
    codes = np.zeros((n, (dim * bits + 7) // 8), np.uint8)
    signs = np.zeros((n, (dim + 7) // 8), np.uint8)
    rn = np.zeros(n, np.float32)
    nm = np.zeros(n, np.float32)
    fn = load().tq_encode_ip
    fn.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                   C.c_float] + [C.c_void_p] * 4
    fn.restype = None
    fn(_p(x), n, _p(rot), _p(s), dim, bits, _p(cb), C.c_float(codebook_scale), _p(codes),
       _p(signs), _p(rn), _p(nm))
    return codes, signs, rn, nm


def tq_ip_scores(queries, rotation, qjl, dim, bits, codebook, codebook_scale, codes, signs,
                 resnorms, norms):
    q = _f32(queries).reshape(-1, dim)
    rot = None if rotation is None else _f32(rotation)
    s = _f32(qjl)
    cb = np.ascontiguousarray(codebook, np.int8)
    codes = np.ascontiguousarray(codes, np.uint8)
    signs = np.ascontiguousarray(signs, np.uint8)
    rn, nm = _f32(resnorms), _f32(norms)
    n = nm.shape[0]
    out = np.zeros((q.shape[0], n), np.float32)
    fn = load().tq_ip_scores
    fn.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                   C.c_float] + [C.c_void_p] * 4 + [C.c_int64, C.c_void_p]
    fn.restype = None
    fn(_p(q), q.shape[0], _p(rot), _p(s), dim, bits, _p(cb), C.c_float(codebook_scale),
       _p(codes), _p(signs), _p(rn), _p(nm), n, _p(out))
    return out
