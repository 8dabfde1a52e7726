"""Step-by-step interpreter of an Eos plan in numpy (test infrastructure
only: the checker of the fused encoder bound from a .mll package, never on a
product path).

Runs an entry's step list the way ExecuteSymbolic does
(runtime/backend/symbolic.go:17-172 with executeStep,
runtime/backend/tensor_ops.go:13-633): every value lives in an environment
by name, params are the dequantized weights, and each step reads its inputs
and binds its outputs. The host ops, in the reference's precisions:

  gather       gatherTensor (tensor_ops.go:938-1166): rows by i32 index; an
               index out of range is an error
  dequant      a dtype relabel of values already dequantized at load
               (tensor_ops.go:225-237)
  matmul       matmulTensor (tensor_ops.go:1168-1249), rank 2 or 3, [in, out]
               right operand, scale attribute (matmulScale, :1291-1315)
  transpose    transposeTensor (tensor_ops.go:1317-1365): last two axes
  softmax      softmaxRows (tensor_ops.go:1757-1788): f32 maximum, f64 exp and
               sum, f32 probabilities times float32(1 / sum)
  masked_softmax  maskedSoftmaxRowsF32 (tensor_ops.go:1825-1865)
  binary_add   f32 elementwise add
  layernorm    layerNormRows (tensor_ops.go:1393-1421): f32 mean and
               variance, float32(1 / sqrt(f64(var) + 1e-5))
  gelu         geluTensor (tensor_ops.go:1926-1934): tanh form, f64 tanh
  normalize    normalizeRows (tensor_ops.go:1367-1391): f64 sum of squares,
               f32 norm, rows of norm 0 unchanged
  mean_pool    meanPoolMaskedTensor (tensor_ops.go:1644-1709): f32 sum of the
               mask != 0 rows times float32(1 / count), count 0 -> zeros
  dot, cosine, l2_distance   dotRows / cosineRows / l2DistanceRows
               (tensor_ops.go:1967-2122) through the C restatement
               (retrieval_oracle.c), per query for the [Q, D] x [Q, N, D] form
  topk         topKTensor (tensor_ops.go:2124-2193): score descending, index
               ascending; k above the row width is an error
  gather       modes "batched" (per-row table) and "shared" as the compiler
               marks them (compiler/compiler.go:1872-1900)
  pack_candidates   NewCandidatePack (runtime/backend/tensor.go:105-118): the
               (ids, scores, docs) triple

One difference in summation order: matmul sums in f64 and rounds once to
f32 where the reference runs an f32 sum in k order (relative difference
below k * 2^-24), and the f32 reductions use numpy's pairwise order.
"""
from __future__ import annotations

import numpy as np

import oracle

F32 = np.float32


def _kernel_op(artifact: dict, name: str) -> tuple[str, dict]:
    for k in artifact.get("kernels", []):
        if k.get("name") == name:
            body = k.get("body", [])
            if len(body) != 2 or body[1].get("op") != "return":
                raise ValueError(f"kernel {name}: body is not one op + return")
            return body[0]["op"], body[0].get("attributes", {}) or {}
    raise ValueError(f"unknown kernel {name}")


def _softmax_rows(x: np.ndarray, mask: np.ndarray | None = None) -> np.ndarray:
    x = x.astype(F32)
    if mask is not None:
        keep = np.broadcast_to(mask != 0, x.shape)
        mx = np.where(keep, x, -np.inf).max(axis=-1, keepdims=True)
        ev = np.where(keep, np.exp((x - mx).astype(np.float64)), 0.0)
    else:
        mx = x.max(axis=-1, keepdims=True)
        ev = np.exp((x - mx).astype(np.float64))
    s = ev.sum(axis=-1, keepdims=True)
    inv = np.where(s != 0, (1.0 / np.where(s != 0, s, 1.0)).astype(F32), F32(1))
    out = ev.astype(F32) * inv
    if mask is not None:
        out = np.where(np.isfinite(mx), out, F32(0))
    return out.astype(F32)


def _layernorm_rows(x: np.ndarray) -> np.ndarray:
    x = x.astype(F32)
    cols = x.shape[-1]
    mean = x.sum(axis=-1, keepdims=True, dtype=F32) / F32(cols)
    c = x - mean
    var = (c * c).sum(axis=-1, keepdims=True, dtype=F32) / F32(cols)
    inv = (1.0 / np.sqrt(var.astype(np.float64) + 1e-5)).astype(F32)
    return (c * inv).astype(F32)


def _gelu(x: np.ndarray) -> np.ndarray:
    x = x.astype(F32)
    inner = F32(0.7978845608) * (x + F32(0.044715) * (x * x * x))
    return (F32(0.5) * x * (F32(1) + np.tanh(inner.astype(np.float64)).astype(F32))).astype(F32)


def _normalize_rows(x: np.ndarray) -> np.ndarray:
    x = x.astype(F32)
    norm = np.sqrt((x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True)).astype(F32)
    return np.where(norm == 0, x, x / np.where(norm == 0, F32(1), norm)).astype(F32)


def _mean_pool(x: np.ndarray, mask: np.ndarray) -> np.ndarray:
    keep = (mask != 0)
    s = (x.astype(F32) * keep[..., None]).sum(axis=-2, dtype=F32)
    cnt = keep.sum(axis=-1)
    inv = np.where(cnt > 0, (1.0 / np.maximum(cnt, 1)).astype(F32), F32(0))
    return (s * inv[..., None]).astype(F32)


def _matmul(a: np.ndarray, b: np.ndarray, attrs: dict) -> np.ndarray:
    out = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(F32)
    scale = (attrs or {}).get("scale", "")
    if scale in ("", "none"):
        return out
    if scale == "rsqrt_rhs_rows":
        return (out * F32(1.0 / np.sqrt(float(b.shape[-2])))).astype(F32)
    return (out * F32(float(scale))).astype(F32)


def run(artifact: dict, params: dict[str, np.ndarray], entry: str,
        inputs: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    """Execute `entry`; params: name -> dequantized f32 values; inputs: name
    -> i32 arrays. Returns the returned values by name."""
    env: dict[str, np.ndarray] = {k: np.asarray(v) for k, v in inputs.items()}
    result = {}
    steps = [s for s in artifact["steps"] if s.get("entry") == entry]
    if not steps:
        raise ValueError(f"entrypoint {entry} has no plan steps")

    def val(name):
        if name in env:
            return env[name]
        if name in params:
            return np.asarray(params[name], F32)
        raise KeyError(f"missing runtime input {name}")

    for st in steps:
        kind = st["kind"]
        ins = [val(n) for n in st.get("inputs", [])]
        outs = st.get("outputs", [])
        if kind == "return":
            for n in outs:
                result[n] = env[n]
            continue
        if kind == "gather":
            table, idx = ins
            idx = np.asarray(idx)
            mode = (st.get("attributes") or {}).get("mode", "")
            if mode == "batched":
                if idx.min() < 0 or idx.max() >= table.shape[1]:
                    raise IndexError("gather index out of range")
                y = np.stack([table[b][idx[b]] for b in range(idx.shape[0])])
            else:
                if idx.min() < 0 or idx.max() >= table.shape[0]:
                    raise IndexError("gather index out of range")
                y = table[idx]
            if y.dtype not in (np.int32, np.int64):
                y = y.astype(F32)
        elif kind == "topk":
            k = int(st["attributes"]["k"])
            s2 = np.atleast_2d(ins[0])
            if k <= 0 or k > s2.shape[1]:
                raise ValueError(f"topk limit {k} out of range for row width {s2.shape[1]}")
            y = np.stack([oracle.topk_scores(row, k)[0] for row in s2]).astype(np.int32)
            if ins[0].ndim == 1:
                y = y[0]
        elif kind == "pack_candidates":
            y = tuple(ins)
        elif kind == "dequant":
            y = ins[0].astype(F32)
        elif kind == "matmul":
            y = _matmul(ins[0], ins[1], st.get("attributes", {}))
        elif kind == "transpose":
            y = np.ascontiguousarray(np.swapaxes(ins[0], -1, -2))
        elif kind == "launch_kernel":
            op, attrs = _kernel_op(artifact, st["kernel"])
            if op == "softmax":
                y = _softmax_rows(ins[0])
            elif op == "masked_softmax":
                m = ins[1]
                y = _softmax_rows(ins[0], m[..., None, :] if m.ndim == ins[0].ndim - 1 else m)
            elif op == "binary_add":
                y = (ins[0].astype(F32) + ins[1].astype(F32)).astype(F32)
            elif op == "layernorm":
                y = _layernorm_rows(ins[0])
            elif op == "gelu":
                y = _gelu(ins[0])
            elif op == "normalize":
                y = _normalize_rows(ins[0])
            elif op == "mean_pool":
                y = _mean_pool(ins[0], ins[1])
            elif op in ("dot", "cosine", "l2_distance"):
                q, docs = ins
                if q.ndim == 1:
                    y = oracle.score_rows(op, q, docs)
                else:
                    y = np.stack([oracle.score_rows(op, q[b], docs[b]) for b in range(q.shape[0])])
            else:
                raise ValueError(f"kernel op {op} not in this interpreter")
        else:
            raise ValueError(f"step kind {kind} not in this interpreter")
        env[outs[0]] = y
    return result
