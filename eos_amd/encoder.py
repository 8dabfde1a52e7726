"""q8 encoders on the MI355X backend.

Host-side mirrors of the reference's two embedder families:
- ``Encoder``: the bert_embedder step (runtime/backend/bert_embedder_ops.go:
  101-197, BERTEmbedderReferenceWithPooling). ``embed(input_ids,
  attention_mask, token_type_ids)`` returns the masked mean-pooled,
  L2-normalized sentence embeddings [batch, hidden].
- ``CompactEncoder``: the compact transformer graph of the default embedder
  (models/default_embedding.go:419-505). ``embed(tokens, attention_mask,
  role_ids)`` returns the masked mean of the per-token normalized (and
  optionally projected) states [batch, output_dim].
Errors follow the reference: ids outside their tables are rejected
(runtime/backend/tensor_ops.go:1484-1492). All arithmetic runs in libeoship's
gfx950 kernels.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, Runtime


@dataclass
class EncoderLayerWeights:
    """One post-LN layer: int8 codes in HF [out, in] layout + per-output-channel scales."""
    w_qkv: np.ndarray  # int8 [3H, H]
    s_qkv: np.ndarray  # f32 [3H]
    b_qkv: np.ndarray  # f32 [3H]
    w_o: np.ndarray
    s_o: np.ndarray
    b_o: np.ndarray
    ln1_gamma: np.ndarray
    ln1_beta: np.ndarray
    w_1: np.ndarray    # int8 [F, H]
    s_1: np.ndarray
    b_1: np.ndarray
    w_2: np.ndarray    # int8 [H, F]
    s_2: np.ndarray
    b_2: np.ndarray
    ln2_gamma: np.ndarray
    ln2_beta: np.ndarray

    def dequantized(self):
        """The 16 f32 tensors in the reference order (q,k,v split), code * scale."""
        H = self.w_o.shape[0]
        wq = self.w_qkv.astype(np.float32) * self.s_qkv[:, None]
        wo = self.w_o.astype(np.float32) * self.s_o[:, None]
        w1 = self.w_1.astype(np.float32) * self.s_1[:, None]
        w2 = self.w_2.astype(np.float32) * self.s_2[:, None]
        b = self.b_qkv
        return [wq[:H], b[:H], wq[H:2 * H], b[H:2 * H], wq[2 * H:], b[2 * H:], wo, self.b_o,
                self.ln1_gamma, self.ln1_beta, w1, self.b_1, w2, self.b_2, self.ln2_gamma,
                self.ln2_beta]


@dataclass
class EncoderWeights:
    hidden: int
    heads: int
    intermediate: int
    ln_eps: float
    gelu: int  # 1 erf, 2 tanh
    tok: np.ndarray     # f32 [V, H]
    pos: np.ndarray     # f32 [P, H]
    typ: np.ndarray     # f32 [T, H]
    emb_gamma: np.ndarray
    emb_beta: np.ndarray
    layers: list = field(default_factory=list)


def quantize_per_channel(w: np.ndarray):
    """Symmetric absmax int8 per output channel (rows): scale = max|w|/127,
    code = clamp(round(w/scale), +-127) -- the reference's q8 grid
    (runtime/mll_export.go:918-942) applied per row."""
    w = np.asarray(w, dtype=np.float32)
    mx = np.max(np.abs(w), axis=1)
    scale = np.where(mx > 0, mx / np.float32(127.0), np.float32(0.0)).astype(np.float32)
    safe = np.where(scale > 0, scale, np.float32(1.0))
    codes = np.clip(np.rint(w / safe[:, None]), -127, 127).astype(np.int8)
    codes[scale == 0] = 0
    return codes, scale


def quantize_per_tensor(w: np.ndarray, bits: int = 8):
    """The reference's per-tensor grid (packQuantizedTensorStorage,
    runtime/mll_export.go:897-942): levels = 2^(bits-1) - 1, scale =
    float32(max|w|) / levels, code = clamp(round-half-away(float32(w / scale)),
    +-levels). q4 codes are passed unpacked (the payload nibble is code + 8,
    runtime/weight_file.go:334-350). Returns int8 codes and the f32 scale (0
    for an all-zero tensor)."""
    w = np.asarray(w, dtype=np.float32)
    levels = np.float32((1 << (bits - 1)) - 1)
    mx = np.float32(np.max(np.abs(w))) if w.size else np.float32(0.0)
    if mx == 0:
        return np.zeros(w.shape, np.int8), np.float32(0.0)
    scale = np.float32(mx / levels)
    q = (w / scale).astype(np.float32)
    q = np.sign(q) * np.floor(np.abs(q).astype(np.float64) + 0.5)  # exact in f64
    codes = np.clip(q, -levels, levels).astype(np.int8)
    return codes, scale


@dataclass
class CompactLayerWeights:
    """One compact layer: int8 codes in the reference's [in, out] layout, one
    scale per tensor (models/default_embedding.go:425-431)."""
    attn_q: np.ndarray   # int8 [D, D]
    s_q: float
    attn_k: np.ndarray
    s_k: float
    attn_v: np.ndarray
    s_v: float
    attn_o: np.ndarray
    s_o: float
    ffn_up: np.ndarray   # int8 [D, H]
    s_up: float
    ffn_down: np.ndarray  # int8 [H, D]
    s_down: float

    def dequantized(self):
        """(wq, wk, wv, wo, wup, wdown) f32 = code * scale, [in, out]."""
        f = lambda c, s: c.astype(np.float32) * np.float32(s)
        return (f(self.attn_q, self.s_q), f(self.attn_k, self.s_k), f(self.attn_v, self.s_v),
                f(self.attn_o, self.s_o), f(self.ffn_up, self.s_up),
                f(self.ffn_down, self.s_down))


@dataclass
class CompactWeights:
    """DefaultEmbeddingPackageConfig-shaped weights (models/default_embedding.go:264-300)."""
    model_dim: int
    heads: int
    hidden_dim: int
    max_sequence: int
    token_embedding: np.ndarray  # int8 [V, D]
    s_token: float
    role_embedding: np.ndarray   # int8 [3, D]
    s_role: float
    layers: list = field(default_factory=list)
    output_projection: np.ndarray | None = None  # int8 [D, O]
    s_output: float = 0.0

    @property
    def output_dim(self) -> int:
        p = self.output_projection
        return self.model_dim if p is None else int(p.shape[1])


def _p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


class Encoder:
    """An encoder bound on the device."""

    def __init__(self, rt: Runtime, w: EncoderWeights):
        self.rt, self.w = rt, w
        H, F = w.hidden, w.intermediate
        self._keep = []

        def f32(x, shape):
            a = np.ascontiguousarray(x, dtype=np.float32)
            if a.shape != shape:
                raise ValueError(f"expected {shape}, got {a.shape}")
            self._keep.append(a)
            return a

        def i8(x, shape):
            a = np.ascontiguousarray(x, dtype=np.int8)
            if a.shape != shape:
                raise ValueError(f"expected {shape}, got {a.shape}")
            self._keep.append(a)
            return a

        layers = (_lib.EosHipEncoderLayer * max(len(w.layers), 1))()
        for i, L in enumerate(w.layers):
            x = layers[i]
            x.w_qkv = _p(i8(L.w_qkv, (3 * H, H)), C.c_int8)
            x.s_qkv = _p(f32(L.s_qkv, (3 * H,)), C.c_float)
            x.b_qkv = _p(f32(L.b_qkv, (3 * H,)), C.c_float)
            x.w_o = _p(i8(L.w_o, (H, H)), C.c_int8)
            x.s_o = _p(f32(L.s_o, (H,)), C.c_float)
            x.b_o = _p(f32(L.b_o, (H,)), C.c_float)
            x.ln1_gamma = _p(f32(L.ln1_gamma, (H,)), C.c_float)
            x.ln1_beta = _p(f32(L.ln1_beta, (H,)), C.c_float)
            x.w_1 = _p(i8(L.w_1, (F, H)), C.c_int8)
            x.s_1 = _p(f32(L.s_1, (F,)), C.c_float)
            x.b_1 = _p(f32(L.b_1, (F,)), C.c_float)
            x.w_2 = _p(i8(L.w_2, (H, F)), C.c_int8)
            x.s_2 = _p(f32(L.s_2, (H,)), C.c_float)
            x.b_2 = _p(f32(L.b_2, (H,)), C.c_float)
            x.ln2_gamma = _p(f32(L.ln2_gamma, (H,)), C.c_float)
            x.ln2_beta = _p(f32(L.ln2_beta, (H,)), C.c_float)
        desc = _lib.EosHipEncoderDesc(
            layers=len(w.layers), hidden=H, heads=w.heads, intermediate=F,
            vocab=w.tok.shape[0], max_positions=w.pos.shape[0], type_vocab=w.typ.shape[0],
            ln_eps=w.ln_eps, gelu=w.gelu)
        tok = f32(w.tok, (w.tok.shape[0], H))
        pos = f32(w.pos, (w.pos.shape[0], H))
        typ = f32(w.typ, (w.typ.shape[0], H))
        eg = f32(w.emb_gamma, (H,))
        eb = f32(w.emb_beta, (H,))
        self.out_dim = H
        self.handle = C.c_void_p()
        _lib.call("eoship_encoder_bind", rt.handle, C.byref(desc), _p(tok, C.c_float),
                  _p(pos, C.c_float), _p(typ, C.c_float), _p(eg, C.c_float), _p(eb, C.c_float),
                  layers, C.byref(self.handle))
        self._keep = []

    def release(self) -> None:
        # After the runtime is closed the object cannot be released any more
        # (its stream is gone); the handle is only dropped.
        if self.handle and self.rt.handle:
            _lib.call("eoship_encoder_release", self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def embed(self, input_ids: np.ndarray, attention_mask: np.ndarray,
              token_type_ids: np.ndarray | None = None) -> np.ndarray:
        ids = np.ascontiguousarray(input_ids, dtype=np.int32)
        mask = np.ascontiguousarray(attention_mask, dtype=np.int32)
        if ids.ndim != 2 or mask.shape != ids.shape:
            raise ValueError("input_ids and attention_mask must both be [batch, tokens]")
        types = None
        if token_type_ids is not None:
            types = np.ascontiguousarray(token_type_ids, dtype=np.int32)
            if types.shape != ids.shape:
                raise ValueError("token_type_ids must match input_ids")
        out = np.zeros((ids.shape[0], self.out_dim), np.float32)
        _lib.call("eoship_encoder_forward", self.rt.handle, self.handle,
                  ids.ctypes.data_as(C.c_void_p),
                  types.ctypes.data_as(C.c_void_p) if types is not None else None,
                  mask.ctypes.data_as(C.c_void_p), C.c_int32(ids.shape[0]),
                  C.c_int32(ids.shape[1]), out.ctypes.data_as(C.c_void_p))
        return out

    def embed_device(self, d_ids: DeviceBuffer, d_mask: DeviceBuffer, batch: int, tokens: int,
                     d_out: DeviceBuffer, d_types: DeviceBuffer | None = None) -> None:
        """Enqueue a forward on device buffers (no wait)."""
        _lib.call("eoship_encoder_forward_device", self.rt.handle, self.handle, d_ids.ptr,
                  d_types.ptr if d_types is not None else None, d_mask.ptr, C.c_int32(batch),
                  C.c_int32(tokens), d_out.ptr)

    def status(self) -> int:
        st = C.c_int32()
        _lib.call("eoship_encoder_status", self.rt.handle, self.handle, C.byref(st))
        return st.value

    def set_fused_tail(self, fused: bool) -> None:
        """BERT family at hidden 384 / 512 / 768: run the layer tail as one
        fused kernel (default) or as the unfused GEMM + LayerNorm launches."""
        _lib.call("eoship_encoder_set_fused_tail", self.rt.handle, self.handle, C.c_int32(int(fused)))

    def set_pooling(self, pooling: str) -> None:
        """BERT family: "masked_mean" (default) or "cls" (bert_embedder's
        pooling attribute, runtime/backend/bert_embedder_ops.go:150-152)."""
        modes = {"masked_mean": 0, "cls": 1}
        if pooling not in modes:
            raise ValueError(f"unsupported pooling {pooling!r}; supported values are masked_mean and cls")
        _lib.call("eoship_encoder_set_pooling", self.rt.handle, self.handle,
                  C.c_int32(modes[pooling]))

    def attention_moves(self) -> int:
        """Diagnostic of the last forward: attention wavefronts that moved their
        softmax exponent reference after a sequence's first key block."""
        mv = C.c_int64()
        _lib.call("eoship_encoder_attention_moves", self.rt.handle, self.handle, C.byref(mv))
        return int(mv.value)


class CompactEncoder(Encoder):
    """A compact (family (a)) embedder bound on the device; ``embed`` takes
    (tokens, attention_mask, role_ids) and returns [batch, output_dim]."""

    def __init__(self, rt: Runtime, w: CompactWeights, options: dict | None = None):
        """options: graph options {rope, role, scaled_scores, attend_padding}
        (0/1 each; None: the compactTransformerSource graph, 1/1/1/0); with
        role 0 the role table is not read."""
        self.rt, self.w = rt, w
        D, F = w.model_dim, w.hidden_dim
        keep = []

        def i8(x, shape):
            a = np.ascontiguousarray(x, dtype=np.int8)
            if a.shape != shape:
                raise ValueError(f"expected {shape}, got {a.shape}")
            keep.append(a)
            return _p(a, C.c_int8)

        layers = (_lib.EosHipCompactLayer * max(len(w.layers), 1))()
        for i, L in enumerate(w.layers):
            x = layers[i]
            x.attn_q, x.s_q = i8(L.attn_q, (D, D)), L.s_q
            x.attn_k, x.s_k = i8(L.attn_k, (D, D)), L.s_k
            x.attn_v, x.s_v = i8(L.attn_v, (D, D)), L.s_v
            x.attn_o, x.s_o = i8(L.attn_o, (D, D)), L.s_o
            x.ffn_up, x.s_up = i8(L.ffn_up, (D, F)), L.s_up
            x.ffn_down, x.s_down = i8(L.ffn_down, (F, D)), L.s_down
        vocab = int(np.asarray(w.token_embedding).shape[0])
        tok = i8(w.token_embedding, (vocab, D))
        opts = None
        if options is not None:
            full = {"rope": 1, "role": 1, "scaled_scores": 1, "attend_padding": 0}
            unknown = set(options) - set(full)
            if unknown:
                raise ValueError(f"unknown compact options {sorted(unknown)}")
            full.update({k: int(v) for k, v in options.items()})
            opts = _lib.EosHipCompactOptions(**full)
        role = None
        if opts is None or opts.role:
            role = i8(w.role_embedding, (3, D))
        proj = None
        if w.output_projection is not None:
            proj = i8(w.output_projection, (D, w.output_dim))
        desc = _lib.EosHipCompactDesc(layers=len(w.layers), model_dim=D, heads=w.heads,
                                      hidden_dim=F, vocab=vocab, max_sequence=w.max_sequence,
                                      output_dim=w.output_dim)
        self.out_dim = w.output_dim
        self.handle = C.c_void_p()
        _lib.call("eoship_encoder_bind_compact_opts", rt.handle, C.byref(desc),
                  C.byref(opts) if opts is not None else None, tok, C.c_float(w.s_token), role,
                  C.c_float(w.s_role), layers, proj, C.c_float(w.s_output),
                  C.byref(self.handle))
        del keep

    def embed(self, tokens: np.ndarray, attention_mask: np.ndarray,
              role_ids: np.ndarray | None = None) -> np.ndarray:
        return super().embed(tokens, attention_mask, role_ids)


class TinyEmbed:
    """The examples/embed.eos pipeline (gather -> matmul -> l2_normalize) with
    f16 weights resident on the device; ``embed(tokens)`` returns f16 [T, E]."""

    def __init__(self, rt: Runtime, token_embedding: np.ndarray, projection: np.ndarray):
        table = np.ascontiguousarray(token_embedding, dtype=np.float16)
        proj = np.ascontiguousarray(projection, dtype=np.float16)
        if table.ndim != 2 or proj.ndim != 2 or proj.shape[0] != table.shape[1]:
            raise ValueError("token_embedding [V, D] and projection [D, E] required")
        self.rt, self.edim = rt, proj.shape[1]
        self.handle = C.c_void_p()
        _lib.call("eoship_embed_bind", rt.handle, table.ctypes.data_as(C.c_void_p),
                  C.c_int32(table.shape[0]), C.c_int32(table.shape[1]),
                  proj.ctypes.data_as(C.c_void_p), C.c_int32(proj.shape[1]), C.byref(self.handle))

    def release(self) -> None:
        # After the runtime is closed the object cannot be released any more
        # (its stream is gone); the handle is only dropped.
        if self.handle and self.rt.handle:
            _lib.call("eoship_embed_release", self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def embed(self, tokens: np.ndarray) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        out = np.zeros((t.shape[0], self.edim), np.float16)
        _lib.call("eoship_embed_run", self.rt.handle, self.handle, t.ctypes.data_as(C.c_void_p),
                  C.c_int32(t.shape[0]), out.ctypes.data_as(C.c_void_p))
        return out

    def embed_device(self, d_tokens: DeviceBuffer, n: int, d_out: DeviceBuffer) -> None:
        _lib.call("eoship_embed_run_device", self.rt.handle, self.handle, d_tokens.ptr,
                  C.c_int32(n), d_out.ptr)
