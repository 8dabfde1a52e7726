"""Host side of the MLL package reader and the plan binding (libeoship).

``MllPackage`` opens a package through ``eoship_mll_open`` (container,
BLAKE3 section digests, STRG, TNSR, XMTA metadata; the XKBI kernel images
are never read) and gives access to its sections, tensors and metadata.
``MllPackage.classify`` matches an entry's plan against the fused encoder
graph (``eoship_mll_classify``) and ``MllEncoder`` binds it
(``eoship_encoder_bind_mll``). Reference counterparts: DecodeMLL / ReadFile
(artifact/eos/mll.go:332-420), decodeWeightFileFromMLLReader and
decodeTensorEntry (runtime/weight_file.go:248-415), ExecuteSymbolic
(runtime/backend/symbolic.go:17-172) for the embedding entries.
"""
from __future__ import annotations

import ctypes as C
import json
import os

import numpy as np

from . import _lib
from .encoder import Encoder
from .runtime import Runtime

KIND_NAMES = {_lib_kind: name for _lib_kind, name in
              ((1, "q8"), (2, "q4"), (3, "f32"), (4, "f16"), (5, "i32"), (6, "i64"))}


class MllPackage:
    """A parsed, digest-verified MLL package (the library keeps a copy of the bytes)."""

    def __init__(self, source: str | bytes | os.PathLike):
        if isinstance(source, (bytes, bytearray, memoryview)):
            data = bytes(source)
        else:
            with open(source, "rb") as f:
                data = f.read()
        buf = (C.c_uint8 * len(data)).from_buffer_copy(data) if data else (C.c_uint8 * 1)()
        self.handle = C.c_void_p()
        _lib.call("eoship_mll_open", C.cast(buf, C.c_void_p), C.c_uint64(len(data)),
                  C.byref(self.handle))
        info = _lib.EosHipMllInfo()
        _lib.call("eoship_mll_info", self.handle, C.byref(info))
        self.profile = info.profile
        self.n_sections = info.sections
        self.n_strings = info.strings
        self.n_tensors = info.tensors
        self.has_metadata = bool(info.has_metadata)
        self.module_name = info.module_name.decode()
        self.module_version = info.module_version.decode()

    def close(self) -> None:
        if self.handle:
            _lib.load().eoship_mll_close(self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def section(self, tag: str) -> bytes:
        body, size = C.c_void_p(), C.c_uint64()
        _lib.call("eoship_mll_section", self.handle, tag.encode(), C.byref(body), C.byref(size))
        return C.string_at(body, size.value) if size.value else b""

    def metadata(self) -> dict:
        """The XMTA document (MLLMetadata)."""
        return json.loads(self.section("XMTA"))

    def tensor(self, key: int | str) -> dict:
        """{name, kind, storage_dtype, shape, scale, payload (bytes), codes
        (int8 for q8/q4), values (dequantized f32 as the reference decodes)}."""
        t = _lib.EosHipMllTensor()
        if isinstance(key, str):
            _lib.call("eoship_mll_tensor", self.handle, C.c_int64(-1), key.encode(), C.byref(t))
        else:
            _lib.call("eoship_mll_tensor", self.handle, C.c_int64(key), None, C.byref(t))
        shape = tuple(int(t.dims[i]) for i in range(t.rank))
        payload = C.string_at(t.data, t.bytes) if t.bytes else b""
        kind = KIND_NAMES[t.kind]
        out = {"name": t.name.decode(), "kind": kind, "storage_dtype": t.storage_dtype,
               "shape": shape, "scale": float(t.scale), "payload": payload}
        n = int(t.elements)
        if kind == "q8":
            out["codes"] = np.frombuffer(payload, np.int8).reshape(shape)
        elif kind == "q4":
            nib = np.frombuffer(payload, np.uint8)
            both = np.stack([nib & 0xF, nib >> 4], axis=1).reshape(-1)[:n]
            out["codes"] = (both.astype(np.int16) - 8).astype(np.int8).reshape(shape)
        if "codes" in out:
            sc = np.float32(t.scale)
            out["values"] = (out["codes"].astype(np.float32) * sc if sc > 0
                             else np.zeros(shape, np.float32))
        elif kind == "f32":
            out["values"] = np.frombuffer(payload, "<f4").reshape(shape)
        elif kind in ("i32", "i64"):
            out["values"] = np.frombuffer(payload, "<i4" if kind == "i32" else "<i8").reshape(shape)
        return out

    def tensor_names(self) -> list[str]:
        return [self.tensor(i)["name"] for i in range(self.n_tensors)]

    def classify(self, entry: str | None = None) -> dict:
        """The plan route of an entry (raises EosHipError "not handled ..." otherwise)."""
        plan = _lib.EosHipMllPlan()
        _lib.call("eoship_mll_classify", self.handle, entry.encode() if entry else None,
                  C.byref(plan))
        return plan_dict(plan)


ROUTES = {1: "compact_embedder", 2: "bert_embedder"}


def plan_dict(p) -> dict:
    d = {
        "route": ROUTES.get(p.route, p.route),
        "layers": p.layers, "distinct_layers": p.distinct_layers, "model_dim": p.model_dim,
        "heads": p.heads, "hidden_dim": p.hidden_dim, "vocab": p.vocab,
        "max_sequence": p.max_sequence, "output_dim": p.output_dim, "batched": bool(p.batched),
        "steps": p.steps,
        "options": {"rope": p.options.rope, "role": p.options.role,
                    "scaled_scores": p.options.scaled_scores,
                    "attend_padding": p.options.attend_padding},
        "entry": p.entry.decode(), "token_input": p.token_input.decode(),
        "mask_input": p.mask_input.decode(), "output_name": p.output_name.decode(),
    }
    if p.route == 2:
        d.update({"pooling": "cls" if p.pooling == 1 else "masked_mean",
                  "type_vocab": p.type_vocab, "ln_eps": p.ln_eps,
                  "weights_quantized": bool(p.weights_quantized),
                  "type_input": p.type_input.decode(), "max_positions": p.max_sequence})
    return d


class MllEncoder(Encoder):
    """An embedding entry of an MLL package bound to the fused encoder.
    ``embed(tokens, mask[, token_type_ids])`` takes [batch, tokens] i32 arrays
    and returns [batch, output_dim] f32. A bert_embedder entry (route
    "bert_embedder") runs the fused BERT encoder with the step's pooling and
    takes token type ids (None: all 0); a compact-family entry ignores them.

    attend_padding: -1 runs the plan's own softmax semantics (the [B, T]
    entry as given: padding positions are keys and queries when the plan's
    softmax is unmasked); 0 attends only each sequence's mask != 0 positions,
    which is what the reference's EmbeddingModel returns for ragged batches
    (it groups them by length, runtime/embedding_model.go:689-691)."""

    def __init__(self, rt: Runtime, pkg: MllPackage, entry: str | None = None,
                 attend_padding: int = -1):
        self.rt = rt
        self.handle = C.c_void_p()
        plan = _lib.EosHipMllPlan()
        _lib.call("eoship_encoder_bind_mll", rt.handle, pkg.handle,
                  entry.encode() if entry else None, C.c_int32(attend_padding),
                  C.byref(self.handle), C.byref(plan))
        self.plan = plan_dict(plan)
        self.out_dim = self.plan["output_dim"]

    def embed(self, tokens: np.ndarray, attention_mask: np.ndarray,
              token_type_ids: np.ndarray | None = None) -> np.ndarray:
        types = token_type_ids if self.plan["route"] == "bert_embedder" else None
        return super().embed(tokens, attention_mask, types)
