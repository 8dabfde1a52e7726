"""Synthetic MLL packages for the reader and plan tests: the family-(a)
encoder plan in the shape the reference's sealed export writes
(artifact/eos/mll.go:112-330; the shipped default embedder's XMTA artifact),
with seeded q8 weights, and variants of its step list."""
from __future__ import annotations

import copy
import json

import numpy as np

from oracle import mll_oracle
from oracle.blake3 import blake3 as _py_blake3


def blake3(data: bytes) -> bytes:
    """Section digests of the synthetic packages: the library's BLAKE3 for
    bodies past 64 KiB (the pure-Python restatement takes minutes on the
    dense weights of a BERT package), else the Python one. Both are pinned
    to the specification and to each other in tests/test_mll.py."""
    if len(data) <= 65536:
        return _py_blake3(data)
    import ctypes as C
    from eos_amd import _lib
    out = (C.c_uint8 * 32)()
    _lib.call("eoship_blake3", C.c_char_p(data), C.c_uint64(len(data)), out)
    return bytes(out)


def _kernel(name, op, attrs=None):
    body = {"kind": "reduce", "name": "result", "op": op, "inputs": ["x"], "outputs": ["result"]}
    if attrs:
        body["attributes"] = attrs
    return {"name": name, "body": [body, {"kind": "return", "op": "return", "outputs": ["result"]}]}


def encoder_artifact(layers: list[dict], masked: bool = False, scale: str | None = None,
                     batched: bool = True) -> dict:
    """Plan of the embedding entry: layers is a list of parameter-name dicts
    {q, k, v, o, up, down}; masked uses masked_softmax(scores, mask); scale
    sets the score matmul's scale attribute."""
    entry = "embed_batch" if batched else "embed"
    shape = ["B", "T"] if batched else ["T"]
    steps = []

    def st(kind, name, ins, outs, kernel=None, attrs=None):
        s = {"entry": entry, "kind": kind, "name": name, "inputs": ins, "outputs": outs}
        if kernel:
            s["kernel"] = kernel
        if attrs:
            s["attributes"] = attrs
        steps.append(s)

    st("gather", "gather", ["token_embedding", "tokens"], ["hidden_q"])
    st("dequant", "dequant", ["hidden_q"], ["hidden"])
    deq = {}
    for L in layers:
        for p in L.values():
            if p not in deq:
                deq[p] = p + "_f"
                st("dequant", "dequant", [p], [deq[p]])
    x = "hidden"
    for i, L in enumerate(layers, 1):
        st("matmul", "matmul", [x, deq[L["q"]]], [f"q{i}"])
        st("matmul", "matmul", [x, deq[L["k"]]], [f"k{i}"])
        st("matmul", "matmul", [x, deq[L["v"]]], [f"v{i}"])
        st("transpose", "transpose", [f"k{i}"], [f"kt{i}"])
        st("matmul", "matmul", [f"q{i}", f"kt{i}"], [f"scores{i}"],
           attrs={"scale": scale} if scale else None)
        if masked:
            st("launch_kernel", "masked_softmax", [f"scores{i}", "attention_mask"], [f"probs{i}"],
               kernel="masked_softmax")
        else:
            st("launch_kernel", "softmax", [f"scores{i}"], [f"probs{i}"], kernel="softmax")
        st("matmul", "matmul", [f"probs{i}", f"v{i}"], [f"mixed{i}"])
        st("matmul", "matmul", [f"mixed{i}", deq[L["o"]]], [f"attended{i}"])
        st("launch_kernel", "binary_add", [f"attended{i}", x], [f"res{i}"], kernel="binary_add")
        st("launch_kernel", "layernorm", [f"res{i}"], [f"attn_hidden{i}"], kernel="layernorm")
        st("matmul", "matmul", [f"attn_hidden{i}", deq[L["up"]]], [f"ffn{i}"])
        st("launch_kernel", "gelu", [f"ffn{i}"], [f"act{i}"], kernel="gelu")
        st("matmul", "matmul", [f"act{i}", deq[L["down"]]], [f"proj{i}"])
        st("launch_kernel", "binary_add", [f"proj{i}", f"attn_hidden{i}"], [f"res2_{i}"],
           kernel="binary_add")
        st("launch_kernel", "layernorm", [f"res2_{i}"], [f"encoded{i}"], kernel="layernorm")
        x = f"encoded{i}"
    st("launch_kernel", "normalize", [x], ["normalized"], kernel="normalize")
    st("launch_kernel", "mean_pool", ["normalized", "attention_mask"], ["result"],
       kernel="mean_pool")
    steps.append({"entry": entry, "kind": "return", "outputs": ["result"]})
    params = []
    for name in ["token_embedding"] + sorted({p for L in layers for p in L.values()}):
        params.append({"name": name, "type": {"kind": "tensor", "tensor": {"dtype": "q8"}},
                       "binding": "weights/" + name})
    tens = lambda shp: {"kind": "tensor", "tensor": {"dtype": "i32", "shape": shp}}
    kernels = [_kernel("softmax", "softmax", {"axis": "-1"}), _kernel("binary_add", "binary_add",
               {"operator": "+"}), _kernel("layernorm", "layernorm"), _kernel("gelu", "gelu"),
               _kernel("normalize", "normalize"), _kernel("mean_pool", "mean_pool"),
               _kernel("masked_softmax", "masked_softmax")]
    return {
        "version": "manta/v0alpha1", "name": "synthetic-embedder", "params": params,
        "entry_points": [{"name": entry, "kind": "pipeline",
                          "inputs": [{"name": "tokens", "type": tens(shape)},
                                     {"name": "attention_mask", "type": tens(shape)}],
                          "outputs": [{"name": "result", "type": tens(["D"])}]}],
        "kernels": kernels, "steps": steps,
    }


def weights(vocab: int, dim: int, ffn: int, names: list[str], seed: int,
            gain: float = 1.0) -> dict:
    """Seeded int8 codes (about N(0, 40), clipped to +-127) and per-tensor
    scales giving weights of std gain / sqrt(fan in): name -> (codes, scale).
    Names starting with "up" are [dim, ffn], with "down" [ffn, dim], the
    token table [vocab, dim], the rest [dim, dim]."""
    rng = np.random.default_rng(seed)
    out = {}
    for n in names:
        if n == "token_embedding":
            shp, fan = (vocab, dim), 1.0
        elif n.startswith("up"):
            shp, fan = (dim, ffn), dim
        elif n.startswith("down"):
            shp, fan = (ffn, dim), ffn
        else:
            shp, fan = (dim, dim), dim
        codes = np.clip(np.rint(rng.normal(0.0, 40.0, size=shp)), -127, 127).astype(np.int8)
        scale = gain / np.sqrt(fan) / 40.0 * rng.uniform(0.8, 1.2)
        out[n] = (codes, float(np.float32(scale)))
    return out


def package(artifact: dict, w: dict, extra_sections=(), bad_digest=None, scales=None,
            max_sequence: int = 256, logical=None, payloads=None) -> bytes:
    """A sealed-profile container: STRG, TNSR (w as Q8 payloads unless
    payloads overrides name -> (dtype code, bytes)), XMTA, plus extra
    (tag, body, flags) sections."""
    names = list(w)
    strings = [""] + names
    entries = []
    for n in names:
        codes, _ = w[n]
        dt, payload = (mll_oracle.DTYPE_Q8, codes.tobytes())
        if payloads and n in payloads:
            dt, payload = payloads[n]
        entries.append((strings.index(n), dt, codes.shape, payload))
    meta = {
        "version": "manta/mll/v0alpha1", "module_name": artifact["name"],
        "module_version": "manta/v0alpha1", "artifact": artifact,
        "json_files": {"embedding_manifest": {
            "batch_entry": artifact["entry_points"][0]["name"], "token_input": "tokens",
            "mask_input": "attention_mask", "output_name": "result",
            "tokenizer": {"vocab_size": int(w["token_embedding"][0].shape[0]),
                          "max_sequence": max_sequence}}},
        "logical_tensor_dtypes": logical if logical is not None else {n: "q8" for n in names},
        "tensor_scales": scales if scales is not None else {n: w[n][1] for n in names},
    }
    secs = [("HEAD", b"\0" * 16, 1), ("STRG", mll_oracle.strg_body(strings), 1),
            ("TNSR", mll_oracle.tnsr_body(entries), 0x11),
            ("XMTA", json.dumps(meta).encode(), 0x22)]
    secs += list(extra_sections)
    return mll_oracle.write(secs, blake3, bad_digest=bad_digest)


def dequantized(w: dict) -> dict:
    return {n: c.astype(np.float32) * np.float32(s) for n, (c, s) in w.items()}


def mutate(artifact: dict, fn) -> dict:
    a = copy.deepcopy(artifact)
    fn(a)
    return a


def retrieval_artifact(form: str, op: str = "cosine", k: int = 2) -> dict:
    """The plans the reference's compiler emits for examples/*.eos
    (compiler/compiler.go:1767-1960): a launch_kernel of the score op class,
    topk with its k attribute, gathers (mode "batched" for the [Q, ...]
    forms), pack_candidates. form: score, select, rerank, retrieve
    (documents are the param "docs"), candidates, packed, batch (documents
    and candidate ids are inputs)."""
    entry = form
    batched = form == "batch"
    steps = []

    def st(kind, name, ins, outs, kernel=None, attrs=None):
        s = {"entry": entry, "kind": kind, "name": name, "inputs": ins, "outputs": outs}
        if kernel:
            s["kernel"] = kernel
        if attrs:
            s["attributes"] = attrs
        steps.append(s)

    tens = lambda dt, shp: {"kind": "tensor", "tensor": {"dtype": dt, "shape": shp}}
    inputs = [{"name": "query", "type": tens("f16", ["Q", "D"] if batched else ["D"])}]
    params = []
    if form in ("score", "select", "rerank", "retrieve"):
        params.append({"name": "docs", "type": tens("q4", ["N", "D"]), "binding": "weights/docs"})
    else:
        inputs.append({"name": "docs", "type": tens("q4", ["Q", "N", "D"] if batched else ["N", "D"])})
        inputs.append({"name": "candidate_ids", "type": tens("i64", ["Q", "N"] if batched else ["N"])})
    gm = {"mode": "batched"} if batched else None
    st("launch_kernel", op, ["query", "docs"], ["scores"], kernel=op)
    rets = []
    if form == "score":
        rets = ["scores"]
    else:
        st("topk", "topk", ["scores"], ["top"], attrs={"k": str(k)})
        if form == "select":
            st("gather", "gather", ["scores", "top"], ["sel"], attrs=gm)
            rets = ["sel"]
        elif form in ("rerank", "retrieve"):
            st("gather", "gather", ["scores", "top"], ["top_scores"])
            rets = ["top", "top_scores"]
            if form == "retrieve":
                st("gather", "gather", ["docs", "top"], ["top_docs"])
                rets.append("top_docs")
        else:
            st("gather", "gather", ["candidate_ids", "top"], ["top_candidate_ids"], attrs=gm)
            st("gather", "gather", ["scores", "top"], ["top_scores"], attrs=gm)
            st("gather", "gather", ["docs", "top"], ["top_docs"], attrs=gm)
            if form == "packed":
                st("pack_candidates", "pack_candidates",
                   ["top_candidate_ids", "top_scores", "top_docs"], ["pack"])
                rets = ["pack"]
            else:
                rets = ["top_candidate_ids", "top_scores", "top_docs"]
    steps.append({"entry": entry, "kind": "return", "outputs": rets})
    kernels = [{"name": op, "body": [{"kind": "reduce", "name": "result", "op": op,
                                      "inputs": ["query", "docs"], "outputs": ["result"]},
                                     {"kind": "return", "op": "return", "outputs": ["result"]}]}]
    return {"version": "manta/v0alpha1", "name": f"retrieval-{form}", "params": params,
            "entry_points": [{"name": entry, "kind": "pipeline", "inputs": inputs,
                              "outputs": [{"name": r, "type": tens("f32", ["K"])} for r in rets]}],
            "kernels": kernels, "steps": steps}


def retrieval_package(artifact: dict, docs_codes: np.ndarray | None = None,
                      docs_scale: float = 0.0) -> bytes:
    """A sealed-profile container for a retrieval artifact; docs_codes
    (int8 in -8..7, [N, D]) become the q4 param "docs" packed low nibble
    first."""
    strings, entries, scales, logical = [""], [], {}, {}
    if docs_codes is not None:
        flat = (docs_codes.reshape(-1).astype(np.int16) + 8).astype(np.uint8)
        if flat.size % 2:
            flat = np.concatenate([flat, np.array([8], np.uint8)])
        packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8).tobytes()
        strings.append("docs")
        entries.append((1, 12, docs_codes.shape, packed))
        scales["docs"] = docs_scale
        logical["docs"] = "q4"
    meta = {"version": "manta/mll/v0alpha1", "module_name": artifact["name"],
            "module_version": "manta/v0alpha1", "artifact": artifact,
            "logical_tensor_dtypes": logical, "tensor_scales": scales}
    secs = [("HEAD", b"\0" * 16, 1), ("STRG", mll_oracle.strg_body(strings), 1),
            ("TNSR", mll_oracle.tnsr_body(entries), 0x11),
            ("XMTA", json.dumps(meta).encode(), 0x22)]
    return mll_oracle.write(secs, blake3)


BERT_LAYER_ROLES = ["attention_query_weight", "attention_query_bias", "attention_key_weight",
                    "attention_key_bias", "attention_value_weight", "attention_value_bias",
                    "attention_output_weight", "attention_output_bias",
                    "attention_layernorm_weight", "attention_layernorm_bias",
                    "intermediate_weight", "intermediate_bias", "output_weight", "output_bias",
                    "output_layernorm_weight", "output_layernorm_bias"]
BERT_EMB_ROLES = ["token_embeddings", "position_embeddings", "token_type_embeddings",
                  "embedding_layernorm_weight", "embedding_layernorm_bias"]


def bert_artifact(layers: int, heads: int, eps: float = 1e-12, pooling: str = "masked_mean",
                  hidden_act: str = "gelu", attrs: dict | None = None) -> dict:
    """The module the pretrained-BERT importer builds
    (runtime/pretrained_bert_importer.go:901-1009): params for the five
    embedding tensors and 16 per layer, entry bert_embed (input_ids,
    attention_mask, token_type_ids -> embeddings), one bert_embedder step
    with the config attributes, then its return. attrs overrides the
    attribute map."""
    names = list(BERT_EMB_ROLES)
    for l in range(layers):
        names += [f"encoder_layer_{l}_{r}" for r in BERT_LAYER_ROLES]
    ids = {"kind": "tensor", "tensor": {"dtype": "i32", "shape": ["B", "T"]}}
    a = {"epsilon": repr(float(eps)), "hidden_act": hidden_act,
         "num_attention_heads": str(heads), "num_hidden_layers": str(layers),
         "pooling": pooling, "normalization": "l2"}
    if attrs is not None:
        a = attrs
    return {
        "version": "manta/v0alpha1", "name": "pretrained_bert_embedder",
        "params": [{"name": n, "type": {"kind": "tensor", "tensor": {"dtype": "f32"}},
                    "binding": n} for n in names],
        "entry_points": [{"name": "bert_embed", "kind": "pipeline",
                          "inputs": [{"name": "input_ids", "type": ids},
                                     {"name": "attention_mask", "type": ids},
                                     {"name": "token_type_ids", "type": ids}],
                          "outputs": [{"name": "embeddings",
                                       "type": {"kind": "tensor",
                                                "tensor": {"dtype": "f32", "shape": ["B", "H"]}}}]}],
        "steps": [{"entry": "bert_embed", "kind": "bert_embedder",
                   "name": "bert_embedder_reference",
                   "inputs": ["input_ids", "attention_mask", "token_type_ids"] + names,
                   "outputs": ["embeddings"], "attributes": a},
                  {"entry": "bert_embed", "kind": "return", "name": "return_embeddings",
                   "outputs": ["embeddings"]}],
    }


def bert_tensors(w) -> dict:
    """name -> f32 array of an EncoderWeights (datagen.bert_q8_weights) in the
    importer's roles, the dense weights dequantized (codes x per-channel
    scale) so that their per-channel int8 quantization returns the same codes."""
    out = {"token_embeddings": w.tok, "position_embeddings": w.pos,
           "token_type_embeddings": w.typ, "embedding_layernorm_weight": w.emb_gamma,
           "embedding_layernorm_bias": w.emb_beta}
    H = w.hidden
    for l, L in enumerate(w.layers):
        deq = L.dequantized()   # 16 tensors in the reference order
        q, k, v = deq[0], deq[2], deq[4]
        vals = [q, deq[1], k, deq[3], v, deq[5]] + list(deq[6:])
        assert q.shape == (H, H)
        for r, x in zip(BERT_LAYER_ROLES, vals):
            out[f"encoder_layer_{l}_{r}"] = np.asarray(x, np.float32)
    return out


def bert_package(artifact: dict, tensors: dict, q8: tuple = (), q4: tuple = ()) -> bytes:
    """A sealed-profile container holding `tensors` (name -> f32 array) as
    f32 payloads, except the names in q8 / q4, stored as the reference's
    per-tensor packed Q8 / Q4 (packQuantizedTensorStorage,
    runtime/mll_export.go:897-975) with their tensor_scales. The storage
    dtype byte of an f32 payload is not fixed by any shipped package; the
    reader goes by the logical dtype and the payload size."""
    from eos_amd.encoder import quantize_per_tensor
    names = list(tensors)
    strings = [""] + names
    entries, scales, logical = [], {}, {}
    for n in names:
        x = np.ascontiguousarray(tensors[n], np.float32)
        if n in q8 or n in q4:
            bits = 8 if n in q8 else 4
            codes, sc = quantize_per_tensor(x, bits)
            scales[n] = float(sc)
            if bits == 8:
                entries.append((strings.index(n), mll_oracle.DTYPE_Q8, x.shape, codes.tobytes()))
                logical[n] = "q8"
            else:
                flat = (codes.reshape(-1).astype(np.int16) + 8).astype(np.uint8)
                if flat.size % 2:
                    flat = np.concatenate([flat, np.array([8], np.uint8)])
                packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8).tobytes()
                entries.append((strings.index(n), 12, x.shape, packed))
                logical[n] = "q4"
        else:
            entries.append((strings.index(n), 1, x.shape, x.tobytes()))
            logical[n] = "f32"
    meta = {"version": "manta/mll/v0alpha1", "module_name": artifact["name"],
            "module_version": "manta/v0alpha1", "artifact": artifact,
            "logical_tensor_dtypes": logical, "tensor_scales": scales}
    secs = [("HEAD", b"\0" * 16, 1), ("STRG", mll_oracle.strg_body(strings), 1),
            ("TNSR", mll_oracle.tnsr_body(entries), 0x11),
            ("XMTA", json.dumps(meta).encode(), 0x22)]
    return mll_oracle.write(secs, blake3)


def golden_bert_tensors() -> dict:
    """The reference's BERT golden fixture (tests/golden/bert_tiny, hidden 16,
    4 heads, intermediate 32, 2 layers) in the importer's roles (f32)."""
    import os
    from safetensors.numpy import load_file
    g = load_file(os.path.join(os.path.dirname(__file__), "golden", "bert_tiny",
                               "model.safetensors"))
    gt = {"token_embeddings": g["embeddings.word_embeddings.weight"],
          "position_embeddings": g["embeddings.position_embeddings.weight"],
          "token_type_embeddings": g["embeddings.token_type_embeddings.weight"],
          "embedding_layernorm_weight": g["embeddings.LayerNorm.weight"],
          "embedding_layernorm_bias": g["embeddings.LayerNorm.bias"]}
    hf = ["attention.self.query.weight", "attention.self.query.bias", "attention.self.key.weight",
          "attention.self.key.bias", "attention.self.value.weight", "attention.self.value.bias",
          "attention.output.dense.weight", "attention.output.dense.bias",
          "attention.output.LayerNorm.weight", "attention.output.LayerNorm.bias",
          "intermediate.dense.weight", "intermediate.dense.bias", "output.dense.weight",
          "output.dense.bias", "output.LayerNorm.weight", "output.LayerNorm.bias"]
    for l in range(2):
        for role, name in zip(BERT_LAYER_ROLES, hf):
            gt[f"encoder_layer_{l}_{role}"] = g[f"encoder.layer.{l}.{name}"]
    return gt
