"""MLL package reader and plan classifier (CPU: no kernel runs).

The C++ reader (eoship_mll_*) is checked against the pure-Python restatement
in oracle/mll_oracle.py and against the BLAKE3 section digests the shipped
default embedder package holds (written by the reference's exporter); the
BLAKE3 restatements against the published digest of the empty input and
each other. The plan interpreter (oracle/plan_oracle.py) is pinned against
the C restatement of the compact graph (oracle.compact_embed), which the
reference's tensor-op known answers pin (tests/test_compact_oracle.py)."""
import ctypes as C
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from eos_amd import _lib
from eos_amd._lib import EosHipError
from eos_amd.mll import MllPackage
from oracle import mll_oracle, plan_oracle
from oracle.blake3 import EMPTY_DIGEST, blake3
from tests import mll_synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "default_embedder")
SHIPPED = os.path.join(GOLDEN, "corkscrewdb-default-embedder.mll")


@pytest.fixture(scope="module")
def shipped_bytes():
    with open(SHIPPED, "rb") as f:
        return f.read()


def _lib_blake3(data: bytes) -> bytes:
    out = (C.c_uint8 * 32)()
    _lib.call("eoship_blake3", C.c_char_p(data) if data else None, C.c_uint64(len(data)), out)
    return bytes(out)


def test_blake3_known_answer_and_restatements_agree():
    assert blake3(b"").hex() == EMPTY_DIGEST
    assert _lib_blake3(b"").hex() == EMPTY_DIGEST
    rng = np.random.default_rng(0)
    # single block, block edges, chunk edges, 2^k chunk trees and ragged trees
    for n in [1, 63, 64, 65, 1023, 1024, 1025, 2048, 2049, 3072, 4096, 4097, 5 * 1024 + 7,
              8 * 1024, 9 * 1024 + 1, 31 * 1024 + 100]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert _lib_blake3(data) == blake3(data), n


def test_shipped_package_identity_and_digests(shipped_bytes):
    """The fixture is the reference's shipped package (manifest SHA-256), and
    both BLAKE3 restatements reproduce every section digest it stores."""
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        manifest = json.load(f)
    assert hashlib.sha256(shipped_bytes).hexdigest() == manifest["artifact"]["sha256"]
    assert len(shipped_bytes) == manifest["artifact"]["bytes"]
    pk = mll_oracle.read(shipped_bytes, digest=blake3)   # raises on any mismatch
    assert set(pk["sections"]) == {"HEAD", "STRG", "DIMS", "TYPE", "PARM", "ENTR", "BUFF", "KRNL",
                                   "MEMP", "TNSR", "SCHM", "XMTA"}
    for tag, s in pk["sections"].items():
        body = shipped_bytes[s["offset"]:s["offset"] + s["size"]]
        assert _lib_blake3(body) == s["digest"], tag


def test_reader_matches_python_restatement(shipped_bytes):
    pk = mll_oracle.read(shipped_bytes)
    with MllPackage(SHIPPED) as m:
        assert m.module_name == "eos-embed-v1" and m.module_version == "manta/v0alpha1"
        assert m.n_sections == len(pk["sections"]) and m.n_strings == len(pk["strings"])
        assert m.n_tensors == len(pk["tensors"]) == 7
        assert m.metadata() == pk["meta"]
        for name, t in pk["tensors"].items():
            got = m.tensor(name)
            assert got["kind"] == "q8" and got["storage_dtype"] == mll_oracle.DTYPE_Q8
            assert got["shape"] == t["shape"]
            assert np.float32(got["scale"]) == np.float32(t["scale"]) > 0
            np.testing.assert_array_equal(got["codes"], t["codes"])
            np.testing.assert_array_equal(got["values"], t["values"])
        assert m.section("STRG") == shipped_bytes[pk["sections"]["STRG"]["offset"]:][
            :pk["sections"]["STRG"]["size"]]
        with pytest.raises(EosHipError, match="XKBI"):
            m.section("XKBI")


def _open_bytes(data):
    return MllPackage(data)


@pytest.mark.parametrize("where", ["tnsr_payload", "xmta", "strg"])
def test_reader_rejects_corrupted_sections(shipped_bytes, where):
    pk = mll_oracle.read(shipped_bytes)
    s = {"tnsr_payload": pk["sections"]["TNSR"], "xmta": pk["sections"]["XMTA"],
         "strg": pk["sections"]["STRG"]}[where]
    bad = bytearray(shipped_bytes)
    bad[s["offset"] + s["size"] - 3] ^= 0x01
    with pytest.raises(EosHipError, match="BLAKE3 digest"):
        _open_bytes(bytes(bad))


def test_reader_rejects_bad_framing(shipped_bytes):
    with pytest.raises(EosHipError, match="not an MLL file"):
        _open_bytes(b"XLL\0" + shipped_bytes[4:])
    with pytest.raises(EosHipError, match="version"):
        _open_bytes(shipped_bytes[:5] + b"\x02" + shipped_bytes[6:])
    with pytest.raises(EosHipError, match="bytes"):
        _open_bytes(shipped_bytes[:-1])
    with pytest.raises(EosHipError, match="not an MLL file"):
        _open_bytes(b"MLL")


def _synth(masked=False, scale=None, tied=False, gain=1.0, **kw):
    layers = [dict(q="q1", k="k1", v="v1", o="o1", up="up1", down="down1")]
    layers.append(layers[0] if tied else dict(q="q2", k="k2", v="v2", o="o2", up="up2",
                                              down="down2"))
    names = ["token_embedding"] + sorted({p for L in layers for p in L.values()})
    w = mll_synth.weights(300, 128, 256, names, seed=5, gain=gain)
    art = mll_synth.encoder_artifact(layers, masked=masked, scale=scale)
    return art, w


def test_xkbi_is_never_read():
    """An XKBI section with a wrong digest and non-JSON bytes still opens (its
    bytes are neither hashed nor decoded); any other section with a wrong
    digest is refused; an unknown required section is refused, an unknown
    optional one is ignored."""
    art, w = _synth()
    xkbi = ("XKBI", b"\x7fELF not json \x00\x01", 0x22)
    data = mll_synth.package(art, w, extra_sections=[xkbi], bad_digest={"XKBI"})
    with MllPackage(data) as m:
        assert m.n_sections == 5
        with pytest.raises(EosHipError, match="never read"):
            m.section("XKBI")
    with pytest.raises(EosHipError, match="XMTA fails its BLAKE3"):
        MllPackage(mll_synth.package(art, w, bad_digest={"XMTA"}))
    with pytest.raises(EosHipError, match="required section ZZZZ"):
        MllPackage(mll_synth.package(art, w, extra_sections=[("ZZZZ", b"abc", 1)]))
    with MllPackage(mll_synth.package(art, w, extra_sections=[("ZZZZ", b"abc", 2)])) as m:
        assert m.n_sections == 5


def test_packed_q4_payloads_and_scale_policy():
    """Q4 payloads (offset-binary nibbles, low nibble first) decode as (nibble - 8)
    * scale; packed payloads without a scale must be all zero codes
    (decodeTensorEntry / requireAllZeroPackedPayload, runtime/weight_file.go:305-440)."""
    art, w = _synth()
    rng = np.random.default_rng(9)
    q4 = rng.integers(-8, 8, size=w["o1"][0].shape).astype(np.int8)
    w = dict(w)
    w["o1"] = (q4, 0.03)
    flat = (q4.reshape(-1).astype(np.int16) + 8).astype(np.uint8)
    packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8).tobytes()
    logical = {n: "q8" for n in w}
    logical["o1"] = "q4"
    data = mll_synth.package(art, w, logical=logical, payloads={"o1": (12, packed)})
    py = mll_oracle.read(data)
    with MllPackage(data) as m:
        t = m.tensor("o1")
        assert t["kind"] == "q4"
        np.testing.assert_array_equal(t["codes"], q4)
        np.testing.assert_array_equal(t["codes"], py["tensors"]["o1"]["codes"])
        np.testing.assert_array_equal(t["values"], q4.astype(np.float32) * np.float32(0.03))
    scales = {n: s for n, (_, s) in w.items()}
    scales["v1"] = 0.0
    with pytest.raises(EosHipError, match="no dequantization scale"):
        MllPackage(mll_synth.package(art, w, scales=scales, logical=logical,
                                     payloads={"o1": (12, packed)}))
    w["v1"] = (np.zeros_like(w["v1"][0]), 0.0)
    with MllPackage(mll_synth.package(art, w, scales=scales, logical=logical,
                                      payloads={"o1": (12, packed)})) as m:
        assert not m.tensor("v1")["codes"].any() and not m.tensor("v1")["values"].any()


def test_metadata_validation():
    art, w = _synth()
    scales = {n: s for n, (_, s) in w.items()}
    scales["q1"] = -1.0
    with pytest.raises(EosHipError, match="finite and non-negative"):
        MllPackage(mll_synth.package(art, w, scales=scales))


def test_classifier_on_shipped_package():
    with MllPackage(SHIPPED) as m:
        p = m.classify()
        assert p["route"] == "compact_embedder" and p["entry"] == "embed_pooled_batch"
        assert (p["layers"], p["distinct_layers"], p["model_dim"], p["heads"], p["hidden_dim"],
                p["vocab"], p["max_sequence"], p["output_dim"]) == (2, 1, 256, 1, 512, 16384,
                                                                   256, 256)
        assert p["options"] == {"rope": 0, "role": 0, "scaled_scores": 0, "attend_padding": 1}
        assert p["batched"] and p["steps"] == 41
        single = m.classify("embed_pooled")
        assert not single["batched"] and single["layers"] == 2
        with pytest.raises(EosHipError, match="unknown entrypoint"):
            m.classify("nope")


def test_classifier_variants_and_refusals():
    art, w = _synth(masked=True, scale="rsqrt_rhs_rows")
    with MllPackage(mll_synth.package(art, w)) as m:
        p = m.classify()
        assert p["options"] == {"rope": 0, "role": 0, "scaled_scores": 1, "attend_padding": 0}
        assert p["distinct_layers"] == 2 and (p["model_dim"], p["hidden_dim"]) == (128, 256)

    def steps_of(a):
        return a["steps"]

    def replace_kernel_op(a, kernel, op):
        for k in a["kernels"]:
            if k["name"] == kernel:
                k["body"][0]["op"] = op

    cases = [
        ("gelu op class changed", lambda a: replace_kernel_op(a, "gelu", "relu"), "op class \"relu\""),
        ("residual from the wrong value",
         lambda a: steps_of(a)[next(i for i, s in enumerate(a["steps"])
                                     if s.get("outputs") == ["res1"])].update(
             inputs=["attended1", "q1"]), "residual add"),
        ("no return", lambda a: a["steps"].pop(), "no return"),
        ("score scale not handled",
         lambda a: next(s for s in a["steps"] if s.get("outputs") == ["scores1"]).update(
             attributes={"scale": "rsqrt_lhs_rows"}), "scale \"rsqrt_lhs_rows\""),
        ("unknown step kind",
         lambda a: a["steps"].insert(3, {"entry": "embed_batch", "kind": "conv2d", "name": "c",
                                         "inputs": ["hidden"], "outputs": ["c"]}),
         "step kind \"conv2d\""),
    ]
    for label, fn, msg in cases:
        bad = mll_synth.mutate(art, fn)
        with MllPackage(mll_synth.package(bad, w)) as m:
            with pytest.raises(EosHipError, match="not handled|no return") as ei:
                m.classify()
            assert msg in str(ei.value), (label, str(ei.value))


def test_plan_interpreter_matches_c_restatement(shipped_bytes):
    """The plan run step by step (numpy) equals the C restatement of the same
    graph (no RoPE, no roles, unscaled scores, softmax over every position)
    on the shipped weights, for a padded batch and the single entry."""
    pk = mll_oracle.read(shipped_bytes)
    art = pk["meta"]["artifact"]
    params = {k: v["values"] for k, v in pk["tensors"].items()}
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 16384, (3, 48)).astype(np.int32)
    mask = np.ones((3, 48), np.int32)
    mask[1, 30:] = 0
    mask[2, 1:] = 0
    got = plan_oracle.run(art, params, "embed_pooled_batch",
                          {"tokens": ids, "attention_mask": mask})["result"]
    L = tuple(params[n] for n in ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_up", "projection"))
    want = oracle.compact_embed(params["token_embedding"], None, [L, L], ids, mask, None, 1,
                                flags=oracle.COMPACT_NO_ROPE | oracle.COMPACT_UNSCALED |
                                oracle.COMPACT_ATTEND_ALL)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    one = plan_oracle.run(art, params, "embed_pooled",
                          {"tokens": ids[1], "attention_mask": mask[1]})["result"]
    np.testing.assert_allclose(one, got[1], rtol=0, atol=1e-6)
    # Without the padding keys the result differs (the plan's softmax is unmasked).
    keyed = oracle.compact_embed(params["token_embedding"], None, [L, L], ids, mask, None, 1,
                                 flags=oracle.COMPACT_NO_ROPE | oracle.COMPACT_UNSCALED)
    assert np.abs(keyed[1] - got[1]).max() > 1e-4
    np.testing.assert_allclose(keyed[0], got[0], rtol=0, atol=2e-6)


def test_plan_interpreter_masked_scaled_variant():
    art, w = _synth(masked=True, scale="rsqrt_rhs_rows")
    params = mll_synth.dequantized(w)
    rng = np.random.default_rng(6)
    ids = rng.integers(0, 300, (2, 40)).astype(np.int32)
    mask = np.ones((2, 40), np.int32)
    mask[1, 17:] = 0
    got = plan_oracle.run(art, params, "embed_batch", {"tokens": ids, "attention_mask": mask})[
        "result"]
    layers = [tuple(params[f"{p}{i}"] for p in ("q", "k", "v", "o", "up", "down")) for i in (1, 2)]
    want = oracle.compact_embed(params["token_embedding"], None, layers, ids, mask, None, 1,
                                flags=oracle.COMPACT_NO_ROPE)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_retrieval_classifier_forms():
    """The retrieval plans of examples/*.eos as the compiler emits them: each
    form maps to its op, k, document source and output list."""
    rng = np.random.default_rng(0)
    codes = rng.integers(-8, 8, (50, 20)).astype(np.int8)
    want = {"score": (0, True, ["scores"]), "select": (3, True, ["top_scores"]),
            "rerank": (3, True, ["top_index", "top_scores"]),
            "retrieve": (3, True, ["top_index", "top_scores", "top_docs"]),
            "candidates": (3, False, ["top_ids", "top_scores", "top_docs"]),
            "packed": (3, False, ["pack"]), "batch": (3, False, ["top_ids", "top_scores",
                                                                "top_docs"])}
    from eos_amd.retrieval import plan_dict
    for form, (k, param, outs) in want.items():
        art = mll_synth.retrieval_artifact(form, "dot", 3)
        data = mll_synth.retrieval_package(art, codes if param else None, 0.05)
        with MllPackage(data) as m:
            p = _lib.EosHipRetrievalPlan()
            _lib.call("eoship_mll_classify_retrieval", m.handle, None, C.byref(p))
            d = plan_dict(p)
            assert (d["op"], d["k"], d["docs_param"], d["outputs"]) == ("dot", k, param, outs), form
            assert d["batched"] == (form == "batch")
            if param:
                assert (d["docs_rows"], d["dim"], d["docs_q4"]) == (50, 20, True)
            # The encoder classifier refuses a retrieval plan.
            with pytest.raises(EosHipError, match="not handled|no complete|inputs"):
                m.classify(form)
    bad = mll_synth.mutate(mll_synth.retrieval_artifact("candidates"),
                           lambda a: a["steps"].insert(1, {"entry": "candidates", "kind": "topk",
                                                          "name": "topk", "inputs": ["scores"],
                                                          "outputs": ["t2"],
                                                          "attributes": {"k": "0"}}))
    with MllPackage(mll_synth.retrieval_package(bad)) as m:
        with pytest.raises(EosHipError, match="topk limit"):
            _lib.call("eoship_mll_classify_retrieval", m.handle, None,
                      C.byref(_lib.EosHipRetrievalPlan()))


def _bert(layers=2, heads=4, hidden=128, inter=256):
    from eos_amd import datagen
    w = datagen.bert_q8_weights(layers, hidden, heads, inter, 300, 64, seed=41,
                                random_affine=True)
    return w, mll_synth.bert_tensors(w)


def test_bert_embedder_plans_classify():
    """The pretrained-BERT importer's module (one bert_embedder step and its
    return, runtime/pretrained_bert_importer.go:901-1009) classifies with
    the step's configuration; f32 dense weights are marked for per-channel
    quantization at bind, q8 payloads are used as stored."""
    w, t = _bert()
    art = mll_synth.bert_artifact(2, 4, eps=1e-7, pooling="cls")
    with MllPackage(mll_synth.bert_package(art, t)) as m:
        p = m.classify()
    assert p["route"] == "bert_embedder" and p["entry"] == "bert_embed"
    assert (p["layers"], p["model_dim"], p["heads"], p["hidden_dim"], p["vocab"],
            p["max_positions"], p["type_vocab"], p["output_dim"]) == (2, 128, 4, 256, 300, 64, 2,
                                                                      128)
    assert p["pooling"] == "cls" and p["ln_eps"] == 1e-7 and p["weights_quantized"]
    assert (p["token_input"], p["mask_input"], p["type_input"], p["output_name"]) == (
        "input_ids", "attention_mask", "token_type_ids", "embeddings")
    dense = [n for n in t if n.endswith("_weight") and "layernorm" not in n]
    art2 = mll_synth.bert_artifact(2, 4, attrs={})      # eps, act, pooling defaulted
    art2["steps"][0]["attributes"] = {"num_hidden_layers": "2", "num_attention_heads": "4"}
    with MllPackage(mll_synth.bert_package(art2, t, q8=tuple(dense))) as m:
        p = m.classify()
    assert p["pooling"] == "masked_mean" and p["ln_eps"] == 1e-12 and not p["weights_quantized"]


def test_bert_embedder_refusals():
    """What bertEmbedderConfigFromAttrs and BERTEmbedderReferenceWithPooling
    reject (runtime/backend/bert_embedder_ops.go:10-77, 101-152), and shapes
    outside the fused encoder, are refused with the step named."""
    w, t = _bert()

    def attrs(**kv):
        a = {"num_hidden_layers": "2", "num_attention_heads": "4", "epsilon": "1e-12",
             "hidden_act": "gelu", "pooling": "masked_mean"}
        a.update(kv)
        return mll_synth.bert_artifact(2, 4, attrs=a)

    cases = [
        (attrs(hidden_act="relu"), "unsupported hidden_act \"relu\""),
        (attrs(pooling="max"), "unsupported pooling \"max\""),
        (attrs(num_hidden_layers="two"), "num_hidden_layers \"two\" is invalid"),
        (attrs(num_hidden_layers="0"), "num_hidden_layers \"0\" is invalid"),
        (attrs(num_attention_heads="-4"), "num_attention_heads \"-4\" is invalid"),
        (attrs(epsilon="-1e-5"), "epsilon must be non-negative"),
        (attrs(epsilon="abc"), "epsilon \"abc\" is invalid"),
        (attrs(num_hidden_layers="3"), "expects 56 tensors for 3 layers, got 40"),
        (attrs(num_attention_heads="3"), "not a multiple of num_attention_heads"),
        (mll_synth.mutate(attrs(), lambda a: a["steps"].insert(
            1, {"entry": "bert_embed", "kind": "normalize", "name": "n", "inputs": ["embeddings"],
                "outputs": ["e2"]})), "beside a bert_embedder step"),
        (mll_synth.mutate(attrs(), lambda a: a["steps"].pop()), "no return step"),
    ]
    for art, msg in cases:
        with MllPackage(mll_synth.bert_package(art, t)) as m:
            with pytest.raises(EosHipError) as ei:
                m.classify()
            assert msg in str(ei.value), (msg, str(ei.value))
    # A layer tensor of the wrong shape, and one that is missing.
    bad = dict(t)
    bad["encoder_layer_1_intermediate_bias"] = np.zeros(100, np.float32)
    with MllPackage(mll_synth.bert_package(mll_synth.bert_artifact(2, 4), bad)) as m:
        with pytest.raises(EosHipError, match="layer 1 tensor shapes"):
            m.classify()
    del bad["encoder_layer_1_intermediate_bias"]
    with MllPackage(mll_synth.bert_package(mll_synth.bert_artifact(2, 4), bad)) as m:
        with pytest.raises(EosHipError, match="missing"):
            m.classify()
    # Head dim 8 (hidden 128, 16 heads) is outside the MFMA attention kernels
    # and inside the general-shape path: it classifies.
    with MllPackage(mll_synth.bert_package(attrs(num_attention_heads="16"), t)) as m:
        p = m.classify()
    assert p["route"] == "bert_embedder" and (p["model_dim"], p["heads"]) == (128, 16)
    # A head dim above 64 at a hidden width the MFMA kernels do not take is
    # outside both.
    w72, t72 = _bert(heads=1, hidden=72, inter=96)
    with MllPackage(mll_synth.bert_package(mll_synth.bert_artifact(2, 1), t72)) as m:
        with pytest.raises(EosHipError, match="hidden 72, head dim 72, intermediate 96 outside"):
            m.classify()
    # The golden fixture's model (hidden 16, 4 heads, intermediate 32)
    # classifies for the general-shape path.
    with MllPackage(mll_synth.bert_package(mll_synth.bert_artifact(2, 4),
                                           mll_synth.golden_bert_tensors())) as m:
        p = m.classify()
    assert p["route"] == "bert_embedder"
    assert (p["model_dim"], p["heads"], p["hidden_dim"], p["vocab"]) == (16, 4, 32, 17)


def test_long_names_are_refused():
    """Entry, input and param names of 64 bytes or more do not fit the plan's
    fixed fields: both classifiers refuse them (no truncated name reaches a
    bind)."""
    long = "q" * 70
    art = mll_synth.retrieval_artifact("candidates", "dot", 3)
    art = json.loads(json.dumps(art).replace('"query"', f'"{long}"'))
    with MllPackage(mll_synth.retrieval_package(art, None)) as m:
        with pytest.raises(EosHipError, match="64 bytes or more"):
            _lib.call("eoship_mll_classify_retrieval", m.handle, None,
                      C.byref(_lib.EosHipRetrievalPlan()))
    w, t = _bert()
    art = mll_synth.bert_artifact(2, 4)
    art = json.loads(json.dumps(art).replace('"input_ids"', '"' + "i" * 64 + '"'))
    with MllPackage(mll_synth.bert_package(art, t)) as m:
        with pytest.raises(EosHipError, match="64 bytes or more"):
            m.classify()
