"""GPU parity of the encoder bound from MLL packages (eoship_encoder_bind_mll)
against the plan run step by step on the CPU (oracle/plan_oracle.py).

Bar (the benchmark's north star): per sequence, cosine >= 0.9999 and max-abs error
<= 2e-2 between the GPU embedding and the oracle's, both from the same
dequantized q8 weights."""
import os

import numpy as np
import pytest

from eos_amd._lib import EosHipError
from eos_amd.mll import MllEncoder, MllPackage
from oracle import mll_oracle, plan_oracle
from tests import mll_synth

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
ABS_MAX = 2e-2
SHIPPED = os.path.join(os.path.dirname(__file__), "golden", "default_embedder",
                       "corkscrewdb-default-embedder.mll")


def _case(name):
    print(f"[case] {name}", flush=True)


def _check(got, want):
    n = np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1)
    live = n > 0
    cos = np.sum(got * want, axis=1)[live] / n[live]
    err = np.max(np.abs(got - want))
    print(f"  min cos {cos.min() if live.any() else 1.0:.8f}  max abs {err:.3e}", flush=True)
    if live.any():
        assert cos.min() >= COS_MIN
    assert err <= ABS_MAX
    np.testing.assert_array_equal(got[~live], want[~live])


@pytest.fixture(scope="module")
def shipped():
    with open(SHIPPED, "rb") as f:
        data = f.read()
    pk = mll_oracle.read(data)
    params = {k: v["values"] for k, v in pk["tensors"].items()}
    return data, pk["meta"]["artifact"], params


def _ragged(batch, tokens, vocab, lengths, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(4, vocab, (batch, tokens)).astype(np.int32)
    mask = np.zeros((batch, tokens), np.int32)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1
        ids[b, n:] = 0          # pad id
    return ids, mask


def test_shipped_package_padded_batch_as_plan(rt, shipped):
    """The [B, T] entry run as given (softmax over every position, padding
    included; the mask selects the pooled rows), as ExecuteSymbolic runs it."""
    _case("shipped package, plan semantics, padded batch")
    data, art, params = shipped
    enc = MllEncoder(rt, MllPackage(data))
    assert enc.plan["options"]["attend_padding"] == 1 and enc.out_dim == 256
    lengths = [256, 1, 17, 100, 255, 64, 128, 200]
    ids, mask = _ragged(8, 256, 16384, lengths, seed=21)
    got = enc.embed(ids, mask)
    want = plan_oracle.run(art, params, "embed_pooled_batch",
                           {"tokens": ids, "attention_mask": mask})["result"]
    _check(got, want)
    enc.release()


def test_shipped_package_length_grouped(rt, shipped):
    """attend_padding 0: each sequence attends only its own tokens, which is
    what the reference's EmbeddingModel returns for a ragged batch (it runs
    each length group without padding): checked against the plan run on each
    sequence alone at its own length (the single-sequence entry)."""
    _case("shipped package, length-grouped batch")
    data, art, params = shipped
    enc = MllEncoder(rt, MllPackage(data), attend_padding=0)
    lengths = [3, 256, 77, 1, 130, 31]
    ids, mask = _ragged(6, 256, 16384, lengths, seed=22)
    got = enc.embed(ids, mask)
    want = np.stack([plan_oracle.run(art, params, "embed_pooled",
                                     {"tokens": ids[b, :n], "attention_mask": mask[b, :n]})[
        "result"] for b, n in enumerate(lengths)])
    _check(got, want)
    enc.release()


def test_shipped_package_single_entry_and_errors(rt, shipped):
    _case("shipped package, single entry, id and length errors")
    data, art, params = shipped
    pkg = MllPackage(data)
    enc = MllEncoder(rt, pkg, entry="embed_pooled")
    ids, mask = _ragged(1, 200, 16384, [200], seed=23)
    got = enc.embed(ids, mask)
    want = plan_oracle.run(art, params, "embed_pooled",
                           {"tokens": ids[0], "attention_mask": mask[0]})["result"][None]
    _check(got, want)
    # Padding ids are gathered too under the plan's semantics: out of range is an error.
    ids2, mask2 = _ragged(2, 64, 16384, [64, 10], seed=24)
    ids2[1, 40] = 16384
    with pytest.raises(EosHipError, match="out of range"):
        enc.embed(ids2, mask2)
    with pytest.raises(EosHipError, match="position"):
        enc.embed(np.zeros((1, 257), np.int32), np.ones((1, 257), np.int32))
    enc.release()


@pytest.mark.parametrize("masked,scale,tied", [(True, "rsqrt_rhs_rows", False),
                                               (False, None, True), (True, None, False)])
def test_synthetic_plans(rt, masked, scale, tied):
    """Variants the classifier routes: masked_softmax (keys by mask) and the
    rsqrt_rhs_rows score scale, tied or untied layers, D = 128 (head dim
    128), FFN 256, with O(10)-logit attention."""
    _case(f"synthetic plan masked={masked} scale={scale} tied={tied}")
    layers = [dict(q="q1", k="k1", v="v1", o="o1", up="up1", down="down1")]
    layers.append(layers[0] if tied else dict(q="q2", k="k2", v="v2", o="o2", up="up2",
                                              down="down2"))
    names = ["token_embedding"] + sorted({p for L in layers for p in L.values()})
    w = mll_synth.weights(300, 128, 256, names, seed=31 + tied)
    art = mll_synth.encoder_artifact(layers, masked=masked, scale=scale)
    data = mll_synth.package(art, w, max_sequence=160)
    enc = MllEncoder(rt, MllPackage(data))
    assert enc.plan["options"]["attend_padding"] == (0 if masked else 1)
    assert enc.plan["distinct_layers"] == (1 if tied else 2)
    lengths = [160, 1, 33, 64, 65, 159, 2]
    ids, mask = _ragged(7, 160, 300, lengths, seed=33)
    got = enc.embed(ids, mask)
    want = plan_oracle.run(art, mll_synth.dequantized(w), "embed_batch",
                           {"tokens": ids, "attention_mask": mask})["result"]
    _check(got, want)
    enc.release()


def _bert_oracle_layers(pkg, layers, requantize):
    """The 16 f32 tensors per layer the GPU computes with: the package's
    values (q8 payloads: code x tensor scale), with f32 dense weights
    quantized per output channel as the bind does."""
    from eos_amd.encoder import quantize_per_channel
    out = []
    for l in range(layers):
        row = []
        for k, role in enumerate(mll_synth.BERT_LAYER_ROLES):
            t = pkg.tensor(f"encoder_layer_{l}_{role}")
            v = np.asarray(t["values"], np.float32)
            if k in (0, 2, 4, 6, 10, 12) and t["kind"] == "f32" and requantize:
                c, s = quantize_per_channel(v)
                v = c.astype(np.float32) * s[:, None]
            row.append(v)
        out.append(row)
    return out


@pytest.mark.parametrize("pooling", ["masked_mean", "cls"])
@pytest.mark.parametrize("storage", ["f32", "q8"])
def test_bert_embedder_package(rt, pooling, storage):
    """A bert_embedder package (the pretrained-BERT importer's module) bound
    through eoship_encoder_bind_mll embeds within the contract of
    oracle.bert_embed on the weights the GPU computes with (f32 dense
    weights quantized per output channel at bind; q8 payloads as stored),
    for both poolings; ragged lengths, token types, position 0 masked in one
    sequence (CLS still reads it) and a sequence with no active position."""
    import oracle
    from eos_amd import datagen
    _case(f"bert_embedder package {storage} {pooling}")
    L, H, heads, F = 2, 384, 12, 1536
    w = datagen.bert_q8_weights(L, H, heads, F, 3000, 256, seed=57, random_affine=True)
    t = mll_synth.bert_tensors(w)
    dense = tuple(n for n in t if n.endswith("_weight") and "layernorm" not in n
                  and n.startswith("encoder_layer_"))
    art = mll_synth.bert_artifact(L, heads, eps=1e-12, pooling=pooling)
    pkg = MllPackage(mll_synth.bert_package(art, t, q8=dense if storage == "q8" else ()))
    enc = MllEncoder(rt, pkg)
    assert enc.plan["route"] == "bert_embedder" and enc.plan["pooling"] == pooling
    assert enc.plan["weights_quantized"] == (storage == "f32")
    ids, mask = _ragged(7, 200, 3000, [200, 17, 1, 120, 0, 64, 199], 58)
    mask[3, 0] = 0                       # position 0 masked
    mask[5, 10:20] = 0                   # a hole
    rng = np.random.default_rng(59)
    types = rng.integers(0, 2, ids.shape).astype(np.int32)
    got = enc.embed(ids, mask, types)
    layers = _bert_oracle_layers(pkg, L, requantize=True)
    want = oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta, layers, ids, mask,
                             types, heads, 1e-12, pooling=pooling)
    if pooling == "masked_mean":
        assert np.all(got[4] == 0) and np.all(want[4] == 0)
    else:
        assert np.all(np.isfinite(got)) and abs(np.linalg.norm(got[4]) - 1) < 1e-5
    _check(got, want)
    enc.release()
    pkg.close()


@pytest.mark.parametrize("pooling", ["masked_mean", "cls"])
def test_bert_embedder_golden_fixture(rt, pooling):
    """The reference's own BERT golden fixture (hidden 16, 4 heads of dim 4,
    intermediate 32: runtime/testdata/pretrained_bert_golden/) as a
    bert_embedder package, bound through eoship_encoder_bind_mll (f32 dense
    weights quantized per output channel at bind) and run by the
    general-shape kernels: equal to oracle.bert_embed on the weights the GPU
    computes with to f32 rounding, and within the contract of golden.json's
    embeddings (masked mean pooling, the fixture's own)."""
    import json
    import oracle
    _case(f"bert golden fixture on the GPU, {pooling}")
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "bert_tiny",
                                    "golden.json")))
    t = mll_synth.golden_bert_tensors()
    pkg = MllPackage(mll_synth.bert_package(mll_synth.bert_artifact(2, 4, pooling=pooling), t))
    enc = MllEncoder(rt, pkg)
    assert enc.plan["route"] == "bert_embedder" and enc.plan["model_dim"] == 16
    n, T = len(g["texts"]), g["max_length"]
    ids = np.array(g["input_ids"], np.int32).reshape(n, T)
    mask = np.array(g["attention_mask"], np.int32).reshape(n, T)
    types = np.array(g["token_type_ids"], np.int32).reshape(n, T)
    got = enc.embed(ids, mask, types)
    layers = _bert_oracle_layers(pkg, 2, requantize=True)
    want = oracle.bert_embed(t["token_embeddings"], t["position_embeddings"],
                             t["token_type_embeddings"], t["embedding_layernorm_weight"],
                             t["embedding_layernorm_bias"], layers, ids, mask, types, 4, 1e-12,
                             pooling=pooling)
    err = float(np.max(np.abs(got - want)))
    print(f"  vs oracle on the bound weights: max abs {err:.3e}", flush=True)
    assert err <= 1e-5
    if pooling == "masked_mean":
        _check(got, np.array(g["embeddings"], np.float32))
    enc.release()
    pkg.close()


def test_bert_embedder_package_refuses_attend_padding(rt):
    _case("bert_embedder package attend_padding refusal")
    from eos_amd import datagen
    w = datagen.bert_q8_weights(1, 128, 4, 256, 100, 32, seed=3)
    pkg = MllPackage(mll_synth.bert_package(mll_synth.bert_artifact(1, 4), mll_synth.bert_tensors(w)))
    with pytest.raises(EosHipError, match="attend_padding 1"):
        MllEncoder(rt, pkg, attend_padding=1)
    pkg.close()
