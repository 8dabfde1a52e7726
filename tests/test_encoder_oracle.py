"""Pins the encoder CPU oracle (oracle/encoder_oracle.c): the reference's own
BERT golden fixture (a from-scratch HF BertModel with committed weights and
expected embeddings, runtime/testdata/pretrained_bert_golden/, gate from
runtime/pretrained_bert_golden_parity_test.go:99-103), the tiny embed known
answer (runtime/runtime_test.go:616-686, weights :1911-1922), and independent
numpy f64 forms of each piece. CPU only."""
import json
import math
import os

import numpy as np
import pytest

import oracle
from eos_amd import datagen

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bert_tiny")


def _golden():
    from safetensors.numpy import load_file
    t = load_file(os.path.join(GOLDEN, "model.safetensors"))
    g = json.load(open(os.path.join(GOLDEN, "golden.json")))
    cfg = json.load(open(os.path.join(GOLDEN, "config.json")))
    return t, g, cfg


def _layers_from_hf(t, n):
    out = []
    for i in range(n):
        p = f"encoder.layer.{i}."
        out.append([t[p + "attention.self.query.weight"], t[p + "attention.self.query.bias"],
                    t[p + "attention.self.key.weight"], t[p + "attention.self.key.bias"],
                    t[p + "attention.self.value.weight"], t[p + "attention.self.value.bias"],
                    t[p + "attention.output.dense.weight"], t[p + "attention.output.dense.bias"],
                    t[p + "attention.output.LayerNorm.weight"], t[p + "attention.output.LayerNorm.bias"],
                    t[p + "intermediate.dense.weight"], t[p + "intermediate.dense.bias"],
                    t[p + "output.dense.weight"], t[p + "output.dense.bias"],
                    t[p + "output.LayerNorm.weight"], t[p + "output.LayerNorm.bias"]])
    return out


def test_bert_golden_fixture():
    t, g, cfg = _golden()
    L = max(int(k.split(".")[2]) for k in t if k.startswith("encoder.layer.")) + 1
    n, T = len(g["texts"]), g["max_length"]
    ids = np.array(g["input_ids"], np.int32).reshape(n, T)
    mask = np.array(g["attention_mask"], np.int32).reshape(n, T)
    types = np.array(g["token_type_ids"], np.int32).reshape(n, T)
    out = oracle.bert_embed(t["embeddings.word_embeddings.weight"],
                            t["embeddings.position_embeddings.weight"],
                            t["embeddings.token_type_embeddings.weight"],
                            t["embeddings.LayerNorm.weight"], t["embeddings.LayerNorm.bias"],
                            _layers_from_hf(t, L), ids, mask, types, cfg["num_attention_heads"],
                            cfg["layer_norm_eps"])
    want = np.array(g["embeddings"], np.float64)
    cos = np.sum(out * want, axis=1) / (np.linalg.norm(out, axis=1) * np.linalg.norm(want, axis=1))
    assert cos.min() >= 0.9999 and np.max(np.abs(out - want)) <= 2e-3
    # the restatement is far inside the reference gate
    assert np.max(np.abs(out - want)) < 1e-5


def test_tiny_embed_known_answer():
    table = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    proj = np.eye(2, dtype=np.float32)
    out = oracle.tiny_embed(table, proj, np.array([0, 2], np.int32))
    np.testing.assert_allclose(out, [[1, 0], [0.70710677, 0.70710677]], rtol=0, atol=1e-7)


def test_dense_hf_matches_f64():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 13)).astype(np.float32)
    w = rng.standard_normal((5, 13)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    want = (x.astype(np.float64) @ w.astype(np.float64).T + b).astype(np.float32)
    np.testing.assert_array_equal(oracle.dense_hf(x, w, b), want)


def _attn_f64(q, k, v, mask, heads):
    B, T = mask.shape
    H = q.shape[1]
    hd = H // heads
    out = np.zeros((B * T, H))
    for b in range(B):
        act = np.nonzero(mask[b])[0]
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            Q = q[b * T:(b + 1) * T, sl].astype(np.float64)
            K = k[b * T + act, sl].astype(np.float64)
            V = v[b * T + act, sl].astype(np.float64)
            if len(act) == 0:
                continue
            lg = Q @ K.T / math.sqrt(hd)
            p = np.exp(lg - lg.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[b * T:(b + 1) * T, sl] = p @ V
    return out


def test_attention_matches_f64_and_masks():
    rng = np.random.default_rng(1)
    B, T, H, heads = 3, 9, 16, 4
    q, k, v = (rng.standard_normal((B * T, H)).astype(np.float32) for _ in range(3))
    mask = np.ones((B, T), np.int32)
    mask[0, 5:] = 0
    mask[1, :] = 0  # no active key: context stays zero
    mask[2, 2] = 0  # a hole
    got = oracle.bert_attention(q, k, v, mask, heads)
    np.testing.assert_allclose(got, _attn_f64(q, k, v, mask, heads), rtol=0, atol=2e-6)
    assert np.all(got[T:2 * T] == 0)


def test_pool_and_normalize_edge_cases():
    h = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
    mask = np.array([[1, 0, 1], [0, 0, 0]], np.int32)
    p = oracle.mean_pool_masked(h, mask)
    np.testing.assert_array_equal(p[0], (h[0, 0] + h[0, 2]) * np.float32(0.5))
    np.testing.assert_array_equal(p[1], 0)
    n = oracle.normalize_rows(np.array([[3, 4], [0, 0]], np.float32))
    np.testing.assert_allclose(n, [[0.6, 0.8], [0, 0]], rtol=0, atol=1e-7)


def test_quantize_per_channel_grid():
    w = np.array([[0.5, -1.0, 0.25], [0.0, 0.0, 0.0]], np.float32)
    from eos_amd.encoder import quantize_per_channel
    c, s = quantize_per_channel(w)
    assert s[0] == np.float32(1.0 / 127) and s[1] == 0
    np.testing.assert_array_equal(c[0], [64, -127, 32])
    np.testing.assert_array_equal(c[1], 0)


def test_encoder_batch_masks():
    ids, mask, lens = datagen.encoder_batch(64, 512, 30522, 32, 512, 8, 9)
    assert lens.min() >= 32 and lens.max() <= 512
    np.testing.assert_array_equal(mask.sum(axis=1), lens)
    assert ids.max() < 30522 and ids.min() >= 0


def test_cls_pooling_is_position_zero_of_the_pinned_hidden_states():
    """CLS pooling (clsPoolTensor, bert_embedder_ops.go:183-196): the golden
    model's hidden states give the golden masked-mean embeddings through an
    independent numpy mean + f64 L2 (which ties them to the fixture), and
    oracle.bert_embed(pooling="cls") equals position 0 of those states,
    normalized, whatever the mask says at position 0. A sequence whose only
    active position is 0 pools identically both ways."""
    t, g, cfg = _golden()
    L = max(int(k.split(".")[2]) for k in t if k.startswith("encoder.layer.")) + 1
    n, T = len(g["texts"]), g["max_length"]
    ids = np.array(g["input_ids"], np.int32).reshape(n, T)
    mask = np.array(g["attention_mask"], np.int32).reshape(n, T)
    types = np.array(g["token_type_ids"], np.int32).reshape(n, T)
    args = (t["embeddings.word_embeddings.weight"], t["embeddings.position_embeddings.weight"],
            t["embeddings.token_type_embeddings.weight"], t["embeddings.LayerNorm.weight"],
            t["embeddings.LayerNorm.bias"], _layers_from_hf(t, L))
    heads, eps = cfg["num_attention_heads"], cfg["layer_norm_eps"]
    h = oracle.bert_hidden(*args, ids, mask, types, heads, eps).astype(np.float64)
    m = mask.astype(np.float64)
    mean = (h * m[:, :, None]).sum(axis=1) / m.sum(axis=1, keepdims=True)
    mean /= np.linalg.norm(mean, axis=1, keepdims=True)
    np.testing.assert_allclose(mean, np.array(g["embeddings"]), atol=2e-5)

    def unit(x):
        return x / np.linalg.norm(x, axis=1, keepdims=True)

    cls = oracle.bert_embed(*args, ids, mask, types, heads, eps, pooling="cls")
    np.testing.assert_allclose(cls, unit(h[:, 0, :]), atol=2e-7)
    assert np.max(np.abs(cls - mean)) > 1e-2        # CLS is not the mean here
    # Position 0 masked: its row is still computed (attending to the active
    # positions) and pooled.
    mask2 = mask.copy()
    mask2[1, 0] = 0
    h2 = oracle.bert_hidden(*args, ids, mask2, types, heads, eps).astype(np.float64)
    cls2 = oracle.bert_embed(*args, ids, mask2, types, heads, eps, pooling="cls")
    np.testing.assert_allclose(cls2, unit(h2[:, 0, :]), atol=2e-7)
    assert np.max(np.abs(cls2[1] - cls[1])) > 1e-4
    np.testing.assert_array_equal(cls2[[0, 2]], cls[[0, 2]])
    # Only position 0 active: CLS == masked mean.
    mask3 = np.zeros_like(mask)
    mask3[:, 0] = 1
    a = oracle.bert_embed(*args, ids, mask3, types, heads, eps, pooling="cls")
    b = oracle.bert_embed(*args, ids, mask3, types, heads, eps)
    np.testing.assert_allclose(a, b, atol=1e-7)
