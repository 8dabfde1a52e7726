"""Pins the compact-family (family (a)) restatement in oracle/encoder_oracle.c.

Known answers come from the reference's own tensor-op tests
(runtime/backend/tensor_ops_test.go): ropeRows :646-672, layerNormRows
:465-491, maskedSoftmaxRows :590-631, geluTensor :633-644 with approxGELU
:1149-1153. The graph order (models/default_embedding.go:484-505) is checked
against an independent float64 composition, and invariants the graph fixes
(padding does not change a sequence's embedding, zero layers reduce to
mean(normalize(rope(tok + role)))) close what the pieces leave open. CPU only."""
import math

import numpy as np
import pytest

import oracle
from eos_amd import datagen
from eos_amd.encoder import quantize_per_tensor


def test_rope_known_answers():
    # tensor_ops_test.go:646-656: row 0 is position 0 (identity), row 1 is
    # position 1 rotated by 1 rad.
    out = oracle.rope_rows(np.array([[1, 0], [0, 1]], np.float32), seq=2)
    np.testing.assert_allclose(out, [[1, 0], [-0.84147096, 0.5403023]], rtol=0, atol=1e-7)
    # :658-672: a batched [2, 2, 2] tensor restarts positions per sequence.
    x = np.array([[1, 0], [0, 1], [1, 0], [0, 1]], np.float32)
    out = oracle.rope_rows(x, seq=2)
    np.testing.assert_allclose(out, [[1, 0], [-0.84147096, 0.5403023]] * 2, rtol=0, atol=1e-7)


def test_rope_textbook_frequencies_and_relative_position():
    # RoPE (Su et al.): pair i of D columns turns by pos * 10000^(-2i/D). At
    # D = 4, pair 1 turns 0.01 rad per position: position 100 is 1 rad.
    x = np.zeros((101, 4), np.float32)
    x[:, 2] = 1.0
    out = oracle.rope_rows(x, seq=101)
    np.testing.assert_allclose(out[100], [0, 0, math.cos(1.0), math.sin(1.0)], atol=1e-6)
    np.testing.assert_allclose(out[7, 2:], [math.cos(0.07), math.sin(0.07)], atol=1e-6)
    # rotations keep pair norms, and <rope(a, p), rope(b, q)> depends on p - q only
    rng = np.random.default_rng(3)
    D, T = 16, 40
    a = np.tile(rng.standard_normal(D).astype(np.float32), (T, 1))
    b = np.tile(rng.standard_normal(D).astype(np.float32), (T, 1))
    ra, rb = oracle.rope_rows(a, T), oracle.rope_rows(b, T)
    np.testing.assert_allclose(np.linalg.norm(ra.reshape(T, -1, 2), axis=2),
                               np.linalg.norm(a.reshape(T, -1, 2), axis=2), rtol=1e-6)
    d1 = float(np.dot(ra[5].astype(np.float64), rb[2]))
    d2 = float(np.dot(ra[30].astype(np.float64), rb[27]))
    assert abs(d1 - d2) < 1e-5
    # an odd trailing column is left as is
    odd = oracle.rope_rows(np.ones((3, 5), np.float32), seq=3)
    np.testing.assert_array_equal(odd[:, 4], 1.0)


def test_layer_norm_rows_known_answers():
    # tensor_ops_test.go:465-491: eps = 1e-5 gives 1/sqrt(1 + 1e-5).
    out = oracle.layer_norm_rows(np.array([[2, 4], [6, 8], [1, 3], [5, 7]], np.float32))
    np.testing.assert_allclose(out, [[-0.999995, 0.999995]] * 4, rtol=0, atol=1e-6)
    # a small row shows the epsilon: [a, -a] -> +-a / sqrt(a^2 + 1e-5)
    a = 0.003
    out = oracle.layer_norm_rows(np.array([[a, -a]], np.float32))
    np.testing.assert_allclose(out[0], [a / math.sqrt(a * a + 1e-5), -a / math.sqrt(a * a + 1e-5)],
                               rtol=1e-5)
    # a constant row becomes zeros (no affine terms)
    np.testing.assert_array_equal(oracle.layer_norm_rows(np.full((1, 8), 3.5, np.float32)), 0)


def _softmax_via_attention(logits, mask):
    """Drives compact_single_head_attention so that its scores equal `logits`
    (q = logits row, k = sqrt(d) I, v = I): the output rows are the masked
    softmax probabilities."""
    B, T = mask.shape
    d = T
    q = np.asarray(logits, np.float32).reshape(B * T, d)
    k = np.tile(np.float32(math.sqrt(d)) * np.eye(d, dtype=np.float32), (B, 1))
    v = np.tile(np.eye(d, dtype=np.float32), (B, 1))
    return oracle.compact_single_head_attention(q, k, v, mask)


def test_masked_softmax_known_answers():
    e, e2 = math.exp(1), math.exp(2)
    # tensor_ops_test.go:608-631 (batched, per-sequence key mask); one query
    # row per key slot so the logits block is square.
    logits = np.array([[0, 1, 9], [2, 0, 8], [7, 7, 7],
                       [5, 1, 0], [4, 2, 0], [7, 7, 7]], np.float32)
    mask = np.array([[1, 1, 0], [0, 1, 1]], np.int32)
    out = _softmax_via_attention(logits, mask)
    want = [[1 / (1 + e), e / (1 + e), 0], [e2 / (1 + e2), 1 / (1 + e2), 0], [0.5, 0.5, 0],
            [0, e / (1 + e), 1 / (1 + e)], [0, e2 / (1 + e2), 1 / (1 + e2)], [0, 0.5, 0.5]]
    np.testing.assert_allclose(out, want, rtol=0, atol=2e-6)
    # no active key -> zeros
    out = _softmax_via_attention(logits[:3], np.zeros((1, 3), np.int32))
    np.testing.assert_array_equal(out, 0)


def test_single_head_attention_matches_f64_multihead_form():
    # The one-head f32 path and the BERT f64 path (compact_multihead_attention
    # with one head) compute the same function.
    rng = np.random.default_rng(4)
    B, T, D = 3, 17, 32
    q, k, v = (rng.standard_normal((B * T, D)).astype(np.float32) for _ in range(3))
    mask = np.ones((B, T), np.int32)
    mask[0, 9:] = 0
    mask[2, 3] = 0
    got = oracle.compact_single_head_attention(q, k, v, mask)
    np.testing.assert_allclose(got, oracle.bert_attention(q, k, v, mask, 1), rtol=0, atol=3e-6)


def test_tanh_gelu_known_answers():
    # geluTensor at -1, 0, 1, 2 (tensor_ops_test.go:633-644), values of the
    # tanh form 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
    got = oracle.gelu_tanh(np.array([-1, 0, 1, 2], np.float32))
    np.testing.assert_allclose(got, [-0.15880801, 0.0, 0.84119199, 1.95459769], rtol=0, atol=2e-7)
    # within 1e-3 of the erf GELU x Phi(x), and gelu(x) - gelu(-x) = x
    x = np.linspace(-6, 6, 241).astype(np.float32)
    erf_form = 0.5 * x * (1 + np.array([math.erf(v / math.sqrt(2)) for v in x.astype(np.float64)]))
    g, gn = oracle.gelu_tanh(x), oracle.gelu_tanh(-x)
    assert np.max(np.abs(g - erf_form)) < 1e-3
    np.testing.assert_allclose(g - gn, x, rtol=0, atol=4e-6)


def _graph_f64(tok, role, layers, ids, mask, roles, heads, wout=None):
    """The compactTransformerPipelineBody graph in float64, written from
    models/default_embedding.go:484-505 and the reference op definitions."""
    B, T = ids.shape
    D = tok.shape[1]
    x = (tok[ids] + role[roles]).astype(np.float64).reshape(B * T, D)
    pos = np.tile(np.arange(T), B)
    for c in range(0, D - 1, 2):
        th = pos / (10000.0 ** (c / D))
        x0, x1 = x[:, c].copy(), x[:, c + 1].copy()
        x[:, c] = x0 * np.cos(th) - x1 * np.sin(th)
        x[:, c + 1] = x0 * np.sin(th) + x1 * np.cos(th)

    def ln(y):
        m = y.mean(axis=1, keepdims=True)
        var = ((y - m) ** 2).mean(axis=1, keepdims=True)
        return (y - m) / np.sqrt(var + 1e-5)

    hd = D // heads
    for (wq, wk, wv, wo, wup, wdn) in layers:
        q, k, v = x @ wq, x @ wk, x @ wv
        mixed = np.zeros_like(x)
        for b in range(B):
            act = np.nonzero(mask[b])[0]
            if len(act) == 0:
                continue
            rs = slice(b * T, (b + 1) * T)
            for h in range(heads):
                cs = slice(h * hd, (h + 1) * hd)
                lg = q[rs, cs] @ k[b * T + act, cs].T / math.sqrt(hd)
                p = np.exp(lg - lg.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                mixed[rs, cs] = p @ v[b * T + act, cs]
        h1 = ln(mixed @ wo + x)
        u = h1 @ wup
        g = 0.5 * u * (1 + np.tanh(0.7978845608 * (u + 0.044715 * u ** 3)))
        x = ln(g @ wdn + h1)
    n = np.linalg.norm(x, axis=1, keepdims=True)
    x = np.where(n > 0, x / np.where(n > 0, n, 1), x)
    if wout is not None:
        x = x @ wout
    x = x.reshape(B, T, -1)
    cnt = mask.sum(axis=1)
    pooled = (x * mask[:, :, None]).sum(axis=1)
    return np.where(cnt[:, None] > 0, pooled / np.maximum(cnt, 1)[:, None], 0.0)


def _deq(w):
    tok = w.token_embedding.astype(np.float32) * np.float32(w.s_token)
    role = w.role_embedding.astype(np.float32) * np.float32(w.s_role)
    layers = [L.dequantized() for L in w.layers]
    wout = None
    if w.output_projection is not None:
        wout = w.output_projection.astype(np.float32) * np.float32(w.s_output)
    return tok, role, layers, wout


@pytest.mark.parametrize("D,heads,F,L,O", [(32, 1, 64, 2, None), (32, 4, 64, 2, 16),
                                           (64, 2, 128, 1, None)])
def test_compact_embed_matches_f64_graph(D, heads, F, L, O):
    w = datagen.compact_q8_weights(L, D, heads, F, vocab=97, max_seq=12, out_dim=O, seed=D + heads)
    tok, role, layers, wout = _deq(w)
    ids, mask, _ = datagen.encoder_batch(4, 12, 97, 1, 12, 31, 32)
    mask[3] = 0  # an empty sequence pools to zeros
    roles = datagen.uniform_int(33, ids.size, 0, 3).astype(np.int32).reshape(ids.shape)
    got = oracle.compact_embed(tok, role, layers, ids, mask, roles, heads, wout)
    want = _graph_f64(tok, role, [[a.astype(np.float64) for a in l] for l in layers], ids, mask,
                      roles, heads, None if wout is None else wout.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    np.testing.assert_array_equal(got[3], 0)


def test_compact_embed_padding_invariance_and_zero_layers():
    w = datagen.compact_q8_weights(2, 32, 2, 64, vocab=50, max_seq=16, seed=5)
    tok, role, layers, _ = _deq(w)
    ids, mask, lens = datagen.encoder_batch(3, 16, 50, 2, 16, 41, 42)
    roles = datagen.uniform_int(43, ids.size, 0, 3).astype(np.int32).reshape(ids.shape)
    full = oracle.compact_embed(tok, role, layers, ids, mask, roles, 2)
    for b in range(3):
        n = int(lens[b])
        alone = oracle.compact_embed(tok, role, layers, ids[b:b + 1, :n], mask[b:b + 1, :n],
                                     roles[b:b + 1, :n], 2)
        np.testing.assert_allclose(alone[0], full[b], rtol=0, atol=1e-6)
    # zero layers: mean over active rows of normalize(rope(tok + role))
    z = oracle.compact_embed(tok, role, [], ids, mask, roles, 2)
    x = oracle.rope_rows((tok[ids] + role[roles]).reshape(-1, 32), 16)
    x = oracle.normalize_rows(x).reshape(3, 16, 32)
    np.testing.assert_allclose(z, oracle.mean_pool_masked(x, mask), rtol=0, atol=1e-7)


def test_quantize_per_tensor_grid():
    # packQuantizedTensorStorage (runtime/mll_export.go:918-942): levels
    # 127 (q8) / 7 (q4), round half away from zero, symmetric clamp.
    w = np.array([[0.5, -1.0, 0.25], [-0.5, 0.75, 1.0 / 14]], np.float32)
    c, s = quantize_per_tensor(w, 8)
    assert s == np.float32(1.0) / np.float32(127)
    np.testing.assert_array_equal(c, [[64, -127, 32], [-64, 95, 9]])
    # q4: the quotient is formed in f32, 0.5 / float32(1/7) = 3.4999998 -> 3
    c4, s4 = quantize_per_tensor(w, 4)
    assert s4 == np.float32(1.0) / np.float32(7)
    np.testing.assert_array_equal(c4, [[3, -7, 2], [-3, 5, 1]])
    # scale 1 exactly: halves round away from zero (math.Round), not to even
    c, s = quantize_per_tensor(np.array([127, 2.5, -2.5, 0.5, -130], np.float32) * (127 / 130))
    h, sh = quantize_per_tensor(np.array([127, 2.5, -2.5, 0.5], np.float32))
    assert sh == 1.0
    np.testing.assert_array_equal(h, [127, 3, -3, 1])
    assert c[-1] == -127 and c[0] == 124
    z, sz = quantize_per_tensor(np.zeros((2, 2), np.float32))
    assert sz == 0 and not z.any()
