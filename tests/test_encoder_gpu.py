"""GPU parity of the q8 encoder (libeoship on gfx950) against the CPU oracle.

Bar (the benchmark's north star): per sequence, cosine >= 0.9999 and max-abs error
<= 2e-2 between the GPU embedding and the oracle's, both using the same
dequantized int8 per-channel weights; the oracle follows the reference's f32/f64
host path (oracle/encoder_oracle.c)."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen
from eos_amd.encoder import Encoder

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
ABS_MAX = 2e-2


def _case(name):
    print(f"[case] {name}", flush=True)


def _oracle(w, ids, mask, types=None):
    return oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta,
                             [L.dequantized() for L in w.layers], ids, mask, types, w.heads,
                             w.ln_eps)


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


@pytest.mark.parametrize("hidden,heads,inter,tokens", [(384, 12, 1536, 256), (512, 8, 2048, 300),
                                                       (768, 12, 3072, 96)])
def test_encoder_matches_oracle(rt, hidden, heads, inter, tokens):
    _case(f"encoder H={hidden} heads={heads} F={inter} T={tokens}")
    w = datagen.bert_q8_weights(2, hidden, heads, inter, 2000, 512, seed=hidden,
                                random_affine=True)
    ids, mask, lens = datagen.encoder_batch(6, tokens, 2000, 1, tokens, hidden + 1, hidden + 2)
    mask[0, :] = (np.arange(tokens) < 1)      # a single active token
    mask[1, :] = 1                            # full length
    types = (np.arange(tokens)[None, :] % 2 * mask).astype(np.int32)
    enc = Encoder(rt, w)
    got = enc.embed(ids, mask, types)
    _check(got, _oracle(w, ids, mask, types))


@pytest.mark.parametrize("hidden,heads,inter,tokens,pooling", [(384, 12, 1536, 200, "masked_mean"),
                                                                (512, 8, 2048, 700, "cls"),
                                                                (16, 4, 32, 40, "masked_mean")])
def test_encoder_batch_position_invariance(rt, hidden, heads, inter, tokens, pooling):
    """Positions restart with every sequence and nothing of a sequence's
    neighbours reaches it (the batch-row invariance the reference checks in
    runtime/backends/cuda/cuda_embed_pooled_parity_linux_test.go:140-182): the
    same sequence in every row embeds the same in each row, a permuted batch
    gives each sequence the embedding it had, and so do a batch of one and a
    batch padded to half the width, bit for bit (a row's arithmetic in every
    kernel is independent of where the row lies in the packed batch and of
    the batch's width). Covers the MFMA path (hidden 384; hidden 512 over 700 tokens, the
    12-wavefront attention workgroups, with CLS pooling) and the general-shape
    kernels (hidden 16)."""
    _case(f"batch-position invariance H={hidden} T={tokens} {pooling}")
    w = datagen.bert_q8_weights(2, hidden, heads, inter, 1000, tokens, seed=hidden + 90,
                                random_affine=True)
    ids, mask, _ = datagen.encoder_batch(6, tokens, 1000, 1, tokens, hidden + 91, hidden + 92)
    mask[1, :] = 1
    mask[4, 3:7] = 0
    types = (np.arange(tokens)[None, :] % 2 * mask).astype(np.int32)
    enc = Encoder(rt, w)
    if pooling == "cls":
        enc.set_pooling("cls")
    base = enc.embed(ids, mask, types)
    want = oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta,
                             [L.dequantized() for L in w.layers], ids, mask, types, w.heads,
                             w.ln_eps, pooling=pooling)
    _check(base, want)
    rep = enc.embed(np.repeat(ids[1:2], 5, axis=0), np.repeat(mask[1:2], 5, axis=0),
                    np.repeat(types[1:2], 5, axis=0))
    perm = np.array([3, 0, 5, 1, 4, 2])
    got = enc.embed(ids[perm], mask[perm], types[perm])
    one = enc.embed(ids[4:5], mask[4:5], types[4:5])
    # The sequences that fit in half the width, in a batch padded to that
    # width (at hidden 512 the 700-token batch runs the 12-wavefront
    # attention workgroups, the 350-token batch the 4-wavefront ones).
    half = tokens // 2
    short = np.array([b for b in range(6) if not mask[b, half:].any()])
    assert short.size > 0
    nar = enc.embed(ids[short, :half], mask[short, :half], types[short, :half])
    d_rep = float(np.max(np.abs(rep - base[1])))
    d_perm = float(np.max(np.abs(got - base[perm])))
    d_one = float(np.max(np.abs(one[0] - base[4])))
    d_nar = float(np.max(np.abs(nar - base[short])))
    print(f"  max diff: replicated {d_rep:.3e}  permuted {d_perm:.3e}  alone {d_one:.3e}  "
          f"narrower batch {d_nar:.3e} ({short.size} sequences)", flush=True)
    assert d_rep == 0.0 and d_perm == 0.0 and d_one == 0.0 and d_nar == 0.0
    enc.release()


def test_encoder_mask_holes_and_empty_sequence(rt):
    _case("encoder mask holes / empty")
    w = datagen.bert_q8_weights(1, 384, 12, 1536, 500, 128, seed=3, random_affine=True)
    ids, mask, _ = datagen.encoder_batch(4, 128, 500, 64, 128, 5, 6)
    rng = np.random.default_rng(2)
    mask[2] = (rng.random(128) < 0.5).astype(np.int32)   # holes keep absolute positions
    mask[3] = 0                                           # no active token -> zeros
    enc = Encoder(rt, w)
    got = enc.embed(ids, mask)
    want = _oracle(w, ids, mask)
    assert np.all(got[3] == 0) and np.all(want[3] == 0)
    _check(got, want)


def test_encoder_sequences_are_independent(rt):
    """A sequence's embedding does not depend on the rest of the batch."""
    _case("encoder batch independence")
    w = datagen.bert_q8_weights(2, 384, 12, 1536, 1000, 256, seed=4, random_affine=True)
    ids, mask, _ = datagen.encoder_batch(5, 200, 1000, 10, 200, 7, 8)
    enc = Encoder(rt, w)
    full = enc.embed(ids, mask)
    for b in (0, 3):
        one = enc.embed(ids[b:b + 1], mask[b:b + 1])
        np.testing.assert_allclose(one[0], full[b], rtol=0, atol=2e-6)


def test_encoder_rejects_out_of_range_ids(rt):
    _case("encoder id validation")
    from eos_amd._lib import EosHipError
    w = datagen.bert_q8_weights(1, 384, 12, 1536, 100, 64, seed=5)
    enc = Encoder(rt, w)
    ids = np.zeros((2, 16), np.int32)
    mask = np.ones((2, 16), np.int32)
    ids[1, 3] = 100
    with pytest.raises(EosHipError, match="out of range"):
        enc.embed(ids, mask)
    ids[1, 3] = 99
    enc.embed(ids, mask)
    with pytest.raises(EosHipError, match="position"):
        enc.embed(np.zeros((1, 65), np.int32), np.ones((1, 65), np.int32))


def test_baseline_c3_full_size(rt):
    """Benchmark config c3 at full size: 6 layers, hidden 384, 12 heads, FFN
    1536, batch 64 x 512, lengths U[32, 512]; a quarter of the batch (the
    shortest and longest sequences among them) checked against the oracle
    (sequences are independent), all 64 unit-norm."""
    _case("c3 full size 64 x 512")
    w = datagen.bert_q8_weights(6, 384, 12, 1536, 30522, 512, seed=7)
    ids, mask, lens = datagen.encoder_batch(64, 512, 30522, 32, 512, 8, 9)
    enc = Encoder(rt, w)
    got = enc.embed(ids, mask)
    np.testing.assert_allclose(np.linalg.norm(got, axis=1), 1.0, atol=1e-5)
    pick = np.array(sorted({*range(12), int(np.argmin(lens)), int(np.argmax(lens)), 37, 63}))
    assert len(pick) >= 15
    _check(got[pick], _oracle(w, ids[pick], mask[pick]))


def test_baseline_c4_long_context(rt):
    """Benchmark config c4 at full size: 4 layers, hidden 512, 8 heads (hd 64),
    FFN 2048, batch 4 x 8192, lengths U[4096, 8192] (seed 10). The two
    shortest sequences and the longest (the most key blocks, so the most
    chances for the lazy-rescale move) are checked against the oracle on
    their own valid tokens (sequences are independent and padding never
    reaches a valid token)."""
    _case("c4 full size 4 x 8192")
    w = datagen.bert_q8_weights(4, 512, 8, 2048, 30522, 8192, seed=10)
    ids, mask, lens = datagen.encoder_batch(4, 8192, 30522, 4096, 8192, 11, 10)
    enc = Encoder(rt, w)
    got = enc.embed(ids, mask)
    np.testing.assert_allclose(np.linalg.norm(got, axis=1), 1.0, atol=1e-5)
    order = np.argsort(lens, kind="stable")
    for b in (*order[:2], order[-1]):
        b = int(b)
        print(f"  sequence {b}: {int(lens[b])} tokens", flush=True)
        n = int(lens[b])
        want = _oracle(w, ids[b:b + 1, :n], np.ones((1, n), np.int32))
        _check(got[b:b + 1], want)


def test_fused_tail_split_launch(rt):
    """At hidden 512 the layer tail's first launch covers one 64-row block
    per CU and a second launch takes the rows after it in 32-row blocks. A
    batch with more packed rows than the first launch covers: the sequences
    around the boundary row and the last one match the oracle on their own
    valid tokens, and each embeds bit for bit as it does in a batch of one
    (where the second launch has no rows)."""
    first = rt.info()["compute_units"] * 64
    nseq = first // 400 + 4
    _case(f"fused tail split: hidden 512, {nseq} x 512 tokens, first launch {first} rows")
    w = datagen.bert_q8_weights(2, 512, 8, 2048, 2000, 512, seed=81, random_affine=True)
    ids, mask, lens = datagen.encoder_batch(nseq, 512, 2000, 400, 512, 82, 83)
    rows8 = (lens.astype(np.int64) + 7) // 8 * 8
    off = np.concatenate([[0], np.cumsum(rows8)[:-1]])
    assert off[-1] + rows8[-1] > first
    check = sorted({int(b) for b in np.nonzero((off < first + 600) & (off + rows8 > first - 600))[0]}
                   | {nseq - 1})
    enc = Encoder(rt, w)
    got = enc.embed(ids, mask)
    for b in check:
        n = int(lens[b])
        print(f"  sequence {b}: rows {int(off[b])}..{int(off[b] + n - 1)}", flush=True)
        _check(got[b:b + 1], _oracle(w, ids[b:b + 1, :n], np.ones((1, n), np.int32)))
        alone = enc.embed(ids[b:b + 1], mask[b:b + 1])
        assert np.array_equal(alone, got[b:b + 1])
    enc.release()


def _peaked_batch(tokens, vocab, special):
    """Sequences with the planted high-scoring tokens at chosen positions:
    (ids, mask); `special` maps sequence -> [(position, token id)], every
    other token is drawn from ids >= 3."""
    rng = np.random.default_rng(77)
    b = len(special)
    ids = rng.integers(3, vocab, size=(b, tokens)).astype(np.int32)
    mask = np.ones((b, tokens), np.int32)
    for s, plants in special.items():
        for p, t in plants:
            ids[s, p] = t
    mask[4, 40:] = 0
    ids[4, 40:] = 0
    return ids, mask


@pytest.mark.parametrize("hidden,heads,inter", [(384, 12, 1536), (512, 8, 2048), (512, 4, 1024)])
def test_attention_late_maximum_moves_reference(rt, hidden, heads, inter):
    """Peaked, late-maximum attention (trained-model regime): a key far above
    every earlier one (about 25-40 nats) appears after the first key block,
    so the lazy-rescale branch moves the exponent reference, rescales O and
    the partial sums and recomputes the block (enc_kernels.hip attention).
    Sequence 0 moves twice (a weaker key in block 1..2, the strongest later),
    sequence 1 has its maximum in block 0 (no move), sequence 2 only at its
    end, sequence 3 has no planted key, sequence 4 is short with the key at
    its last positions. Only one lane of a query's pair holds the key."""
    hd = hidden // heads
    _case(f"peaked attention hd={hd}")
    peaked = {"alpha": 4.0, "beta": 3.0, "tokens": {1: 1.0, 2: 0.6}}
    w = datagen.bert_q8_weights(2, hidden, heads, inter, 2000, 512, seed=hidden + heads,
                                random_affine=True, peaked=peaked)
    special = {0: [(80, 2), (200, 1)], 1: [(5, 1), (150, 2)], 2: [(300, 1)], 3: [],
               4: [(35, 1), (38, 2)]}
    ids, mask = _peaked_batch(320, 2000, special)
    enc = Encoder(rt, w)
    got = enc.embed(ids, mask)
    moves = enc.attention_moves()
    print(f"  later-block reference moves: {moves}", flush=True)
    assert moves > 0
    _check(got, _oracle(w, ids, mask))


def test_w8a8_outlier_channels(rt):
    """LayerNorm outputs with a few channels 30-50x the others (as trained
    BERT models have): the per-row int8 activations of the QKV and FFN-up
    GEMMs then leave the other channels a few levels, and the contract must
    still hold (a float64 simulation of this case gives min cos 0.9999987)."""
    _case("W8A8 with outlier channels")
    w = datagen.bert_q8_weights(3, 384, 12, 1536, 2000, 512, seed=31, random_affine=True)
    rng = np.random.default_rng(32)
    for nch, factor in ((3, 50.0), (8, 30.0)):
        ch = rng.choice(384, nch, replace=False)
        gammas = [w.emb_gamma] + [L.ln1_gamma for L in w.layers] + [L.ln2_gamma for L in w.layers]
        for g in gammas:
            g[ch] *= np.float32(factor)
        for L in w.layers:
            L.ln1_beta[ch[:1]] += np.float32(0.5 * factor)
        ids, mask, _ = datagen.encoder_batch(8, 256, 2000, 16, 256, 33 + nch, 34 + nch)
        enc = Encoder(rt, w)
        _check(enc.embed(ids, mask), _oracle(w, ids, mask))
        enc.release()


@pytest.mark.parametrize("hidden,heads,inter,gelu", [(384, 12, 1536, 1), (384, 6, 768, 2),
                                                      (512, 8, 2048, 1), (768, 12, 3072, 1)])
def test_fused_tail_matches_unfused_and_oracle(rt, hidden, heads, inter, gelu):
    """The fused layer tail (O projection through the second LayerNorm in one
    kernel per row block) against the unfused GEMM + LayerNorm launches, which
    round at the same points: embeddings equal to within a few f16 units, and
    both within the contract against the oracle. Ragged lengths put partial
    row blocks at every sequence boundary and at the end."""
    _case(f"fused tail H={hidden} heads={heads} F={inter} gelu={gelu}")
    w = datagen.bert_q8_weights(2, hidden, heads, inter, 3000, 256, seed=hidden + gelu,
                                random_affine=True, gelu=gelu)
    ids, mask, _ = datagen.encoder_batch(9, 200, 3000, 1, 200, hidden + 11, hidden + 12)
    enc = Encoder(rt, w)
    fused = enc.embed(ids, mask)
    enc.set_fused_tail(False)
    plain = enc.embed(ids, mask)
    enc.release()
    d = np.max(np.abs(fused - plain))
    print(f"  fused vs unfused max abs {d:.3e}", flush=True)
    assert d <= 2e-3
    _check(fused, _oracle(w, ids, mask))


def test_encoder_cls_pooling(rt):
    """CLS pooling (bert_embedder pooling "cls", bert_embedder_ops.go:183-196)
    on the fused encoder: position 0's hidden state, normalized. Position 0
    masked (its row is computed anyway, attending to the active positions),
    a sequence with no active position (its CLS row attends to nothing), and
    the unfused layer path agree with the oracle."""
    _case("encoder CLS pooling")
    w = datagen.bert_q8_weights(2, 512, 8, 2048, 1000, 300, seed=61, random_affine=True)
    ids, mask, _ = datagen.encoder_batch(6, 300, 1000, 1, 300, 62, 63)
    mask[1, 0] = 0
    mask[2, :] = 0
    mask[3, :5] = 0
    mask[4, :] = 0
    mask[4, 0] = 1                       # only position 0 active: CLS == mean
    enc = Encoder(rt, w)
    mean = enc.embed(ids, mask)
    enc.set_pooling("cls")
    got = enc.embed(ids, mask)
    want = oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta,
                             [L.dequantized() for L in w.layers], ids, mask, None, w.heads,
                             w.ln_eps, pooling="cls")
    _check(got, want)
    np.testing.assert_allclose(got[4], mean[4], atol=1e-6)
    enc.set_fused_tail(False)
    _check(enc.embed(ids, mask), want)
    enc.release()


@pytest.mark.parametrize("hidden,heads,inter,pooling", [(16, 4, 32, "masked_mean"),
                                                          (64, 2, 100, "cls"),
                                                          (200, 5, 300, "masked_mean"),
                                                          (128, 16, 256, "cls")])
def test_encoder_general_shapes(rt, hidden, heads, inter, pooling):
    """Shapes outside the MFMA kernels (hidden 16 / 64 / 200, head dims 4,
    32 at hidden 64, 40 and 8) run the general-shape kernels: within f32
    rounding of the oracle on the same dequantized weights, for both
    poolings; ragged lengths, position 0 masked, a mask hole, a sequence
    with no active position, token types."""
    _case(f"encoder general shape H={hidden} heads={heads} F={inter} {pooling}")
    w = datagen.bert_q8_weights(2, hidden, heads, inter, 500, 64, seed=hidden + heads,
                                random_affine=True)
    ids, mask, _ = datagen.encoder_batch(6, 64, 500, 1, 64, hidden + 7, hidden + 8)
    mask[1, 0] = 0
    mask[2, :] = 0
    mask[3, 5:9] = 0
    types = (np.arange(64)[None, :] % 2 * mask).astype(np.int32)
    enc = Encoder(rt, w)
    if pooling == "cls":
        enc.set_pooling("cls")
    got = enc.embed(ids, mask, types)
    want = oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta,
                             [L.dequantized() for L in w.layers], ids, mask, types, w.heads,
                             w.ln_eps, pooling=pooling)
    err = float(np.max(np.abs(got - want)))
    print(f"  max abs {err:.3e}", flush=True)
    assert err <= 1e-5
    if pooling == "masked_mean":
        assert np.all(got[2] == 0)
    enc.release()


@pytest.mark.parametrize("pooling", ["masked_mean", "cls"])
def test_attention_wide_workgroups(rt, pooling):
    """Head dim 64 over inputs longer than 512 tokens runs 12-wavefront
    attention workgroups (384 queries each): ragged lengths on both sides of
    the 384-query boundaries, one and zero active tokens, position 0 masked
    (the CLS row then follows the active rows), a mask hole; against the
    oracle on each sequence's valid tokens."""
    _case(f"wide attention workgroups {pooling}")
    w = datagen.bert_q8_weights(2, 512, 8, 2048, 1000, 1100, seed=71, random_affine=True)
    lengths = [1100, 1, 0, 385, 384, 383, 767, 769]
    rng = np.random.default_rng(72)
    ids = rng.integers(1, 1000, (len(lengths), 1100)).astype(np.int32)
    mask = np.zeros_like(ids)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1
    mask[3, 0] = 0
    mask[6, 100:140] = 0
    enc = Encoder(rt, w)
    if pooling == "cls":
        enc.set_pooling("cls")
    got = enc.embed(ids, mask)
    want = oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta,
                             [L.dequantized() for L in w.layers], ids, mask, None, w.heads,
                             w.ln_eps, pooling=pooling)
    _check(got, want)
    enc.release()


def test_encoder_rejects_out_of_range_ids_at_masked_positions(rt):
    """The reference range-checks every input id, masked positions included
    (BERTEmbeddingsReference, tensor_ops.go:1476-1489)."""
    _case("encoder id validation at masked positions")
    from eos_amd._lib import EosHipError
    w = datagen.bert_q8_weights(1, 384, 12, 1536, 100, 64, seed=5)
    enc = Encoder(rt, w)
    ids = np.zeros((2, 16), np.int32)
    mask = np.ones((2, 16), np.int32)
    mask[1, 10:] = 0
    ids[1, 12] = 100
    with pytest.raises(EosHipError, match="out of range"):
        enc.embed(ids, mask)
    ids[1, 12] = 0
    types = np.zeros_like(ids)
    types[0, 15] = 2                     # type table has 2 rows
    mask[0, 15] = 0
    with pytest.raises(EosHipError, match="out of range"):
        enc.embed(ids, mask, types)
    types[0, 15] = 1
    enc.embed(ids, mask, types)
