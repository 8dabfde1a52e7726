"""GPU parity of the compact (family (a)) embedder against the CPU oracle.

Bar (the benchmark's north star, as for the BERT family): per sequence, cosine >=
0.9999 and max-abs error <= 2e-2 between the GPU embedding and
oracle.compact_embed (oracle/encoder_oracle.c, the reference's f32 graph of
models/default_embedding.go:484-505), both on the same dequantized per-tensor
q8 weights."""
import numpy as np
import pytest

import oracle
from eos_amd import datagen
from eos_amd._lib import EosHipError
from eos_amd.encoder import CompactEncoder

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
ABS_MAX = 2e-2


def _case(name):
    print(f"[case] {name}", flush=True)


def _oracle(w, ids, mask, roles):
    tok = w.token_embedding.astype(np.float32) * np.float32(w.s_token)
    role = w.role_embedding.astype(np.float32) * np.float32(w.s_role)
    wout = None
    if w.output_projection is not None:
        wout = w.output_projection.astype(np.float32) * np.float32(w.s_output)
    return oracle.compact_embed(tok, role, [L.dequantized() for L in w.layers], ids, mask, roles,
                                w.heads, wout)


def _check(got, want):
    n = np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1)
    live = n > 0
    cos = np.sum(got.astype(np.float64) * want, axis=1)[live] / n[live]
    err = np.max(np.abs(got - want))
    print(f"  min cos {cos.min() if live.any() else 1.0:.8f}  max abs {err:.3e}", flush=True)
    if live.any():
        assert cos.min() >= COS_MIN
    assert err <= ABS_MAX
    np.testing.assert_array_equal(got[~live], want[~live])


@pytest.mark.parametrize("D,heads,F,L,O,T", [
    (128, 1, 256, 2, None, 256),   # DefaultEmbeddingPackageConfig defaults
    (128, 1, 256, 2, 64, 200),     # with an output projection
    (256, 2, 512, 2, None, 160),   # two heads of 128
    (384, 12, 1536, 1, 256, 96),   # many small heads
    (512, 8, 1024, 1, None, 64),
])
def test_compact_matches_oracle(rt, D, heads, F, L, O, T):
    _case(f"compact D={D} heads={heads} F={F} L={L} O={O} T={T}")
    w = datagen.compact_q8_weights(L, D, heads, F, vocab=3000, max_seq=256, out_dim=O, seed=D + F)
    ids, mask, _ = datagen.encoder_batch(6, T, 3000, 1, T, D + 3, D + 4)
    mask[0, :] = (np.arange(T) < 1)   # a single active token
    mask[1, :] = 1                    # full length
    mask[2, 5:9] = 0                  # a hole: positions keep their index
    mask[3, :] = 0                    # empty: zeros
    roles = datagen.uniform_int(D + 5, ids.size, 0, 3).astype(np.int32).reshape(ids.shape)
    enc = CompactEncoder(rt, w)
    got = enc.embed(ids, mask, roles)
    assert got.shape == (6, w.output_dim)
    _check(got, _oracle(w, ids, mask, roles))
    assert not got[3].any()
    enc.release()


def test_stale_memory_does_not_leak_into_embeddings(rt):
    """Activation rows no kernel writes (pad rows between packed sequences,
    rows past a sequence that attention's V blocks cover) may hold anything
    a freed buffer left behind: a freed block filled with f16 NaN is reused
    by the encoder's buffers, and the embeddings must still match."""
    from eos_amd.runtime import DeviceBuffer
    _case("compact on reused NaN-filled memory")
    poison = DeviceBuffer(rt, 256 << 20)
    poison.upload(np.full(128 << 20, 0xFFFF, np.uint16))
    poison.free()
    w = datagen.compact_q8_weights(2, 128, 1, 256, vocab=3000, max_seq=256, out_dim=64, seed=61)
    ids, mask, _ = datagen.encoder_batch(6, 200, 3000, 1, 200, 62, 63)
    mask[3, :] = 0
    roles = datagen.uniform_int(64, ids.size, 0, 3).astype(np.int32).reshape(ids.shape)
    enc = CompactEncoder(rt, w)
    got = enc.embed(ids, mask, roles)
    assert np.isfinite(got).all()
    _check(got, _oracle(w, ids, mask, roles))
    enc.release()


def test_compact_batch_position_invariance(rt):
    """RoPE positions restart with every sequence (the reference's
    TestCUDARoPEBatchedRowsAreBatchPositionInvariant,
    runtime/backends/cuda/cuda_embed_pooled_parity_linux_test.go:140-182):
    the same sequence in every row embeds the same in each row, a permuted
    batch gives each sequence the embedding it had, and so does a batch of
    one, bit for bit."""
    _case("compact batch-position invariance")
    w = datagen.compact_q8_weights(2, 128, 1, 256, vocab=3000, max_seq=256, out_dim=64, seed=93)
    ids, mask, _ = datagen.encoder_batch(6, 160, 3000, 1, 160, 94, 95)
    mask[1, :] = 1
    mask[4, 3:7] = 0
    roles = datagen.uniform_int(96, ids.size, 0, 3).astype(np.int32).reshape(ids.shape)
    enc = CompactEncoder(rt, w)
    base = enc.embed(ids, mask, roles)
    _check(base, _oracle(w, ids, mask, roles))
    rep = enc.embed(np.repeat(ids[1:2], 5, axis=0), np.repeat(mask[1:2], 5, axis=0),
                    np.repeat(roles[1:2], 5, axis=0))
    perm = np.array([3, 0, 5, 1, 4, 2])
    got = enc.embed(ids[perm], mask[perm], roles[perm])
    one = enc.embed(ids[4:5], mask[4:5], roles[4:5])
    d_rep = float(np.max(np.abs(rep - base[1])))
    d_perm = float(np.max(np.abs(got - base[perm])))
    d_one = float(np.max(np.abs(one[0] - base[4])))
    print(f"  max diff: replicated {d_rep:.3e}  permuted {d_perm:.3e}  alone {d_one:.3e}",
          flush=True)
    assert d_rep == 0.0 and d_perm == 0.0 and d_one == 0.0
    enc.release()


def test_compact_q4_weights_and_no_roles(rt):
    _case("compact q4 weights, role ids omitted")
    w = datagen.compact_q8_weights(2, 128, 1, 256, vocab=500, max_seq=64, seed=9, bits=4)
    assert int(np.max(np.abs(w.layers[0].attn_q))) <= 7
    ids, mask, _ = datagen.encoder_batch(5, 64, 500, 3, 64, 11, 12)
    enc = CompactEncoder(rt, w)
    got = enc.embed(ids, mask)
    _check(got, _oracle(w, ids, mask, np.zeros_like(ids)))
    enc.release()


def test_compact_rejects_bad_ids_and_shapes(rt):
    _case("compact validation")
    w = datagen.compact_q8_weights(1, 128, 1, 256, vocab=100, max_seq=32, seed=13)
    enc = CompactEncoder(rt, w)
    ids, mask, _ = datagen.encoder_batch(2, 32, 100, 32, 32, 14, 15)
    roles = np.zeros_like(ids)
    roles[1, 4] = 3  # role_embedding has 3 rows
    with pytest.raises(EosHipError, match="out of range"):
        enc.embed(ids, mask, roles)
    bad = ids.copy()
    bad[0, 0] = 100
    with pytest.raises(EosHipError, match="out of range"):
        enc.embed(bad, mask)
    long_ids = np.zeros((1, 33), np.int32)
    with pytest.raises(EosHipError, match="exceed"):
        enc.embed(long_ids, np.ones_like(long_ids))
    # a valid call after the errors still matches
    _check(enc.embed(ids, mask), _oracle(w, ids, mask, np.zeros_like(ids)))
    enc.release()
    w.heads = 3  # 128 / 3 is not a head size the kernels take
    with pytest.raises(EosHipError, match="head dim"):
        CompactEncoder(rt, w)
