"""TurboQuant corpus encoder: f32 vectors -> (packed codes, norms), the MSE
stage of the corpus-side Quantize (turboquant.NewIPWithSeed /
IPQuantizer.Quantize, called at runtime/retrieval_turboquant.go:700,708; the
quantizer module is not vendored under the reference, so the arithmetic is the
build-defined one of oracle/tq_oracle.c tq_encode).

CPU pins of the oracle:
- identity rotation, one-hot inputs: the hot coordinate takes the top centroid
  and every zero coordinate the lower of the two centroids nearest 0 (an exact
  tie on the symmetric grid), norm = |a|;
- an independent f64 brute force (matrix product, distance table, first
  minimum) over random rotated inputs;
- the Lloyd-Max distortion of the reconstruction R^T (norm * s * C[code]) lies
  between the information-theoretic floor 4^-b and the TurboQuant bound
  (sqrt(3) pi / 2) 4^-b; a wrong code choice or a transposed rotation lands far
  outside it;
- encode -> scan: scores estimate the true inner products within the
  quantization noise, and a vector's own score is its best one.
GPU: codes and norms are bit-exact against the oracle (both kernels: d <= 512
and d <= 1024), including zero rows, ragged counts and odd row widths; host and
device entry points agree; encoder output -> encode on the device matches."""
import math

import numpy as np
import pytest

import oracle
from eos_amd import datagen


def _vectors(n, d, seed, sigma=1.0):
    """Gaussian directions with lognormal(0, sigma) length scales."""
    x = datagen.normal(seed, n * d).reshape(n, d)
    scale = datagen.lognormal(seed + 1, n, sigma)
    return (x * scale[:, None]).astype(np.float32)


def _unpack(codes, d, bits):
    per = 8 // bits
    out = np.zeros((codes.shape[0], codes.shape[1] * per), np.int64)
    for e in range(per):
        out[:, e::per] = (codes >> (e * bits)) & ((1 << bits) - 1)
    return out[:, :d]


# ----------------------------------------------------------------------- CPU

@pytest.mark.parametrize("bits", [2, 4])
def test_one_hot_closed_form(bits):
    d = 16
    cb, s = datagen.turboquant_codebook(bits, d)
    assert np.array_equal(cb, -cb[::-1])  # symmetric grid
    x = np.zeros((2 * d, d), np.float32)
    for i in range(d):
        x[i, i] = 0.75 + i
        x[d + i, i] = -(2.0 + i)
    codes, norms = oracle.tq_encode(x, None, d, bits, cb, s)
    np.testing.assert_array_equal(norms, np.abs(x).max(axis=1))
    u = _unpack(codes, d, bits)
    levels = 1 << bits
    zero_code = levels // 2 - 1  # lower of the two centroids nearest 0
    for r in range(2 * d):
        hot = r % d
        want = np.full(d, zero_code)
        want[hot] = levels - 1 if r < d else 0
        np.testing.assert_array_equal(u[r], want)


@pytest.mark.parametrize("bits,d", [(2, 64), (4, 384), (4, 100)])
def test_matches_f64_brute_force(bits, d):
    x = _vectors(300, d, 71 + d)
    rot = datagen.orthogonal(72 + d, d).astype(np.float32)
    cb, s = datagen.turboquant_codebook(bits, d)
    codes, norms = oracle.tq_encode(x, rot, d, bits, cb, s)
    x64 = x.astype(np.float64)
    u = x64 @ rot.astype(np.float64).T
    nrm = np.sqrt(np.sum(x64 * x64, axis=1))
    nc = nrm[:, None] * (float(s) * cb.astype(np.float64))[None, :]
    want = np.argmin(np.abs(u[:, :, None] - nc[:, None, :]), axis=2)
    np.testing.assert_array_equal(_unpack(codes, d, bits), want)
    np.testing.assert_allclose(norms, nrm.astype(np.float32), rtol=2e-7, atol=0)
    np.testing.assert_array_equal(codes, datagen.pack_codes(want, bits))


@pytest.mark.parametrize("bits", [2, 4])
def test_distortion_within_turboquant_bound(bits):
    d, n = 256, 400
    x = _vectors(n, d, 81)
    rot = datagen.orthogonal(82, d).astype(np.float32)
    cb, s = datagen.turboquant_codebook(bits, d)
    codes, norms = oracle.tq_encode(x, rot, d, bits, cb, s)
    y = (float(s) * cb.astype(np.float64))[_unpack(codes, d, bits)] * norms[:, None]
    xh = y @ rot.astype(np.float64)
    rel = np.sum((xh - x) ** 2, axis=1) / np.sum(x.astype(np.float64) ** 2, axis=1)
    mse = float(rel.mean())
    assert 4.0 ** -bits < mse < math.sqrt(3) * math.pi / 2 * 4.0 ** -bits
    # the same codes under the transposed rotation reconstruct nothing
    bad = np.sum((y @ rot.astype(np.float64).T - x) ** 2, axis=1) / np.sum(
        x.astype(np.float64) ** 2, axis=1)
    assert bad.mean() > 1.5


def test_encode_then_scan_estimates_inner_products():
    """Scores of encoded vectors estimate <q, x> to within a few times the
    4-bit quantization noise |x| sqrt(D_4 / d), and a vector ranks itself first."""
    d, n, bits = 128, 500, 4
    x = _vectors(n, d, 91, sigma=0.25)
    rot = datagen.orthogonal(92, d).astype(np.float32)
    cb, s = datagen.turboquant_codebook(bits, d)
    codes, norms = oracle.tq_encode(x, rot, d, bits, cb, s)
    q = datagen.unit_rows(x[:40].astype(np.float64)).astype(np.float32)
    _, sc = oracle.tq_scores(q, rot, d, bits, cb, s, codes, norms)
    true = q.astype(np.float64) @ x.astype(np.float64).T
    err = np.abs(sc - true) / np.linalg.norm(x.astype(np.float64), axis=1)[None, :]
    assert err.max() < 6 * math.sqrt(0.0095 / d)
    ids, _ = oracle.tq_topk(q, rot, d, bits, cb, s, codes, norms, 1)
    np.testing.assert_array_equal(ids[:, 0], np.arange(40))


# ----------------------------------------------------------------------- GPU

def _quantizer(rt, d, bits, rot):
    from eos_amd.turboquant import TurboQuantIndex
    cb, s = datagen.turboquant_codebook(bits, d)
    rb = (d * bits + 7) // 8
    return TurboQuantIndex(rt, np.zeros((0, rb), np.uint8), np.zeros(0, np.float32), d, bits, cb,
                           s, rot), cb, s


@pytest.mark.gpu
@pytest.mark.parametrize("d,bits,n,rotate", [(384, 4, 1000, True), (128, 2, 777, True),
                                             (100, 2, 65, False), (768, 4, 33, True),
                                             (1024, 4, 100, True), (513, 4, 50, True),
                                             (31, 2, 3, True)])
def test_encode_bit_exact(rt, d, bits, n, rotate):
    print(f"[case] tq encode d={d} bits={bits} n={n} rotate={rotate}", flush=True)
    x = _vectors(n, d, d + n)
    x[n // 2] = 0.0  # a zero vector: norm 0, every code 0
    rot = datagen.orthogonal(d + 1, d).astype(np.float32) if rotate else None
    tq, cb, s = _quantizer(rt, d, bits, rot)
    got_c, got_n = tq.encode(x)
    want_c, want_n = oracle.tq_encode(x, rot, d, bits, cb, s)
    np.testing.assert_array_equal(got_n, want_n)
    np.testing.assert_array_equal(got_c, want_c)
    assert got_n[n // 2] == 0 and not got_c[n // 2].any()
    tq.release()


@pytest.mark.gpu
def test_encode_device_round_trip_and_validation(rt):
    from eos_amd.runtime import DeviceBuffer
    from eos_amd.turboquant import TurboQuantIndex
    print("[case] tq encode device + round trip", flush=True)
    d, bits, n = 384, 4, 4000
    x = _vectors(n, d, 95, sigma=0.25)
    rot = datagen.orthogonal(96, d).astype(np.float32)
    tq, cb, s = _quantizer(rt, d, bits, rot)
    rb = (d * bits + 7) // 8
    dx = DeviceBuffer.from_array(rt, x)
    dc = DeviceBuffer(rt, n * rb)
    dn = DeviceBuffer(rt, n * 4)
    tq.encode_device(dx, n, dc, dn)
    codes, norms = dc.download(np.uint8, (n, rb)), dn.download(np.float32, n)
    hc, hn = tq.encode(x)
    np.testing.assert_array_equal(codes, hc)
    np.testing.assert_array_equal(norms, hn)
    idx = TurboQuantIndex(rt, codes, norms, d, bits, cb, s, rot)
    q = datagen.unit_rows(x[:64].astype(np.float64)).astype(np.float32)
    ids, sc, _ = idx.top_k(q, 10)
    want_ids, want_sc = oracle.tq_topk(q, rot, d, bits, cb, s, codes, norms, 10)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(sc, want_sc)
    np.testing.assert_array_equal(ids[:, 0], np.arange(64))
    e0c, e0n = tq.encode(np.zeros((0, d), np.float32))
    assert e0c.shape == (0, rb) and e0n.shape == (0,)
    with pytest.raises(ValueError, match="vectors must be"):
        tq.encode(np.zeros((3, d + 1), np.float32))
    for b in (dx, dc, dn):
        b.free()
    idx.release()
    tq.release()


@pytest.mark.gpu
def test_encoder_output_encoded_on_device(rt):
    """Compact embedder forward on device buffers -> TurboQuant encode of its
    output without leaving the device; codes equal the oracle's encode of the
    downloaded embeddings."""
    from eos_amd.encoder import CompactEncoder
    from eos_amd.runtime import DeviceBuffer
    print("[case] compact embed -> tq encode on device", flush=True)
    w = datagen.compact_q8_weights(2, 128, 1, 256, vocab=2000, max_seq=128, seed=97)
    ids, mask, _ = datagen.encoder_batch(48, 128, 2000, 4, 128, 98, 99)
    enc = CompactEncoder(rt, w)
    D = w.output_dim
    rot = datagen.orthogonal(100, D).astype(np.float32)
    tq, cb, s = _quantizer(rt, D, 4, rot)
    d_ids = DeviceBuffer.from_array(rt, ids.astype(np.int32))
    d_mask = DeviceBuffer.from_array(rt, mask.astype(np.int32))
    d_out = DeviceBuffer(rt, 48 * D * 4)
    rb = D // 2
    dc, dn = DeviceBuffer(rt, 48 * rb), DeviceBuffer(rt, 48 * 4)
    enc.embed_device(d_ids, d_mask, 48, 128, d_out)
    tq.encode_device(d_out, 48, dc, dn)
    emb = d_out.download(np.float32, (48, D))
    want_c, want_n = oracle.tq_encode(emb, rot, D, 4, cb, s)
    np.testing.assert_array_equal(dc.download(np.uint8, (48, rb)), want_c)
    np.testing.assert_array_equal(dn.download(np.float32, 48), want_n)
    for b in (d_ids, d_mask, d_out, dc, dn):
        b.free()
    tq.release()
    enc.release()
