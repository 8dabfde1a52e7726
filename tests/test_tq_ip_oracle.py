"""Pins the CPU restatement of the inner-product TurboQuant layout (MSE codes
+ QJL signs + ResNorm + Norm; oracle/tq_oracle.c tq_encode_ip /
tq_ip_scores), test infrastructure for eos_tq_encode_ip / eos_tq_ip_*.

The quantizer is in the un-vendored module, so the pins are what the
mathematics fixes:
* signs and ResNorm against the residual computed independently in numpy
  (f64), and the packing of the sign bits;
* the QJL identity E[sign(<s, r>) <s, y>] = sqrt(2 / pi) <r, y> / |r| for
  Gaussian s: over many sketch matrices the IP estimate is unbiased for
  <q, x>, where the 1-bit MSE estimate alone is biased by about 2 / pi
  (TurboQuant_prod, Zandieh et al. 2025);
* the estimator's variance bound pi / 2 - 1 per unit |r| |y| / d;
* the byte accounting MSE + signs + 8 (runtime/turboquant_bytes.go:14-25)."""
import numpy as np

import oracle


def _setup(d, bits, seed):
    rng = np.random.default_rng(seed)
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32)
    levels = 1 << bits
    # Lloyd-Max-like symmetric grid for N(0, 1/d) on int8 codes
    pts = np.sort(rng.normal(size=levels))
    cb = np.clip(np.rint(pts / np.abs(pts).max() * 127), -127, 127).astype(np.int8)
    if bits == 1:
        cb = np.array([-127, 127], np.int8)
    s_c = float(np.float32(0.8 * np.sqrt(2 / np.pi) / np.sqrt(d) / 127 if bits == 1 else
                           2.5 / np.sqrt(d) / 127))
    return rng, rot, cb, s_c


def test_signs_and_resnorm_match_independent_residual():
    d, bits = 48, 2
    rng, rot, cb, s_c = _setup(d, bits, 0)
    S = rng.normal(size=(d, d)).astype(np.float32)
    x = rng.normal(size=(20, d)).astype(np.float32)
    codes, signs, rn, nm = oracle.tq_encode_ip(x, rot, S, d, bits, cb, s_c)
    c_mse, n_mse = oracle.tq_encode(x, rot, d, bits, cb, s_c)
    np.testing.assert_array_equal(codes, c_mse)
    np.testing.assert_array_equal(nm, n_mse)
    for i in range(20):
        u = rot.astype(np.float64) @ x[i].astype(np.float64)
        nrm = np.linalg.norm(x[i].astype(np.float64))
        bitsv = np.unpackbits(codes[i], bitorder="little").reshape(-1, bits)
        code = (bitsv * (1 << np.arange(bits))).sum(1)[:d]
        r = u - nrm * (s_c * cb[code].astype(np.float64))
        assert abs(rn[i] - np.linalg.norm(r) / nrm) <= 1e-6 * rn[i] + 1e-12
        p = S.astype(np.float64) @ r
        got = np.unpackbits(signs[i], bitorder="little")[:d]
        sure = np.abs(p) > 1e-9 * np.abs(S).sum(1) * np.abs(r).max()
        np.testing.assert_array_equal(got[sure], (p >= 0)[sure])
    assert codes.shape[1] + signs.shape[1] + 8 == (d * bits + 7) // 8 + (d + 7) // 8 + 8


def test_estimator_unbiased_over_sketches():
    """Average over 300 sketch matrices: the IP estimate's bias is within a
    few standard errors of 0, while the 1-bit MSE estimate alone (S = 0
    sketch term dropped) sits near 2 / pi of the true product."""
    d, bits = 64, 1
    rng, rot, cb, s_c = _setup(d, bits, 1)
    x = rng.normal(size=(1, d)).astype(np.float32)
    q = (x + 0.6 * rng.normal(size=(1, d))).astype(np.float32)
    true = float(q[0].astype(np.float64) @ x[0].astype(np.float64))
    est = []
    for t in range(300):
        S = rng.normal(size=(d, d)).astype(np.float32)
        codes, signs, rn, nm = oracle.tq_encode_ip(x, rot, S, d, bits, cb, s_c)
        est.append(oracle.tq_ip_scores(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm)[0, 0])
    est = np.array(est, np.float64)
    se = est.std() / np.sqrt(len(est))
    assert abs(est.mean() - true) < 4 * se + 1e-3 * abs(true)
    # Variance of the 1-bit sketch over S: per row E[t^2] = |y|^2 and
    # E[t] = sqrt(2 / pi) <r^, y>, so Var = (pi / 2 |y|^2 - <r^, y>^2) |r|^2 / d
    # with y = R q and r the rotated-frame residual.
    u = rot.astype(np.float64) @ x[0].astype(np.float64)
    nrm = float(nm[0])
    bitsv = np.unpackbits(codes[0], bitorder="little")[:d]
    r = u - nrm * s_c * cb[bitsv].astype(np.float64)
    y = rot.astype(np.float64) @ q[0].astype(np.float64)
    rhat = r / np.linalg.norm(r)
    want = (np.pi / 2 * (y @ y) - (rhat @ y) ** 2) * (r @ r) / d
    assert 0.7 * want < est.var() < 1.3 * want
    # the MSE part alone (no residual term) is biased low at 1 bit
    zero = np.zeros_like(signs)
    mse_only = oracle.tq_ip_scores(q, rot, np.zeros((d, d), np.float32), d, bits, cb, s_c, codes,
                                   zero, np.zeros_like(rn), nm)[0, 0]
    assert mse_only < 0.85 * true


def test_scores_zero_norm_and_residual_free_vector():
    """A zero vector scores 0; with ResNorm 0 the estimate is the MSE score."""
    d, bits = 32, 4
    rng, rot, cb, s_c = _setup(d, bits, 2)
    S = rng.normal(size=(d, d)).astype(np.float32)
    x = rng.normal(size=(3, d)).astype(np.float32)
    x[1] = 0
    codes, signs, rn, nm = oracle.tq_encode_ip(x, rot, S, d, bits, cb, s_c)
    assert nm[1] == 0 and rn[1] == 0
    q = rng.normal(size=(2, d)).astype(np.float32)
    sc = oracle.tq_ip_scores(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm)
    assert np.all(sc[:, 1] == 0)
    _, mse = oracle.tq_scores(q, rot, d, bits, cb, s_c, codes, nm)
    no_res = oracle.tq_ip_scores(q, rot, S, d, bits, cb, s_c, codes, signs, np.zeros_like(rn), nm)
    np.testing.assert_array_equal(no_res, mse)
