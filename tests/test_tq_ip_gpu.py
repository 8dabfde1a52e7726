"""GPU parity of the inner-product TurboQuant layout (eos_tq_encode_ip,
eos_tq_ip_prepare, eos_tq_ip_scores) against its CPU restatement. Bar:
bit-exact codes, signs, ResNorm, Norm and f32 scores; top-k ids exact."""
import numpy as np
import pytest

import oracle
from eos_amd.turboquant import IPQuantizer

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


@pytest.mark.parametrize("d,bits,n,rotate", [(384, 4, 3000, True), (256, 2, 1001, True),
                                             (128, 1, 777, False), (1000, 4, 100, True),
                                             (37, 2, 65, True), (384, 3, 2000, True),
                                             (29, 3, 99, False)])
def test_ip_layout_matches_oracle(rt, d, bits, n, rotate):
    _case(f"ip layout d={d} bits={bits} n={n} rotate={rotate}")
    rng = np.random.default_rng(d * 7 + bits)
    rot = np.linalg.qr(rng.normal(size=(d, d)))[0].astype(np.float32) if rotate else None
    S = rng.normal(size=(d, d)).astype(np.float32)
    levels = 1 << bits
    cb = np.linspace(-127, 127, levels).round().astype(np.int8)
    s_c = float(np.float32(2.5 / np.sqrt(d) / 127))
    x = rng.normal(size=(n, d)).astype(np.float32)
    x[3] = 0
    iq = IPQuantizer(rt, d, bits, cb, s_c, rot, S)
    codes, signs, rn, nm = iq.encode(x)
    wc, ws, wr, wn = oracle.tq_encode_ip(x, rot, S, d, bits, cb, s_c)
    np.testing.assert_array_equal(codes, wc)
    np.testing.assert_array_equal(signs, ws)
    np.testing.assert_array_equal(rn, wr)
    np.testing.assert_array_equal(nm, wn)
    assert iq.vector_bytes() == codes.shape[1] + signs.shape[1] + 8
    q = rng.normal(size=(11, d)).astype(np.float32)
    sc, tid, tsc = iq.scores(q, codes, signs, rn, nm, k=50)
    want = oracle.tq_ip_scores(q, rot, S, d, bits, cb, s_c, codes, signs, rn, nm)
    np.testing.assert_array_equal(sc, want)
    for i in range(q.shape[0]):
        ids, tops = oracle.topk_scores(want[i], 50)
        np.testing.assert_array_equal(tid[i], ids)
        np.testing.assert_array_equal(tsc[i], tops)
    iq.release()
