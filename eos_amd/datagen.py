"""Seeded synthetic inputs for the benchmark configurations (c1-c5).

Every generator is counter-based (splitmix64 over the element index), so a
(seed, shape) pair always yields the same array on any machine and in any
process; tests, the smoke check and the benchmark all draw from here.
"""
from __future__ import annotations

import math

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Element i is splitmix64's output for state seed + (offset + i + 1) * golden gamma."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, count: int) -> np.ndarray:
    """Uniform doubles in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, count) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, count: int) -> np.ndarray:
    """Standard normal doubles (Box-Muller; u1 in (0, 1])."""
    half = (count + 1) // 2
    u = uniform(seed, 2 * half)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * half, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * math.pi * u2)
    z[1::2] = r * np.sin(2.0 * math.pi * u2)
    return z[:count]


def uniform_int(seed: int, count: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi) (multiply-shift on the top 32 bits)."""
    top = (splitmix64(seed, count) >> np.uint64(32)).astype(np.uint64)
    span = np.uint64(hi - lo)
    return ((top * span) >> np.uint64(32)).astype(np.int64) + lo


def random_bytes(seed: int, count: int) -> np.ndarray:
    words = splitmix64(seed, (count + 7) // 8)
    return words.view(np.uint8)[:count].copy()


def lognormal(seed: int, count: int, sigma: float) -> np.ndarray:
    return np.exp(sigma * normal(seed, count))


def orthogonal(seed: int, d: int) -> np.ndarray:
    """Seeded random orthogonal d x d matrix (QR of a Gaussian, R's diagonal made positive)."""
    g = normal(seed, d * d).reshape(d, d)
    q, r = np.linalg.qr(g)
    q = q * np.sign(np.diag(r))[None, :]
    return q


def unit_rows(x: np.ndarray) -> np.ndarray:
    n = np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True))
    n[n == 0] = 1.0
    return x / n


def lloyd_max_normal(levels: int, iters: int = 500) -> np.ndarray:
    """Lloyd-Max reconstruction points of N(0, 1) (ascending)."""
    def phi(x):
        return math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)

    def cdf(x):
        return 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))

    c = [(-3.0 + 6.0 * (i + 0.5) / levels) for i in range(levels)]
    for _ in range(iters):
        b = [-math.inf] + [(c[i] + c[i + 1]) / 2.0 for i in range(levels - 1)] + [math.inf]
        nc = []
        for i in range(levels):
            lo, hi = b[i], b[i + 1]
            plo = 0.0 if lo == -math.inf else phi(lo)
            phi_hi = 0.0 if hi == math.inf else phi(hi)
            mass = (1.0 if hi == math.inf else cdf(hi)) - (0.0 if lo == -math.inf else cdf(lo))
            nc.append((plo - phi_hi) / mass)
        c = nc
    return np.array(c, dtype=np.float64)


def turboquant_codebook(bits: int, dim: int) -> tuple[np.ndarray, float]:
    """Build-defined TurboQuant codebook on an int8 grid.

    Centroids are the Lloyd-Max points of N(0, 1/dim) (the coordinate law of a
    rotated unit vector), scale s_c = max|c| / 127, grid values round(c / s_c).
    Returns (int8 codes [2^bits], s_c)."""
    c = lloyd_max_normal(1 << bits) / math.sqrt(dim)
    s = float(np.float32(np.max(np.abs(c)) / 127.0))
    grid = np.clip(np.rint(c / s), -127, 127).astype(np.int8)
    return grid, s


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """[n, d] integer codes -> [n, ceil(d*bits/8)] bytes, coordinate j at bits
    j*bits .. j*bits + bits - 1 of the row, low bits first (a 3-bit code may
    straddle two bytes)."""
    n, d = codes.shape
    row_bytes = (d * bits + 7) // 8
    c = codes.astype(np.uint8) & ((1 << bits) - 1)
    bitsv = ((c[:, :, None] >> np.arange(bits, dtype=np.uint8)) & 1).reshape(n, d * bits)
    pad = row_bytes * 8 - d * bits
    bitsv = np.concatenate([bitsv, np.zeros((n, pad), np.uint8)], axis=1)
    return np.packbits(bitsv, axis=1, bitorder="little")


def unpack_codes(packed: np.ndarray, bits: int, d: int) -> np.ndarray:
    """Inverse of pack_codes: [n, row_bytes] -> [n, d] codes."""
    n = packed.shape[0]
    bitsv = np.unpackbits(np.ascontiguousarray(packed, np.uint8), axis=1, bitorder="little")
    bitsv = bitsv[:, :d * bits].reshape(n, d, bits).astype(np.uint8)
    return (bitsv << np.arange(bits, dtype=np.uint8)).sum(axis=2).astype(np.uint8)


class TurboQuantCorpus:
    """Synthetic TurboQuant corpus of the benchmark's flat / multivector configs."""

    def __init__(self, n: int, dim: int, bits: int, seed_codes: int, seed_norms: int,
                 seed_rot: int, norm_sigma: float = 0.25, rotation: bool = True):
        self.n, self.dim, self.bits = n, dim, bits
        row_bytes = (dim * bits + 7) // 8
        if bits == 4 or bits == 2:
            # Uniform codes: every packed byte is uniform over [0, 256).
            self.codes = random_bytes(seed_codes, n * row_bytes).reshape(n, row_bytes)
            if (dim * bits) % 8:
                keep = (dim * bits) % 8
                self.codes[:, -1] &= np.uint8((1 << keep) - 1)
        else:
            raise ValueError("bits must be 2 or 4")
        self.norms = lognormal(seed_norms, n, norm_sigma).astype(np.float32)
        self.rotation = orthogonal(seed_rot, dim).astype(np.float32) if rotation else None
        self.codebook, self.codebook_scale = turboquant_codebook(bits, dim)


def baseline_flat_corpus(n: int = 1_000_000, dim: int = 384) -> TurboQuantCorpus:
    """Benchmark config c2: 4-bit codes (seed 3), lognormal(0, 0.25) norms (seed 4), rotation seed 5."""
    return TurboQuantCorpus(n, dim, 4, seed_codes=3, seed_norms=4, seed_rot=5)


def baseline_queries(q: int, dim: int, seed: int = 6) -> np.ndarray:
    """Gaussian queries, unit-normalized in f64, stored f32."""
    return unit_rows(normal(seed, q * dim).reshape(q, dim)).astype(np.float32)


def bert_q8_weights(layers: int, hidden: int, heads: int, inter: int, vocab: int, npos: int,
                    ntype: int = 2, seed: int = 7, eps: float = 1e-12, gelu: int = 1,
                    random_affine: bool = False, peaked: dict | None = None):
    """Random-init BERT-style encoder (weights N(0, 0.02)) quantized to int8
    per output channel. With random_affine, biases, LayerNorm gamma/beta are
    drawn too (otherwise biases 0, gamma 1, beta 0).

    peaked = {"alpha": a, "beta": b, "tokens": {id: mix}} plants peaked
    attention: with u = (+1, -1, ...) / sqrt(H) and w = (+1, +1, -1, -1, ...)
    / sqrt(H), token `id`'s embedding row becomes 3 (mix u + sqrt(1 - mix^2)
    w), every layer's query bias gets b and its key weights a u^T on the first
    feature of each head. Every query then scores such a key about
    a b mix sqrt(H) / sqrt(hd) above the others (40 nats at a = 4, b = 3, mix
    1, H = 384, hd = 32), so the key's position decides in which key block the
    softmax maximum appears."""
    from .encoder import EncoderLayerWeights, EncoderWeights, quantize_per_channel

    counter = [seed * 1000003]

    def draw(shape, std=0.02):
        counter[0] += 1
        n = int(np.prod(shape))
        return (std * normal(counter[0], n)).astype(np.float32).reshape(shape)

    def vec(n, base=0.0, std=0.02):
        if not random_affine:
            return np.full(n, base, np.float32)
        return (base + draw((n,), std)).astype(np.float32)

    H, F = hidden, inter
    tok = draw((vocab, H))
    pos = draw((npos, H))
    typ = draw((ntype, H))
    hd = H // heads
    if peaked is not None:
        u = np.where(np.arange(H) % 2 == 0, 1.0, -1.0) / np.sqrt(H)
        wdir = np.where((np.arange(H) // 2) % 2 == 0, 1.0, -1.0) / np.sqrt(H)
        for tid, mix in peaked["tokens"].items():
            tok[tid] = (3.0 * (mix * u + np.sqrt(max(0.0, 1.0 - mix * mix)) * wdir)).astype(np.float32)
    w = EncoderWeights(hidden=H, heads=heads, intermediate=F, ln_eps=eps, gelu=gelu, tok=tok,
                       pos=pos, typ=typ, emb_gamma=vec(H, 1.0, 0.1), emb_beta=vec(H, 0.0, 0.05))
    for _ in range(layers):
        # Draw order as before the peaked option (same weights for every seed).
        wqkv = draw((3 * H, H))
        wo, so = quantize_per_channel(draw((H, H)))
        w1, s1 = quantize_per_channel(draw((F, H)))
        w2, s2 = quantize_per_channel(draw((H, F)))
        bqkv = vec(3 * H)
        if peaked is not None:
            for h in range(heads):
                wqkv[H + h * hd] += np.float32(peaked["alpha"]) * u.astype(np.float32)
                bqkv[h * hd] = np.float32(peaked["beta"])
        qkv, sq = quantize_per_channel(wqkv)
        w.layers.append(EncoderLayerWeights(
            w_qkv=qkv, s_qkv=sq, b_qkv=bqkv, w_o=wo, s_o=so, b_o=vec(H),
            ln1_gamma=vec(H, 1.0, 0.1), ln1_beta=vec(H, 0.0, 0.05), w_1=w1, s_1=s1, b_1=vec(F),
            w_2=w2, s_2=s2, b_2=vec(H), ln2_gamma=vec(H, 1.0, 0.1), ln2_beta=vec(H, 0.0, 0.05)))
    return w


def compact_q8_weights(layers: int, dim: int, heads: int, ffn: int, vocab: int, max_seq: int,
                       out_dim: int | None = None, seed: int = 7, bits: int = 8):
    """Random-init compact (family (a)) embedder, quantized per tensor on the
    reference's q8/q4 grid. Embedding tables are N(0, 0.02); dense weights are
    N(0, 1/fan_in) so attention logits are O(1) once LayerNorm has run."""
    from .encoder import CompactLayerWeights, CompactWeights, quantize_per_tensor

    counter = [seed * 1000033]

    def draw(shape, std):
        counter[0] += 1
        n = int(np.prod(shape))
        w = (std * normal(counter[0], n)).astype(np.float32).reshape(shape)
        return quantize_per_tensor(w, bits)

    D, F = dim, ffn
    tok, st = draw((vocab, D), 0.02)
    role, sr = draw((3, D), 0.02)
    w = CompactWeights(model_dim=D, heads=heads, hidden_dim=F, max_sequence=max_seq,
                       token_embedding=tok, s_token=st, role_embedding=role, s_role=sr)
    for _ in range(layers):
        q, sq = draw((D, D), D ** -0.5)
        k, sk = draw((D, D), D ** -0.5)
        v, sv = draw((D, D), D ** -0.5)
        o, so = draw((D, D), D ** -0.5)
        up, su = draw((D, F), D ** -0.5)
        dn, sd = draw((F, D), F ** -0.5)
        w.layers.append(CompactLayerWeights(attn_q=q, s_q=sq, attn_k=k, s_k=sk, attn_v=v, s_v=sv,
                                            attn_o=o, s_o=so, ffn_up=up, s_up=su, ffn_down=dn,
                                            s_down=sd))
    if out_dim is not None and out_dim != D:
        w.output_projection, w.s_output = draw((D, out_dim), D ** -0.5)
    return w


def encoder_batch(batch: int, tokens: int, vocab: int, lo: int, hi: int, seed_ids: int,
                  seed_len: int):
    """Token ids uniform over [0, vocab), valid lengths uniform in [lo, hi];
    mask[b, t] = t < len_b (right padding, runtime/embedding_model.go:1457-1495)."""
    ids = uniform_int(seed_ids, batch * tokens, 0, vocab).astype(np.int32).reshape(batch, tokens)
    lens = uniform_int(seed_len, batch, lo, hi + 1).astype(np.int32)
    mask = (np.arange(tokens)[None, :] < lens[:, None]).astype(np.int32)
    ids = np.where(mask == 1, ids, 0).astype(np.int32)
    return ids, mask, lens
