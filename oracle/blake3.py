"""BLAKE3 hash mode in plain Python (test infrastructure only: the checker of
the library's section-digest verification, never on a product path).

Written from the BLAKE3 specification: 1 KiB chunks of 64-byte blocks, the
seven-round compression function with the message permutation, chaining
values merged into a binary tree as chunks complete, ROOT on the final
compression. Pinned in the tests by the published digest of the empty input
and by the section digests stored in the packages the reference ships
(written by m31labs.dev/mll v0.1.0)."""
from __future__ import annotations

IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A,
      0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
CHUNK_START, CHUNK_END, PARENT, ROOT = 1, 2, 4, 8
M32 = 0xFFFFFFFF
EMPTY_DIGEST = "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"


def _rotr(x: int, n: int) -> int:
    return ((x >> n) | (x << (32 - n))) & M32


def _g(s, a, b, c, d, x, y):
    s[a] = (s[a] + s[b] + x) & M32
    s[d] = _rotr(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b] + y) & M32
    s[d] = _rotr(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 7)


def _compress(cv, block: bytes, counter: int, blen: int, flags: int):
    m = [int.from_bytes(block[4 * i:4 * i + 4], "little") for i in range(16)]
    s = list(cv[:8]) + list(IV[:4]) + [counter & M32, (counter >> 32) & M32, blen, flags]
    for r in range(7):
        _g(s, 0, 4, 8, 12, m[0], m[1])
        _g(s, 1, 5, 9, 13, m[2], m[3])
        _g(s, 2, 6, 10, 14, m[4], m[5])
        _g(s, 3, 7, 11, 15, m[6], m[7])
        _g(s, 0, 5, 10, 15, m[8], m[9])
        _g(s, 1, 6, 11, 12, m[10], m[11])
        _g(s, 2, 7, 8, 13, m[12], m[13])
        _g(s, 3, 4, 9, 14, m[14], m[15])
        if r < 6:
            m = [m[PERM[i]] for i in range(16)]
    return [s[i] ^ s[i + 8] for i in range(8)]


def _chunk(data: bytes, index: int, root: bool):
    cv = list(IV)
    nblocks = max(1, (len(data) + 63) // 64)
    for b in range(nblocks):
        blk = data[64 * b:64 * b + 64]
        flags = (CHUNK_START if b == 0 else 0) | (CHUNK_END if b == nblocks - 1 else 0)
        if root and b == nblocks - 1:
            flags |= ROOT
        cv = _compress(cv, blk.ljust(64, b"\0"), index, len(blk), flags)
    return cv


def _parent(left, right, root: bool):
    blk = b"".join(w.to_bytes(4, "little") for w in list(left) + list(right))
    return _compress(IV, blk, 0, 64, PARENT | (ROOT if root else 0))


def blake3(data: bytes) -> bytes:
    """32-byte BLAKE3 digest of data."""
    n = max(1, (len(data) + 1023) // 1024)
    if n == 1:
        cv = _chunk(data, 0, True)
    else:
        stack = []
        for i in range(n - 1):
            cv = _chunk(data[1024 * i:1024 * i + 1024], i, False)
            total = i + 1
            while total & 1 == 0:
                cv = _parent(stack.pop(), cv, False)
                total >>= 1
            stack.append(cv)
        cv = _chunk(data[1024 * (n - 1):], n - 1, False)
        while len(stack) > 1:
            cv = _parent(stack.pop(), cv, False)
        cv = _parent(stack.pop(), cv, True)
    return b"".join(w.to_bytes(4, "little") for w in cv)
