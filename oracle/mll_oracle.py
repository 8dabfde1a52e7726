"""MLL package reader in plain Python (test infrastructure only: the checker
of libeoship's eoship_mll_* reader, never on a product path).

A second, independent restatement of the container the reference writes
through m31labs.dev/mll v0.1.0 (artifact/eos/mll.go:112-330,
runtime/weight_file.go:122-229; the module itself is not vendored, so the
framing follows the bytes of the packages the reference ships and their
BLAKE3 section digests):

  header   "MLL\\0", version bytes 0x00 0x01, profile byte, reserved byte,
           u64 file size, u64 section count
  entry    64 bytes each from offset 24: tag, u64 offset, u64 size,
           digest[32], u16 flags, u16 schema version, 8 reserved bytes
  STRG     u64 count (implicit "" at index 0 counted), count - 1 x (u32 len, bytes)
  TNSR     u32 count, per tensor u32 name, u8 dtype, u32 rank, u64 dims,
           u64 offset, u64 size (relative to the body), u32 reserved
  XMTA     MLLMetadata JSON (artifact/eos/mll.go:24-34)

Q8 payloads decode as int8 code * tensor_scales[name] and Q4 payloads as
(nibble - 8) * scale, low nibble first (decodeTensorEntry,
runtime/weight_file.go:305-415). The writer below builds synthetic packages
for the tests; its digests come from the caller's hash function.
"""
from __future__ import annotations

import json
import struct

import numpy as np

DTYPE_Q8 = 13
MAGIC = b"MLL\0"


def read(data: bytes, digest=None) -> dict:
    """Parse a package. digest: optional callable(bytes) -> 32 bytes used to
    check every section but XKBI."""
    if data[:4] != MAGIC:
        raise ValueError("not an MLL file")
    size, count = struct.unpack_from("<QQ", data, 8)
    if size != len(data):
        raise ValueError("file size mismatch")
    sections = {}
    for i in range(count):
        e = data[24 + 64 * i:24 + 64 * (i + 1)]
        tag = e[:4].decode("latin-1")
        off, n = struct.unpack_from("<QQ", e, 4)
        flags, schema = struct.unpack_from("<HH", e, 52)
        sections[tag] = {"offset": off, "size": n, "digest": e[20:52], "flags": flags,
                         "schema": schema}
        if digest is not None and tag != "XKBI":
            if digest(data[off:off + n]) != e[20:52]:
                raise ValueError(f"section {tag} digest mismatch")
    s = sections["STRG"]
    body = data[s["offset"]:s["offset"] + s["size"]]
    (nstr,) = struct.unpack_from("<Q", body, 0)
    strings, q = [""], 8
    for _ in range(nstr - 1):
        (ln,) = struct.unpack_from("<I", body, q)
        strings.append(body[q + 4:q + 4 + ln].decode("utf-8"))
        q += 4 + ln
    meta = None
    if "XMTA" in sections:
        x = sections["XMTA"]
        meta = json.loads(data[x["offset"]:x["offset"] + x["size"]])
    scales = (meta or {}).get("tensor_scales", {})
    logical = (meta or {}).get("logical_tensor_dtypes", {})
    t = sections["TNSR"]
    body = data[t["offset"]:t["offset"] + t["size"]]
    (ntens,) = struct.unpack_from("<I", body, 0)
    tensors, q = {}, 4
    for _ in range(ntens):
        name_idx, dtype, rank = struct.unpack_from("<IBI", body, q)
        q += 9
        dims = struct.unpack_from(f"<{rank}Q", body, q)
        q += 8 * rank
        off, n, _reserved = struct.unpack_from("<QQI", body, q)
        q += 20
        name = strings[name_idx]
        payload = body[off:off + n]
        count_el = int(np.prod(dims)) if dims else 1
        ent = {"dtype": dtype, "shape": tuple(int(d) for d in dims), "payload": payload,
               "scale": float(np.float32(scales.get(name, 0.0))), "logical": logical.get(name)}
        if dtype == DTYPE_Q8:
            ent["codes"] = np.frombuffer(payload, np.int8).reshape(ent["shape"])
        elif ent["logical"] == "q4" and n == (count_el + 1) // 2:
            nib = np.frombuffer(payload, np.uint8)
            both = np.stack([nib & 0xF, nib >> 4], axis=1).reshape(-1)[:count_el]
            ent["codes"] = (both.astype(np.int16) - 8).astype(np.int8).reshape(ent["shape"])
        if "codes" in ent:
            sc = np.float32(ent["scale"])
            ent["values"] = ent["codes"].astype(np.float32) * sc
        tensors[name] = ent
    return {"sections": sections, "strings": strings, "tensors": tensors, "meta": meta,
            "profile": data[6]}


def write(sections: list[tuple[str, bytes, int]], digest, profile: int = 1,
          bad_digest: set[str] | None = None) -> bytes:
    """A container of (tag, body, flags) sections; digest: callable(bytes) ->
    32 bytes. Tags in bad_digest get a wrong digest."""
    count = len(sections)
    head = 24 + 64 * count
    out = bytearray()
    offsets, cursor = [], head
    for tag, body, flags in sections:
        if flags & 0x10:  # aligned sections start on a 4 KiB boundary
            cursor = (cursor + 4095) // 4096 * 4096
        offsets.append(cursor)
        cursor += len(body)
    total = cursor
    out += MAGIC + bytes([0x00, 0x01, profile, 0]) + struct.pack("<QQ", total, count)
    for (tag, body, flags), off in zip(sections, offsets):
        d = digest(body)
        if bad_digest and tag in bad_digest:
            d = bytes(32 * [0x5A])
        out += tag.encode("latin-1") + struct.pack("<QQ", off, len(body)) + d
        out += struct.pack("<HH", flags, 1) + bytes(8)
    for (tag, body, flags), off in zip(sections, offsets):
        out += bytes(off - len(out))
        out += body
    return bytes(out)


def strg_body(strings: list[str]) -> bytes:
    """STRG body for strings[0] == "" followed by the rest."""
    assert strings and strings[0] == ""
    b = struct.pack("<Q", len(strings))
    for s in strings[1:]:
        e = s.encode("utf-8")
        b += struct.pack("<I", len(e)) + e
    return b


def tnsr_body(entries: list[tuple[int, int, tuple, bytes]]) -> bytes:
    """TNSR body for (name index, dtype, dims, payload) entries; payloads
    64-byte aligned after the table."""
    hdr = 4 + sum(9 + 8 * len(d) + 20 for _, _, d, _ in entries)
    off = (hdr + 63) // 64 * 64
    table, data = struct.pack("<I", len(entries)), b""
    for name, dtype, dims, payload in entries:
        table += struct.pack("<IBI", name, dtype, len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        table += struct.pack("<QQI", off + len(data), len(payload), 0)
        data += payload
        pad = (-len(data)) % 64
        data += bytes(pad)
    return table + bytes(off - len(table)) + data
