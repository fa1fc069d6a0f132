"""GGUF and .spm file readers restated in plain Python -- TEST INFRASTRUCTURE ONLY.

The checker for the library's C++ file code: the same parse, in the same
order, with the same error texts, written from the reference's Rust.  Only
tests use it.

Pinned by (tests/test_files.py):
  * the reference's own known-answer cases: spm-gguf/tests/safety.rs (bad
    magic, unbounded metadata count, unbounded string, range beyond the file,
    the tiny aligned fixture and its range reads); the hand-written golden
    file spm-file/tests/golden/tiny.spm (kept as tests/golden/tiny.spm) with
    the offsets docs/spm-format.md documents and the two groups it holds;
    spm-file/tests/errors.rs (truncated payload: 5 needed, 4 remain; bad
    magic; incomplete file; wrong group length), encodings.rs (mixed-encoding
    file of 32 + 64 + 5 + 20 bytes; (count, bytes) per group for a
    non-dividing group size) and roundtrip.rs (a multi-stream file);
  * a writer/reader round trip over random descriptors;
  * byte-level agreement with the library on random well-formed files and on
    every single-byte truncation and random corruption of them.
"""
from __future__ import annotations

import struct

# spm-gguf/src/lib.rs:11-16
MAX_METADATA = 1_000_000
MAX_TENSORS = 1_000_000
MAX_STRING = 16 * 1024 * 1024
MAX_ARRAY = 2_000_000
MAX_DIMS = 8
MAX_HEADER_BYTES = 512 * 1024 * 1024
U64 = (1 << 64) - 1


class Refused(Exception):
    """The reference's Err(String) / error enum, by its message."""


def ggml_layout(t: int):
    """(elements, bytes) per block (spm-gguf/src/parse.rs:10-29)."""
    return {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
            9: (32, 40), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
            15: (256, 292), 16: (1, 8)}.get(t)


class _Wire:  # spm-gguf/src/wire.rs:4-91
    def __init__(self, data: bytes):
        self.d, self.pos = data, 0

    def bytes(self, n):
        end = self.pos + n
        if end > U64:
            raise Refused("file position overflow")
        if end > MAX_HEADER_BYTES:
            raise Refused("GGUF header exceeds limit")
        if end > len(self.d):
            raise Refused("unexpected end of GGUF")
        out = self.d[self.pos:end]
        self.pos = end
        return out

    def u(self, fmt):
        return struct.unpack("<" + fmt, self.bytes(struct.calcsize(fmt)))[0]

    def string(self):
        n = self.u("Q")
        if n > MAX_STRING:
            raise Refused(f"string length {n} exceeds limit")
        raw = self.bytes(n)
        try:
            return raw.decode("utf-8", errors="strict")
        except UnicodeDecodeError:
            raise Refused("invalid UTF-8 string") from None

    def value(self, ty, depth):
        if depth > 4:
            raise Refused("metadata nesting exceeds limit")
        scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 10: "Q", 11: "q"}
        if ty in scalar:
            return str(self.u(scalar[ty]))
        if ty == 6:
            self.bytes(4)
            return None
        if ty == 7:
            v = self.u("B")
            if v > 1:
                raise Refused("invalid boolean metadata value")
            return str(v)
        if ty == 8:
            return self.string()
        if ty == 9:
            inner, n = self.u("I"), self.u("Q")
            if n > MAX_ARRAY:
                raise Refused(f"array length {n} exceeds limit")
            for _ in range(n):
                self.value(inner, depth + 1)
            return None
        if ty == 12:
            self.bytes(8)
            return None
        raise Refused(f"unknown metadata type {ty}")


def gguf_read(data: bytes) -> dict:
    """spm-gguf/src/parse.rs:157-182 over the file's bytes: version,
    metadata_count, tensor_data_offset, metadata, tensors (ascending offset,
    each (name, dims, dtype, offset, len))."""
    p = _Wire(data)
    if p.bytes(4) != b"GGUF":  # prelude, parse.rs:31-48
        raise Refused("invalid GGUF magic")
    version = p.u("I")
    if version != 3:
        raise Refused(f"unsupported GGUF version {version}")
    tensors, metadata = p.u("Q"), p.u("Q")
    if tensors > MAX_TENSORS:
        raise Refused("tensor count exceeds limit")
    if metadata > MAX_METADATA:
        raise Refused("metadata count exceeds limit")
    meta = {}
    for _ in range(metadata):  # parse.rs:50-63
        key = p.string()
        ty = p.u("I")
        v = p.value(ty, 0)
        if key in meta:
            raise Refused("duplicate metadata key")
        meta[key] = v if v is not None else f"<{ty}>"
    raw, names = [], set()
    for _ in range(tensors):  # parse.rs:65-92
        name = p.string()
        if name in names:
            raise Refused(f"duplicate tensor name {name}")
        names.add(name)
        nd = p.u("I")
        if nd == 0 or nd > MAX_DIMS:
            raise Refused(f"invalid dimension count {nd}")
        dims = tuple(p.u("Q") for _ in range(nd))
        raw.append((name, dims, p.u("I"), p.u("Q")))
    align = 32
    a = meta.get("general.alignment")  # str::parse::<u64>: optional '+', ASCII digits, fits u64
    if a is not None:
        digits = a[1:] if a.startswith("+") else a
        if digits and digits.isascii() and digits.isdigit() and int(digits) <= U64:
            align = int(digits)
    if align == 0 or align & (align - 1):
        raise Refused("invalid alignment")
    if p.pos + align - 1 > U64:
        raise Refused("alignment overflow")
    base = (p.pos + align - 1) & ~(align - 1)
    if base > len(data):
        raise Refused("tensor data starts beyond file")
    out = []
    for name, dims, dtype, off in raw:  # ranges, parse.rs:94-140
        if off % align:
            raise Refused(f"unaligned tensor {name}")
        if 0 in dims:
            raise Refused(f"tensor {name} has a zero dimension")
        elems = 1
        for d in dims:
            elems *= d
            if elems > U64:
                raise Refused("tensor element count overflow")
        lay = ggml_layout(dtype)
        if lay is None:
            raise Refused(f"unsupported GGML dtype {dtype}")
        block, size = lay
        if elems % block:
            raise Refused(f"tensor {name} does not fill dtype blocks")
        n = elems // block * size
        if n > U64:
            raise Refused("tensor byte length overflow")
        start = base + off
        if start > U64:
            raise Refused("tensor offset overflow")
        if start + n > U64:
            raise Refused("tensor end overflow")
        if start + n > len(data):
            raise Refused(f"tensor {name} extends beyond file")
        out.append((name, dims, dtype, start, n))
    out.sort(key=lambda t: t[3])  # stable, as sort_by_key
    for a_, b_ in zip(out, out[1:]):  # reject_overlaps, parse.rs:142-154
        if a_[3] + a_[4] > b_[3]:
            raise Refused("overlapping tensor ranges")
    return {"version": version, "metadata_count": metadata, "tensor_data_offset": base, "metadata": meta,
            "tensors": out}


def gguf_read_range(data: bytes, tensor, relative_offset: int, length: int, max_bytes: int) -> bytes:
    """spm-gguf/src/tensor.rs:35-67; tensor is (name, dims, dtype, offset, len)."""
    name, _, _, offset, tlen = tensor
    if length > max_bytes:
        raise Refused(f"tensor {name} request is {length} bytes, exceeding limit {max_bytes}")
    if relative_offset + length > U64:
        raise Refused("tensor range overflow")
    if relative_offset + length > tlen:
        raise Refused(f"requested range exceeds tensor {name}")
    start = offset + relative_offset
    return data[start:start + length]


# ------------------------------------------------------------------ .spm --

MAGIC = bytes([0x89, 0x53, 0x50, 0x4D, 0x0D, 0x0A, 0x1A, 0x0A])  # spm-header/src/model.rs:4


def spm_bytes_for(encoding: int, count: int) -> int:
    """spm-layout/src/model.rs:80-91."""
    if encoding == 1:
        return (count + 3) // 4
    if encoding == 2:
        return count * 4
    if encoding == 3:
        return count * 2
    if encoding == 4:
        return (count + 255) // 256 * 210
    if encoding == 5:
        return (count + 255) // 256 * 176
    if encoding == 6:
        return (count + 31) // 32 * 34
    raise Refused(f"unknown .spm encoding profile {encoding}")


def spm_header(src: bytes):
    """spm-header/src/parse.rs:12-58: (major, minor, stream_count)."""
    if len(src) < 32:
        raise Refused(f"header truncated: {len(src)} bytes available, need 32")
    if src[:8] != MAGIC:
        raise Refused("bad magic: not a .spm file, or corrupted in transit")
    major, minor = struct.unpack_from("<HH", src, 8)
    if major > 1:
        raise Refused(f"unsupported .spm major version {major}: this build reads up to 1")
    if src[12] != 0:
        raise Refused(f"unknown endianness discriminant {src[12]}")
    return major, minor, struct.unpack_from("<I", src, 16)[0]


def spm_descriptor(src: bytes):
    """spm-layout/src/wire.rs:12-29: (rows, cols, group_size, encoding, lane_count)."""
    if len(src) < 32:
        raise Refused(f"descriptor truncated: {len(src)} bytes, need 32")
    rows, cols, gs = struct.unpack_from("<III", src, 0)
    if gs == 0:
        raise Refused("group_size must be at least 1")
    if src[12] not in (1, 2, 3, 4, 5, 6):
        raise Refused(f"unknown .spm encoding profile {src[12]}")
    return rows, cols, gs, src[12], struct.unpack_from("<H", src, 14)[0]


def _group_lens(desc):
    """spm-walk cursor order: (stream, weights) per group, zero-weight streams skipped
    (spm-walk/src/cursor.rs:6-58, spm-layout/src/tiling.rs:24-51)."""
    for s, (rows, cols, gs, _, _) in enumerate(desc):
        total = rows * cols
        for g in range((total + gs - 1) // gs):
            yield s, min(gs, total - g * gs)


def spm_read(src: bytes):
    """SpmReader::parse then next_group until None (read.rs:48-101):
    (header, descriptors, groups, error) where groups are
    (stream, scale, count, packed) and error is the PayloadTruncated message
    that stopped the walk, or None."""
    header = spm_header(src)
    desc, at = [], 32
    for _ in range(header[2]):
        desc.append(spm_descriptor(src[at:] if at <= len(src) else b""))
        at += 32
    payload = src[min(at, len(src)):]
    pos, groups = 0, []
    for s, count in _group_lens(desc):
        needed = 4 + spm_bytes_for(desc[s][3], count)
        available = max(len(payload) - pos, 0)
        if needed > available:
            return header, desc, groups, f"payload truncated: group needs {needed} bytes, {available} remain"
        scale = struct.unpack_from("<f", payload, pos)[0]
        groups.append((s, scale, count, payload[pos + 4:pos + needed]))
        pos += needed
    return header, desc, groups, None


def spm_write(desc, groups) -> bytes:
    """SpmWriter (write.rs:23-107) given every group as (scale, payload,
    count) in stream order; refuses what the writer refuses."""
    out = bytearray(MAGIC + struct.pack("<HHB3xI12x", 1, 0, 0, len(desc)))
    for rows, cols, gs, enc, lanes in desc:
        out += struct.pack("<IIIBxH16x", rows, cols, gs, enc, lanes)
    want = list(_group_lens(desc))
    for i, (scale, payload, count) in enumerate(groups):
        if i >= len(want):
            raise Refused(f"only {len(desc)} of {len(desc)} streams were written")
        s, expected = want[i]
        if count != expected or len(payload) != spm_bytes_for(desc[s][3], count):
            raise Refused(f"group expects {expected} weights, got {count}")
        out += struct.pack("<f", scale) + bytes(payload)
    if len(groups) < len(want):
        s = want[len(groups)][0]
        raise Refused(f"only {s} of {len(desc)} streams were written")
    return bytes(out)
