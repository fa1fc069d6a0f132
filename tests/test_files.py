"""GGUF and .spm readers and the .spm writer (host code of libemuhip; no GPU).

The reference's own cases come first, each citing its test; then the library
and the oracle restatement (oracle/files.py) are compared on random
well-formed files, every truncation of them and random corruptions: the same
refusal text, or the same parsed content, byte for byte.
"""
import struct
from pathlib import Path

import numpy as np
import pytest

from emufpga_amd import gguf, spm
from oracle import files as ofiles
from tests import ggufw

GOLDEN = (Path(__file__).resolve().parent / "golden" / "tiny.spm").read_bytes()


def header(tensors, metadata):  # spm-gguf/tests/safety.rs:8-14
    return b"GGUF" + struct.pack("<IQQ", 3, tensors, metadata)


def gguf_error(path) -> str:
    with pytest.raises(gguf.GgufError) as e:
        gguf.read(path)
    return str(e.value)


def oracle_error(data: bytes) -> str:
    with pytest.raises(ofiles.Refused) as e:
        ofiles.gguf_read(data)
    return str(e.value)


# ---------------------------------------------------------------- GGUF ----

def test_rejects_bad_magic(tmp_path):  # safety.rs:16-21
    p = tmp_path / "magic"
    p.write_bytes(b"NOPE")
    assert "magic" in gguf_error(p)
    assert "magic" in oracle_error(b"NOPE")


def test_rejects_unbounded_counts(tmp_path):  # safety.rs:22-27
    data = header(0, ofiles.MAX_METADATA + 1)
    p = tmp_path / "count"
    p.write_bytes(data)
    assert "metadata count" in gguf_error(p)
    assert "metadata count" in oracle_error(data)


def test_rejects_unbounded_strings_before_allocation(tmp_path):  # safety.rs:28-35
    data = header(0, 1) + struct.pack("<Q", ofiles.MAX_STRING + 1)
    p = tmp_path / "string"
    p.write_bytes(data)
    assert "string length" in gguf_error(p)
    assert "string length" in oracle_error(data)


def one_tensor_file(offset: int) -> bytes:  # safety.rs:39-46, 53-60
    v = header(1, 0) + struct.pack("<Q", 1) + b"x" + struct.pack("<IQIQ", 1, 32, 0, offset)
    return v + b"\0" * (64 - len(v))


def test_rejects_tensor_ranges_beyond_the_file(tmp_path):  # safety.rs:36-49
    data = one_tensor_file(4096)
    p = tmp_path / "range"
    p.write_bytes(data)
    assert "beyond file" in gguf_error(p)
    assert "beyond file" in oracle_error(data)


def test_reads_a_tiny_aligned_fixture(tmp_path):  # safety.rs:50-72
    data = one_tensor_file(0) + b"\x01" * (32 * 4)
    p = tmp_path / "tiny"
    p.write_bytes(data)
    c = gguf.read(p)
    assert c.tensors[0].len == 128 and c.tensors[0].offset == 64
    assert gguf.read_tensor_range(p, c.tensors[0], 3, 4, 4) == b"\x01" * 4
    for rel, n, cap in ((127, 2, 2), (0, 5, 4)):
        with pytest.raises(gguf.GgufError):
            gguf.read_tensor_range(p, c.tensors[0], rel, n, cap)
    o = ofiles.gguf_read(data)
    assert o["tensors"][0][3:] == (64, 128)
    assert ofiles.gguf_read_range(data, o["tensors"][0], 3, 4, 4) == b"\x01" * 4
    with pytest.raises(ofiles.Refused):
        ofiles.gguf_read_range(data, o["tensors"][0], 127, 2, 2)
    with pytest.raises(ofiles.Refused):
        ofiles.gguf_read_range(data, o["tensors"][0], 0, 5, 4)


def test_range_errors_name_the_tensor(tmp_path):  # tensor.rs:42-55
    data = one_tensor_file(0) + b"\x01" * 128
    p = tmp_path / "t"
    p.write_bytes(data)
    t = gguf.read(p).tensors[0]
    with pytest.raises(gguf.GgufError, match="tensor x request is 5 bytes, exceeding limit 4"):
        gguf.read_tensor_range(p, t, 0, 5, 4)
    with pytest.raises(gguf.GgufError, match="requested range exceeds tensor x"):
        gguf.read_tensor_range(p, t, 127, 2, 2)
    assert gguf.read_tensor_bytes(p, t, 128) == b"\x01" * 128


def rich_metadata():
    return [("general.architecture", ggufw.STR, "qwen3"), ("u8", ggufw.U8, 255), ("i8", ggufw.I8, -128),
            ("u16", ggufw.U16, 65535), ("i16", ggufw.I16, -32768), ("u32", ggufw.U32, 4294967295),
            ("i32", ggufw.I32, -2147483648), ("f32", ggufw.F32, 1.5e6), ("bool", ggufw.BOOL, 1),
            ("u64", ggufw.U64, 2 ** 64 - 1), ("i64", ggufw.I64, -2 ** 63), ("f64", ggufw.F64, 1e-6),
            ("arr", ggufw.ARR, (ggufw.STR, ["a", "bc"])), ("nested", ggufw.ARR, (ggufw.ARR, [(ggufw.U8, [1, 2])])),
            ("utf8 ключ", ggufw.STR, "значение ✓")]


def test_metadata_rendering_and_numbers(tmp_path):
    data = ggufw.gguf_bytes(rich_metadata(), [("w", (256, 2), 14, bytes(420))])
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    with gguf.GgufFile(p) as f:
        m = f.content.metadata
        assert m["u8"] == "255" and m["i8"] == "-128" and m["i64"] == str(-2 ** 63)
        assert m["u64"] == str(2 ** 64 - 1) and m["bool"] == "1"
        assert m["f32"] == "<6>" and m["f64"] == "<12>" and m["arr"] == "<9>" and m["nested"] == "<9>"
        assert m["utf8 ключ"] == "значение ✓"
        assert f.number("f32") == np.float32(1.5e6) and f.number("f64") == 1e-6 and f.number("u32") == 4294967295
        with pytest.raises(KeyError):
            f.number("arr")
        assert f.content.metadata_count == len(rich_metadata())
    assert ofiles.gguf_read(data)["metadata"] == m


@pytest.mark.parametrize("align_value,expect", [((ggufw.U32, 64), 64), ((ggufw.STR, "+128"), 128),
                                                ((ggufw.F32, 64.0), 32), ((ggufw.STR, "x"), 32),
                                                ((ggufw.U32, 48), "invalid alignment"),
                                                ((ggufw.U32, 0), "invalid alignment")])
def test_general_alignment(tmp_path, align_value, expect):  # parse.rs:163-172
    ty, v = align_value
    a = expect if isinstance(expect, int) else 32
    data = ggufw.gguf_bytes([("general.alignment", ty, v)], [("a", (32,), 0, bytes(128)), ("b", (64,), 8, bytes(68))],
                            align=a)
    p = tmp_path / "a.gguf"
    p.write_bytes(data)
    if isinstance(expect, str):
        assert gguf_error(p) == expect == oracle_error(data)
        return
    c = gguf.read(p)
    assert c.tensor_data_offset % expect == 0
    assert [t.offset % expect for t in c.tensors] == [0, 0]


@pytest.mark.parametrize("mutate,message", [
    (lambda t: t + [("a", (32,), 0, bytes(128))], "duplicate tensor name a"),
    (lambda t: [("z", (32, 0), 0, b"")], "tensor z has a zero dimension"),
    (lambda t: [("q", (32,), 4, bytes(64))], "unsupported GGML dtype 4"),
    (lambda t: [("k", (100,), 14, bytes(210))], "tensor k does not fill dtype blocks"),
    (lambda t: [("d", (1,) * 9, 0, bytes(4))], "invalid dimension count 9"),
])
def test_directory_refusals(tmp_path, mutate, message):  # parse.rs:65-140
    data = ggufw.gguf_bytes([], mutate([("a", (32,), 0, bytes(128))]))
    p = tmp_path / "d.gguf"
    p.write_bytes(data)
    assert gguf_error(p) == message == oracle_error(data)


def test_overlap_unaligned_and_metadata_refusals(tmp_path):
    base = ggufw.gguf_bytes([], [("a", (32,), 0, bytes(128)), ("b", (32,), 0, bytes(128))])
    # b's entry after its name: n_dims u32, dims u64, dtype u32, then the offset u64
    i = base.index(b"\x01\x00\x00\x00\x00\x00\x00\x00b") + 9 + 16
    cases = {
        "overlapping tensor ranges": base[:i] + struct.pack("<Q", 32) + base[i + 8:],
        "unaligned tensor b": base[:i] + struct.pack("<Q", 132) + base[i + 8:],
        "duplicate metadata key": ggufw.gguf_bytes([("k", ggufw.U8, 1), ("k", ggufw.U8, 2)], []),
        "invalid boolean metadata value": ggufw.gguf_bytes([("b", ggufw.BOOL, 2)], []),
        "unknown metadata type 13": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k"
        + struct.pack("<I", 13),
        "invalid UTF-8 string": ggufw.gguf_bytes([(b"\xc0\x80", ggufw.U8, 1)], []),
        "metadata nesting exceeds limit": ggufw.gguf_bytes(
            [("n", ggufw.ARR, (ggufw.ARR, [(ggufw.ARR, [(ggufw.ARR, [(ggufw.ARR, [(ggufw.ARR, [(ggufw.U8, [1])])])])])]))], []),
        "unsupported GGUF version 2": b"GGUF" + struct.pack("<IQQ", 2, 0, 0),
        "tensor count exceeds limit": header(ofiles.MAX_TENSORS + 1, 0),
        "unexpected end of GGUF": b"GGUF\x03\x00",
    }
    for message, data in cases.items():
        p = tmp_path / "c.gguf"
        p.write_bytes(data)
        assert gguf_error(p) == message == oracle_error(data), message


def random_gguf(rng) -> bytes:
    meta = [(f"k{i}", int(t), v) for i, (t, v) in enumerate(
        [(ggufw.U32, int(rng.integers(0, 2 ** 32))), (ggufw.STR, "v" * int(rng.integers(0, 9))),
         (ggufw.I16, int(rng.integers(-2 ** 15, 2 ** 15))), (ggufw.F32, float(rng.normal())),
         (ggufw.ARR, (ggufw.U16, [int(x) for x in rng.integers(0, 2 ** 16, int(rng.integers(0, 5)))])),
         (ggufw.BOOL, int(rng.integers(0, 2)))][:int(rng.integers(0, 7))])]
    dts = [(0, 1, 4), (1, 1, 2), (8, 32, 34), (14, 256, 210), (13, 256, 176), (10, 256, 84)]
    tensors = []
    for i in range(int(rng.integers(0, 5))):
        dt, be, bb = dts[int(rng.integers(0, len(dts)))]
        n = be * int(rng.integers(1, 4))
        dims = (n,) if rng.integers(0, 2) else (be, n // be)
        tensors.append((f"blk.{i}.w", dims, dt, rng.integers(0, 256, n // be * bb, dtype=np.uint8).tobytes()))
    return ggufw.gguf_bytes(meta, tensors)


def compare_gguf(tmp_path, data: bytes):
    p = tmp_path / "r.gguf"
    p.write_bytes(data)
    try:
        want = ofiles.gguf_read(data)
    except ofiles.Refused as e:
        assert gguf_error(p) == str(e)
        return False
    c = gguf.read(p)
    got = {"version": c.version, "metadata_count": c.metadata_count, "tensor_data_offset": c.tensor_data_offset,
           "metadata": c.metadata, "tensors": [(t.name, t.dims, t.dtype, t.offset, t.len) for t in c.tensors]}
    assert got == want
    return True


def test_library_agrees_with_the_oracle_on_random_files(tmp_path):
    rng = np.random.default_rng(2024)
    ok = 0
    for _ in range(40):
        data = random_gguf(rng)
        assert compare_gguf(tmp_path, data)
        for cut in sorted(set(rng.integers(0, len(data), 12).tolist())):
            ok += compare_gguf(tmp_path, data[:cut])
        for _ in range(12):
            b = bytearray(data)
            b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
            ok += compare_gguf(tmp_path, bytes(b))
    assert ok > 50  # corruptions inside tensor bodies still parse


# ----------------------------------------------------------------- .spm ----

def ternary(ws) -> bytes:  # docs/spm-format.md "Ternary weight encoding": LSB pair first
    code = {1: 0b01, 0: 0b00, -1: 0b11}
    out = bytearray((len(ws) + 3) // 4)
    for k, w in enumerate(ws):
        out[k // 4] |= code[w] << (2 * (k % 4))
    return bytes(out)


FIXTURE = spm.OpDescriptor(3, 2, 4, spm.Encoding.TERNARY2_F32_I32, 1)


def test_the_writer_reproduces_the_fixture_byte_for_byte():  # golden.rs:33-47
    w = spm.SpmWriter([FIXTURE])
    w.write_raw_group(1.0, ternary([1, 0, -1, 1]), 4)
    w.write_raw_group(0.5, ternary([-1, 0]), 2)
    assert w.finish() == GOLDEN
    assert ofiles.spm_write([tuple(FIXTURE.__dict__.values())],
                           [(1.0, ternary([1, 0, -1, 1]), 4), (0.5, ternary([-1, 0]), 2)]) == GOLDEN


def test_the_fixture_parses_back_to_the_values_that_built_it():  # golden.rs:49-68
    r = spm.SpmReader(GOLDEN)
    assert r.descriptors == [FIXTURE]
    assert [(g.scale, g.count, g.packed) for g in r] == [(1.0, 4, ternary([1, 0, -1, 1])), (0.5, 2, ternary([-1, 0]))]
    _, desc, groups, err = ofiles.spm_read(GOLDEN)
    assert err is None and desc == [(3, 2, 4, 1, 1)]
    assert [(g[1], g[2], g[3]) for g in groups] == [(1.0, 4, b"\x71"), (0.5, 2, b"\x03")]


def test_the_fixture_matches_the_documented_offsets():  # golden.rs:70-87
    assert GOLDEN[:8] == bytes([0x89, ord("S"), ord("P"), ord("M"), 0x0D, 0x0A, 0x1A, 0x0A])
    assert GOLDEN[16:20] == struct.pack("<I", 1) and GOLDEN[32:36] == struct.pack("<I", 3)
    assert GOLDEN[36:40] == struct.pack("<I", 2) and GOLDEN[40:44] == struct.pack("<I", 4) and GOLDEN[44] == 1
    assert GOLDEN[64:68] == struct.pack("<f", 1.0) and GOLDEN[68] == 0b01_11_00_01
    assert GOLDEN[69:73] == struct.pack("<f", 0.5) and GOLDEN[73] == 0b00_11 and len(GOLDEN) == 74


def test_finishing_with_unwritten_streams_fails():  # errors.rs:22-35
    w = spm.SpmWriter([FIXTURE])
    w.write_raw_group(1.0, ternary([1] * 4), 4)
    with pytest.raises(spm.Incomplete, match="only 0 of 1 streams were written"):
        w.finish()


def test_a_group_of_the_wrong_length_is_refused():  # errors.rs:37-47
    with pytest.raises(spm.GroupLen, match="group expects 4 weights, got 3"):
        spm.SpmWriter([FIXTURE]).write_raw_group(1.0, ternary([1] * 3), 3)


def test_writing_past_the_last_declared_stream_is_refused():  # errors.rs:49-61
    w = spm.SpmWriter([FIXTURE])
    w.write_raw_group(1.0, ternary([1] * 4), 4)
    w.write_raw_group(1.0, ternary([1] * 2), 2)
    with pytest.raises(spm.Incomplete, match="only 1 of 1 streams were written"):
        w.write_raw_group(1.0, ternary([1] * 4), 4)


def test_a_truncated_payload_is_detected_rather_than_read_past():  # errors.rs:63-79
    w = spm.SpmWriter([FIXTURE])
    w.write_raw_group(1.0, ternary([1] * 4), 4)
    w.write_raw_group(0.5, ternary([1] * 2), 2)
    data = w.finish()[:-1]
    r = spm.SpmReader(data)
    assert r.next_group() is not None
    with pytest.raises(spm.PayloadTruncated, match="payload truncated: group needs 5 bytes, 4 remain"):
        r.next_group()
    assert ofiles.spm_read(data)[3] == "payload truncated: group needs 5 bytes, 4 remain"


def test_header_failures_propagate_unchanged():  # errors.rs:81-96
    try:
        data = bytearray(spm.SpmWriter([FIXTURE]).finish())
    except spm.Incomplete:  # groups still owed: the reference falls back to 32 zero bytes
        data = bytearray(32)
    data[0] = 0
    with pytest.raises(spm.HeaderError, match="bad magic"):
        spm.SpmReader(bytes(data))
    data = bytearray(GOLDEN)
    data[0] = 0
    with pytest.raises(spm.HeaderError, match="bad magic: not a .spm file, or corrupted in transit"):
        spm.SpmReader(bytes(data))


def f32s(vals) -> bytes:
    return np.asarray(vals, np.float32).tobytes()


def test_an_f32_stream_roundtrips_bit_for_bit():  # encodings.rs:31-51
    vals = [1.5, -0.25, np.float32(np.pi), 0.0]
    w = spm.SpmWriter([spm.OpDescriptor(2, 2, 4, spm.Encoding.F32)])
    w.write_raw_group(1.0, f32s(vals), 4)
    r = spm.SpmReader(w.finish())
    g = r.next_group()
    assert g.count == 4 and len(g.packed) == 16 and g.packed == f32s(vals)
    assert r.next_group() is None


def test_ternary_and_f32_streams_coexist_in_one_file():  # encodings.rs:53-83
    w = spm.SpmWriter([spm.OpDescriptor(2, 2, 4, spm.Encoding.TERNARY2_F32_I32),
                       spm.OpDescriptor(2, 2, 4, spm.Encoding.F32)])
    w.write_raw_group(2.0, ternary([1, 0, -1, 1]), 4)
    dense = [10.0, -20.0, 30.5, -40.25]
    w.write_raw_group(1.0, f32s(dense), 4)
    data = w.finish()
    assert len(data) == 32 + 64 + 5 + 20
    r = spm.SpmReader(data)
    a, b = r.next_group(), r.next_group()
    assert (a.stream, len(a.packed), a.packed[0]) == (0, 1, 0b01_11_00_01)
    assert (b.stream, len(b.packed)) == (1, 16) and np.frombuffer(b.packed, np.float32).tolist() == dense


@pytest.mark.parametrize("enc,want", [(spm.Encoding.TERNARY2_F32_I32, [(4, 1), (2, 1)]),
                                      (spm.Encoding.F32, [(4, 16), (2, 8)])])
def test_a_group_size_that_does_not_divide(enc, want):  # encodings.rs:85-114
    w = spm.SpmWriter([spm.OpDescriptor(3, 2, 4, enc)])
    for n in (4, 2):
        w.write_raw_group(1.0, ternary([1] * n) if enc == spm.Encoding.TERNARY2_F32_I32 else f32s(range(n)), n)
    assert [(g.count, len(g.packed)) for g in spm.SpmReader(w.finish())] == want


def test_a_payload_of_the_wrong_size_for_its_encoding_is_refused():  # encodings.rs:116-125
    with pytest.raises(spm.GroupLen):
        spm.SpmWriter([spm.OpDescriptor(2, 2, 4, spm.Encoding.F32)]).write_raw_group(1.0, b"\0", 4)


def test_bytes_for_every_profile():  # spm-layout/src/model.rs:80-91
    for enc in spm.Encoding:
        for n in (0, 1, 4, 31, 32, 255, 256, 257, 1000):
            assert spm.bytes_for(enc, n) == ofiles.spm_bytes_for(int(enc), n)
    with pytest.raises(spm.LayoutError):
        spm.bytes_for(7, 1)


@pytest.mark.parametrize("patch,cls,message", [
    ((8, struct.pack("<H", 2)), spm.HeaderError, "unsupported .spm major version 2: this build reads up to 1"),
    ((12, b"\x01"), spm.HeaderError, "unknown endianness discriminant 1"),
    ((40, struct.pack("<I", 0)), spm.LayoutError, "group_size must be at least 1"),
    ((44, b"\x07"), spm.LayoutError, "unknown .spm encoding profile 7"),
    ((16, struct.pack("<I", 3)), spm.LayoutError, "descriptor truncated: 10 bytes, need 32"),
])
def test_header_and_descriptor_refusals(patch, cls, message):
    at, b = patch
    data = GOLDEN[:at] + b + GOLDEN[at + len(b):]
    with pytest.raises(cls) as e:
        spm.SpmReader(data)
    assert str(e.value) == message
    with pytest.raises(ofiles.Refused) as o:
        ofiles.spm_read(data)
    assert str(o.value) == message
    with pytest.raises(spm.HeaderError, match="header truncated: 31 bytes available, need 32"):
        spm.SpmReader(GOLDEN[:31])


def random_spm(rng):
    desc = []
    for _ in range(int(rng.integers(1, 5))):
        enc = int(rng.integers(1, 7))
        unit = {4: 256, 5: 256, 6: 32}.get(enc, 1)
        rows, cols = int(rng.integers(0, 4)), unit * int(rng.integers(1, 3))
        desc.append((rows, cols, unit * int(rng.integers(1, 3)) if unit > 1 else int(rng.integers(1, 9)), enc,
                     int(rng.integers(0, 3))))
    groups = []
    for s, count in ofiles._group_lens(desc):
        n = ofiles.spm_bytes_for(desc[s][3], count)
        groups.append((float(np.float32(rng.normal())), rng.integers(0, 256, n, dtype=np.uint8).tobytes(), count))
    return desc, groups


def test_writer_and_reader_round_trip_and_agree_with_the_oracle():  # roundtrip.rs
    rng = np.random.default_rng(7)
    for _ in range(30):
        desc, groups = random_spm(rng)
        w = spm.SpmWriter([spm.OpDescriptor(*d) for d in desc])
        for scale, payload, count in groups:
            w.write_raw_group(scale, payload, count)
        data = w.finish()
        assert data == ofiles.spm_write(desc, groups)
        r = spm.SpmReader(data)
        got = [(g.stream, g.scale, g.count, g.packed) for g in r]
        _, _, want, err = ofiles.spm_read(data)
        assert err is None and got == want
        assert [(g[1], g[3], g[2]) for g in want] == [(np.float32(s), p, c) for s, p, c in groups]
        # every truncation: same refusal or same groups up to the same point
        for cut in range(0, len(data), max(1, len(data) // 40)):
            part = data[:cut]
            try:
                _, _, want, err = ofiles.spm_read(part)
            except ofiles.Refused as e:
                with pytest.raises(spm.FileError) as got_e:
                    spm.SpmReader(part)
                assert str(got_e.value) == str(e)
                continue
            r = spm.SpmReader(part)
            got = []
            try:
                for g in r:
                    got.append((g.stream, g.scale, g.count, g.packed))
            except spm.PayloadTruncated as e:
                assert str(e) == err
            else:
                assert err is None
            assert got == want
