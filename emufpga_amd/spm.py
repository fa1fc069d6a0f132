""".spm files: the forward-only reader and the writer of
components/format/crates/spm-file (read.rs, write.rs), the descriptor and
encoding profiles of spm-layout (model.rs), on the library's C++ code, plus
device placement of a stream and the Granite expert-layer emission of
spm-granite-moe/src/layout.rs:137-186.

Byte layout (docs/spm-format.md): a 32-byte header, one 32-byte descriptor
per stream, then per stream and per scale group a 4-byte f32 scale followed by
the group's packed weights.  Q6K / Q5K / Q8_0 streams keep GGUF blocks in
source row-major order; F32 streams are column-major.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from . import _lib
from .device import Context


class Encoding(IntEnum):  # spm-layout/src/model.rs:14-58
    TERNARY2_F32_I32 = 1
    F32 = 2
    BF16 = 3
    Q6K = 4
    Q5K = 5
    Q8_0 = 6

    def bytes_for(self, count: int) -> int:
        """Encoding::bytes_for (model.rs:80-91)."""
        return bytes_for(int(self), count)


def bytes_for(encoding: int, count: int) -> int:
    v = C.c_uint64()
    st = _lib.load().emu_spm_bytes_for(encoding, count, C.byref(v))
    if st != _lib.EMU_OK:
        raise LayoutError(f"unknown .spm encoding profile {encoding}")
    return v.value


@dataclass(frozen=True)
class OpDescriptor:  # spm-layout/src/model.rs:113-125
    rows: int
    cols: int
    group_size: int
    encoding: int
    lane_count: int = 1

    def native(self) -> _lib.SpmDescriptor:
        return _lib.SpmDescriptor(self.rows, self.cols, self.group_size, int(self.encoding), self.lane_count)


@dataclass(frozen=True)
class Header:  # spm-header/src/model.rs:37-47
    version_major: int
    version_minor: int
    stream_count: int


@dataclass(frozen=True)
class Group:  # spm-file/src/read.rs:16-25
    stream: int
    scale: float
    count: int
    packed: bytes


class FileError(RuntimeError):
    """spm-file FileError (error.rs:9-41)."""


class HeaderError(FileError):
    """spm-header HeaderError (model.rs:63-89)."""


class LayoutError(FileError):
    """spm-layout LayoutError (model.rs:127-145)."""


class PayloadTruncated(FileError):
    """The payload ended mid-group."""


class GroupLen(FileError):
    """A group offered with the wrong number of weights or bytes."""


class Incomplete(FileError):
    """Fewer groups written than the descriptors call for."""


_HEADER_MESSAGES = ("header truncated", "bad magic", "unsupported .spm major version", "unknown endianness")


class SpmReader:
    """SpmReader (read.rs:33-101): header and directory parsed eagerly; the
    payload only through ``next_group`` (or ``upload_stream``), forward."""

    def __init__(self, data):
        self.lib = _lib.load()
        self._buf = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else data
        self._buf = np.ascontiguousarray(self._buf.view(np.uint8))
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        ptr = self._buf.ctypes.data_as(C.c_void_p) if self._buf.size else None
        st = self.lib.emu_spm_parse(ptr, self._buf.size, C.byref(h), err, len(err))
        if st != _lib.EMU_OK:
            msg = err.value.decode()
            raise (HeaderError if msg.startswith(_HEADER_MESSAGES) else LayoutError)(msg)
        self.h = h
        mj, mn, n = C.c_uint16(), C.c_uint16(), C.c_uint32()
        self.lib.emu_spm_header(h, C.byref(mj), C.byref(mn), C.byref(n))
        self.header = Header(mj.value, mn.value, n.value)
        self.descriptors = []
        d = _lib.SpmDescriptor()
        for i in range(n.value):
            self.lib.emu_spm_descriptor_at(h, i, C.byref(d))
            self.descriptors.append(OpDescriptor(d.rows, d.cols, d.group_size, d.encoding, d.lane_count))

    @classmethod
    def parse(cls, data) -> "SpmReader":
        return cls(data)

    def close(self) -> None:
        if getattr(self, "h", None) is not None:
            self.lib.emu_spm_close(self.h)
        self.h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> tuple[int, int]:
        s, g = C.c_uint32(), C.c_uint64()
        self.lib.emu_spm_position(self.h, C.byref(s), C.byref(g))
        return s.value, g.value

    def next_group(self) -> Group | None:
        has, grp = C.c_int(), _lib.SpmGroup()
        st = self.lib.emu_spm_next_group(self.h, C.byref(has), C.byref(grp))
        if st == _lib.EMU_E_TRUNCATED:
            raise PayloadTruncated(self.lib.emu_spm_error(self.h).decode())
        if st != _lib.EMU_OK:
            raise FileError(self.lib.emu_spm_error(self.h).decode())
        if not has.value:
            return None
        packed = C.string_at(grp.packed, grp.packed_len) if grp.packed_len else b""
        return Group(grp.stream, grp.scale, grp.count, packed)

    def __iter__(self):
        while (g := self.next_group()) is not None:
            yield g

    def upload_stream(self, ctx: Context, d_ptr: int, nbytes: int) -> int:
        """Place the current stream in device memory in the kernels' layout
        (blocks back to back, or a row-major f32 matrix); returns its index."""
        s = C.c_uint32()
        st = self.lib.emu_spm_upload_stream(ctx.h, self.h, C.c_void_p(d_ptr), nbytes, C.byref(s))
        if st == _lib.EMU_E_HIP:
            ctx.check(st, "emu_spm_upload_stream")
        if st == _lib.EMU_E_TRUNCATED:
            raise PayloadTruncated(self.lib.emu_spm_error(self.h).decode())
        if st != _lib.EMU_OK:
            raise FileError(self.lib.emu_spm_error(self.h).decode())
        return s.value


def device_bytes(d: OpDescriptor) -> int:
    """Bytes a stream occupies once placed by ``upload_stream``."""
    n = d.rows * d.cols
    per = {Encoding.Q6K: (256, 210), Encoding.Q5K: (256, 176), Encoding.Q8_0: (32, 34), Encoding.F32: (1, 4)}
    e, b = per[Encoding(d.encoding)]
    return n // e * b


class SpmWriter:
    """SpmWriter (write.rs:15-107): header and directory up front, then groups
    in stream order; ``finish`` refuses a file with groups still owed."""

    def __init__(self, descriptors):
        self.lib = _lib.load()
        arr = (_lib.SpmDescriptor * max(len(descriptors), 1))(*[d.native() for d in descriptors])
        h = C.c_void_p()
        _lib.check(self.lib.emu_spm_writer_create(arr, len(descriptors), C.byref(h)), "emu_spm_writer_create")
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None) is not None:
            self.lib.emu_spm_writer_destroy(self.h)
        self.h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def write_raw_group(self, scale: float, payload: bytes, count: int) -> None:
        buf = np.frombuffer(bytes(payload), np.uint8)
        st = self.lib.emu_spm_write_raw_group(self.h, scale, buf.ctypes.data_as(C.c_void_p) if buf.size else None,
                                              buf.size, count)
        if st == _lib.EMU_E_SHAPE:
            raise GroupLen(self.lib.emu_spm_writer_error(self.h).decode())
        if st == _lib.EMU_E_FORMAT:
            raise Incomplete(self.lib.emu_spm_writer_error(self.h).decode())
        _lib.check(st, "emu_spm_write_raw_group")

    def finish(self) -> bytes:
        p, n = C.POINTER(C.c_uint8)(), C.c_size_t()
        st = self.lib.emu_spm_writer_finish(self.h, C.byref(p), C.byref(n))
        if st == _lib.EMU_E_FORMAT:
            raise Incomplete(self.lib.emu_spm_writer_error(self.h).decode())
        _lib.check(st, "emu_spm_writer_finish")
        return C.string_at(p, n.value)


Q6_VALUES, Q6_BYTES = 256, 210


def emit_moe_layer(gguf_file, layer: int, experts, n_experts: int, width: int, ff: int) -> bytes:
    """One MoE layer as a .spm file (spm-granite-moe/src/layout.rs:137-186):
    the f32 router (n_experts x width, one column per group), then for each
    selected expert its up, gate and down Q6_K matrices, one 256-weight block
    per group with an inert 1.0 scale."""
    from .gguf import F32 as _F32

    descs = [OpDescriptor(n_experts, width, n_experts, Encoding.F32)]
    for _ in experts:
        descs += [OpDescriptor(ff, width, Q6_VALUES, Encoding.Q6K), OpDescriptor(ff, width, Q6_VALUES, Encoding.Q6K),
                  OpDescriptor(width, ff, Q6_VALUES, Encoding.Q6K)]
    w = SpmWriter(descs)
    router = gguf_file.tensor(f"blk.{layer}.ffn_gate_inp.weight")
    if router.dtype != _F32:
        raise FileError(f"tensor {router.name} has unsupported dtype {router.dtype}")
    r = np.frombuffer(gguf_file.read_range(router, 0, router.len, router.len), np.float32)
    r = r.reshape(n_experts, width)
    for col in range(width):
        w.write_raw_group(1.0, np.ascontiguousarray(r[:, col]).tobytes(), n_experts)
    for e in experts:
        for name, cols, rows in (("ffn_up_exps", width, ff), ("ffn_gate_exps", width, ff),
                                 ("ffn_down_exps", ff, width)):
            t = gguf_file.tensor(f"blk.{layer}.{name}.weight")
            if t.dtype != _lib.Q6_K or cols % 256:
                raise FileError(f"tensor {t.name} is not row-aligned Q6_K")
            size = rows * (cols // 256) * Q6_BYTES
            data = gguf_file.read_range(t, e * size, size, size)
            for b in range(0, size, Q6_BYTES):
                w.write_raw_group(1.0, data[b:b + Q6_BYTES], Q6_VALUES)
    out = w.finish()
    w.close()
    return out
