"""GGUF block formats on the device: the spm-gguf decoding API.

Mirrors components/cli/crates/spm-gguf: ``layout`` (parse.rs:10-29) and
``decode_q6_k`` / ``decode_q5_k`` / ``decode_q8_0`` (tensor.rs:103,144,193),
plus ``decode_q2_k``, which the reference lacks.  Each decoder takes the raw
block bytes, decodes them with the gfx950 dequant kernel and returns the f32
values in the reference's element order.  A partial block raises ``Short``,
as the reference returns an error.

The file side mirrors spm-gguf's ``read`` / ``read_tensor_range`` /
``read_tensor_bytes`` over the library's bounded C++ parser; ``GgufFile``
keeps a file open for many range reads and for uploads into device memory.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import Q2_K, Q5_K, Q6_K, Q8_0, F16, F32, check
from .device import Context

# spm-gguf/src/parse.rs:10-29 (subset on the path): dtype -> (elements, bytes)
LAYOUT = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q2_K: (256, 84), Q5_K: (256, 176), Q6_K: (256, 210)}


def layout(dtype: int) -> tuple[int, int]:
    e, b = C.c_uint32(), C.c_uint32()
    check(_lib.load().emu_block_layout(dtype, C.byref(e), C.byref(b)), "emu_block_layout")
    return e.value, b.value


def row_bytes(dtype: int, cols: int) -> int:
    e, b = LAYOUT[dtype]
    if cols % e:
        raise ValueError(f"{cols} columns is not a whole number of {e}-element blocks")
    return cols // e * b


_default_ctx: Context | None = None


def default_context() -> Context:
    global _default_ctx
    if _default_ctx is None:
        _default_ctx = Context(0)
    return _default_ctx


def decode(dtype: int, data: bytes | np.ndarray, ctx: Context | None = None) -> np.ndarray:
    ctx = ctx or default_context()
    raw = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data.view(np.uint8)
    elems, bb = LAYOUT[dtype]
    nblk = raw.size // bb
    src = ctx.upload(raw if raw.size else np.zeros(1, np.uint8))
    out = ctx.alloc(max(nblk * elems * 4, 4))
    ctx.check(ctx.lib.emu_dequant(ctx.h, dtype, src.ptr, raw.size, out.ptr), "emu_dequant")
    return out.read(np.float32, nblk * elems)


def decode_q6_k(data, ctx: Context | None = None) -> np.ndarray:
    return decode(Q6_K, data, ctx)


def decode_q5_k(data, ctx: Context | None = None) -> np.ndarray:
    return decode(Q5_K, data, ctx)


def decode_q8_0(data, ctx: Context | None = None) -> np.ndarray:
    return decode(Q8_0, data, ctx)


def decode_q2_k(data, ctx: Context | None = None) -> np.ndarray:
    return decode(Q2_K, data, ctx)


# ---------------------------------------------------------------- files ----
# The bounded GGUF reader of spm-gguf (parse.rs:157-182 read, tensor.rs:21-67
# read_tensor_bytes / read_tensor_range), on the library's C++ parser.

class GgufError(RuntimeError):
    """A refused file or range; the message is the reference's Err(String)."""


@dataclass(frozen=True)
class TensorInfo:  # spm-gguf/src/model.rs:3-10
    name: str
    dims: tuple
    dtype: int
    offset: int
    len: int


@dataclass
class Content:  # spm-gguf/src/model.rs:12-19
    version: int
    metadata_count: int
    tensor_data_offset: int
    metadata: dict
    tensors: list = field(default_factory=list)


class GgufFile:
    """An open GGUF file: the parsed Content plus range reads and uploads."""

    def __init__(self, path):
        self.lib = _lib.load()
        self.path = str(path)
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        st = self.lib.emu_gguf_open(self.path.encode(), C.byref(h), err, len(err))
        if st != _lib.EMU_OK:
            raise GgufError(err.value.decode(errors="replace"))
        self.h = h
        self.content = self._content()

    def _content(self) -> Content:
        ver, mc, base, nt = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        self.lib.emu_gguf_summary(self.h, C.byref(ver), C.byref(mc), C.byref(base), C.byref(nt))
        meta = {}
        k, v, kn, vn = C.c_void_p(), C.c_void_p(), C.c_size_t(), C.c_size_t()
        for i in range(mc.value):
            self.lib.emu_gguf_metadata_at(self.h, i, C.byref(k), C.byref(kn), C.byref(v), C.byref(vn))
            meta[C.string_at(k, kn.value).decode()] = C.string_at(v, vn.value).decode()
        tensors = []
        info = _lib.GgufTensorInfo()
        for i in range(nt.value):
            self.lib.emu_gguf_tensor_at(self.h, i, C.byref(info))
            tensors.append(TensorInfo(C.string_at(info.name, info.name_len).decode(), tuple(info.dims[:info.n_dims]),
                                      info.dtype, info.offset, info.len))
        return Content(ver.value, mc.value, base.value, meta, tensors)

    def close(self) -> None:
        if self.h is not None:
            self.lib.emu_gguf_close(self.h)
        self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def _fail(self) -> GgufError:
        return GgufError(self.lib.emu_gguf_error(self.h).decode(errors="replace"))

    def index(self, tensor) -> int:
        name = tensor.name if isinstance(tensor, TensorInfo) else str(tensor)
        i = C.c_uint64()
        if self.lib.emu_gguf_find(self.h, name.encode(), C.byref(i)) != _lib.EMU_OK:
            raise self._fail()
        return i.value

    def tensor(self, name: str) -> TensorInfo:
        return self.content.tensors[self.index(name)]

    def number(self, key: str) -> float:
        """A scalar metadata value as a number (floats included)."""
        v = C.c_double()
        st = self.lib.emu_gguf_metadata_number(self.h, key.encode(), C.byref(v))
        if st != _lib.EMU_OK:
            raise KeyError(key)
        return v.value

    def read_range(self, tensor, relative_offset: int, length: int, max_bytes: int) -> bytes:
        out = np.empty(max(length, 1), np.uint8)
        if self.lib.emu_gguf_read_range(self.h, self.index(tensor), relative_offset, length, max_bytes,
                                        out.ctypes.data_as(C.c_void_p)) != _lib.EMU_OK:
            raise self._fail()
        return out[:length].tobytes()

    def upload(self, ctx: Context, tensor, d_ptr: int, relative_offset: int = 0, length: int | None = None) -> None:
        """Place a tensor range in device memory (pinned double-buffered reads)."""
        i = self.index(tensor)
        n = self.content.tensors[i].len - relative_offset if length is None else length
        st = self.lib.emu_gguf_upload(ctx.h, self.h, i, relative_offset, n, C.c_void_p(d_ptr))
        if st == _lib.EMU_E_HIP:
            ctx.check(st, "emu_gguf_upload")
        if st != _lib.EMU_OK:
            raise self._fail()


def read(path) -> Content:
    """spm_gguf::read: parse and validate without loading tensor bodies."""
    with GgufFile(path) as f:
        return f.content


def read_tensor_range(path, tensor: TensorInfo, relative_offset: int, length: int, max_bytes: int) -> bytes:
    """spm_gguf::read_tensor_range (tensor.rs:35-67)."""
    with GgufFile(path) as f:
        return f.read_range(tensor, relative_offset, length, max_bytes)


def read_tensor_bytes(path, tensor: TensorInfo, max_bytes: int) -> bytes:
    """spm_gguf::read_tensor_bytes (tensor.rs:21-28)."""
    return read_tensor_range(path, tensor, 0, tensor.len, max_bytes)


# metadata value types (spm-gguf/src/wire.rs:55-90)
(MT_U8, MT_I8, MT_U16, MT_I16, MT_U32, MT_I32, MT_F32, MT_BOOL, MT_STR, MT_ARR, MT_U64, MT_I64,
 MT_F64) = range(13)
_MT_FMT = {MT_U8: "B", MT_I8: "b", MT_U16: "H", MT_I16: "h", MT_U32: "I", MT_I32: "i", MT_F32: "f", MT_BOOL: "B",
           MT_U64: "Q", MT_I64: "q", MT_F64: "d"}


def _mt_str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _mt_value(ty: int, v) -> bytes:
    if ty == MT_STR:
        return _mt_str(v)
    if ty == MT_ARR:
        inner, items = v
        return struct.pack("<IQ", inner, len(items)) + b"".join(_mt_value(inner, x) for x in items)
    return struct.pack("<" + _MT_FMT[ty], v)


def write(out, metadata, tensors, align: int = 32) -> int:
    """A GGUF v3 file: metadata [(key, type, value)] and tensors
    [(name, dims in GGML order, dtype, data)], each tensor's data at an
    `align`-aligned offset after the directory (the layout read() parses).
    `out` is a path or a binary file object; returns the bytes written."""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    for key, ty, v in metadata:
        head += _mt_str(key) + struct.pack("<I", ty) + _mt_value(ty, v)
    offs, at = [], 0
    for _, _, _, data in tensors:
        offs.append(at)
        at = (at + memoryview(data).nbytes + align - 1) // align * align
    for (name, dims, dtype, _), off in zip(tensors, offs):
        head += _mt_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", dtype, off)
    base = (len(head) + align - 1) // align * align
    head += b"\0" * (base - len(head))
    own = not hasattr(out, "write")
    f = open(out, "wb") if own else out
    try:
        f.write(head)
        pos = 0
        for (_, _, _, data), off in zip(tensors, offs):
            f.write(b"\0" * (off - pos))
            mv = memoryview(data).cast("B")
            f.write(mv)
            pos = off + mv.nbytes
    finally:
        if own:
            f.close()
    return base + pos
