"""GGUF block formats on the device: the spm-gguf decoding API.

Mirrors components/cli/crates/spm-gguf: ``layout`` (parse.rs:10-29) and
``decode_q6_k`` / ``decode_q5_k`` / ``decode_q8_0`` (tensor.rs:103,144,193),
plus ``decode_q2_k``, which the reference lacks.  Each decoder takes the raw
block bytes, decodes them with the gfx950 dequant kernel and returns the f32
values in the reference's element order.  A partial block raises ``Short``,
as the reference returns an error.
"""
from __future__ import annotations

import ctypes as C

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
