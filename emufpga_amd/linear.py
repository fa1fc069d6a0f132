"""Quantized projections: the tensor-engine matvec API on the device.

``streamed`` mirrors spm_linear::streamed (components/tensor/crates/
spm-linear/src/stream.rs:31-55): the result (positions x rows) is W x for
every position, overwriting ``out`` as the reference zero-fills it first.  The
weight source is a device-resident GGUF block matrix instead of a GroupStream;
shape errors map to the reference's LinearError variants (WeightCount,
ActivationLen).  ``project_expert`` mirrors spm-granite-moe
weights::project_expert (weights.rs:41-55) on one expert's slice of an
expert-major 3-D tensor.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import EMU_MV_ACCUMULATE
from .device import Context
from .gguf import row_bytes


class QuantMatrix:
    """A rows x cols GGUF block matrix resident in HBM (bytes uploaded as is)."""

    def __init__(self, ctx: Context, dtype: int, rows: int, cols: int, data):
        self.ctx, self.dtype, self.rows, self.cols = ctx, dtype, rows, cols
        raw = data.view(np.uint8).reshape(-1) if isinstance(data, np.ndarray) else np.frombuffer(bytes(data), np.uint8)
        self.nbytes = int(raw.size)
        self.buf = ctx.upload(raw if raw.size else np.zeros(1, np.uint8))

    @property
    def ptr(self):
        return self.buf.ptr


def streamed(ctx: Context, m: QuantMatrix, batch: tuple[np.ndarray, int], accumulate_into=None) -> np.ndarray:
    """W x for `positions` activation rows; batches of up to 8 per launch."""
    acts, positions = batch
    acts = np.ascontiguousarray(acts, dtype=np.float32).reshape(-1)
    xb = ctx.upload(acts if acts.size else np.zeros(1, np.float32))
    ob = ctx.alloc(max(positions * m.rows * 4, 4))
    flags = 0
    if accumulate_into is not None:
        ob.write(np.ascontiguousarray(accumulate_into, np.float32).reshape(-1))
        flags = EMU_MV_ACCUMULATE
    for p0 in range(0, max(positions, 1), 8):
        n = min(8, positions - p0)
        if n <= 0:
            break
        x_len = max(acts.size - p0 * m.cols, 0)
        ctx.check(ctx.lib.emu_qmatvec(ctx.h, m.dtype, m.ptr, m.nbytes, m.rows, m.cols,
                                      C.c_void_p(xb.addr + p0 * m.cols * 4), x_len, n,
                                      C.c_void_p(ob.addr + p0 * m.rows * 4), flags), "emu_qmatvec")
    return ob.read(np.float32, positions * m.rows)


def project_expert(ctx: Context, dtype: int, experts, rows: int, cols: int, expert: int,
                   inputs: list[np.ndarray]) -> list[np.ndarray]:
    """One expert's rows x cols slice of an expert-major tensor applied to each input."""
    rb = row_bytes(dtype, cols)
    raw = experts.view(np.uint8).reshape(-1) if isinstance(experts, np.ndarray) else np.frombuffer(bytes(experts), np.uint8)
    start = expert * rows * rb
    m = QuantMatrix(ctx, dtype, rows, cols, raw[start:start + rows * rb])
    if not inputs:
        return []
    y = streamed(ctx, m, (np.stack(inputs), len(inputs)))
    return [y[i * rows:(i + 1) * rows] for i in range(len(inputs))]


__all__ = ["QuantMatrix", "streamed", "project_expert"]
