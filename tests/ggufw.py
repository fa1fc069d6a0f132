"""GGUF files for tests: in-memory files from the package's writer, and a
model's weights split into llama.cpp-named tensors."""
from __future__ import annotations

import io

from emufpga_amd.gguf import (MT_ARR as ARR, MT_BOOL as BOOL, MT_F32 as F32, MT_F64 as F64,  # noqa: F401
                              MT_I8 as I8, MT_I16 as I16, MT_I32 as I32, MT_I64 as I64, MT_STR as STR,
                              MT_U8 as U8, MT_U16 as U16, MT_U32 as U32, MT_U64 as U64, write)


def gguf_bytes(metadata, tensors, align: int = 32) -> bytes:
    """metadata: [(key, type, value)]; tensors: [(name, dims, dtype, data bytes)]."""
    buf = io.BytesIO()
    write(buf, metadata, tensors, align)
    return buf.getvalue()


def model_file_tensors(cfg, w: dict):
    """A model's weights (Model.host_weights()) as GGUF (metadata, tensors)."""
    from emufpga_amd.serve import gguf_tensors
    return gguf_tensors(cfg, w)
