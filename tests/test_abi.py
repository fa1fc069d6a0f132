"""The C-ABI library loads and exports every declared entry point (CPU only)."""
import re
from pathlib import Path

import numpy as np

from emufpga_amd import _lib, gguf

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    names = []
    for hdr in sorted((ROOT / "include").glob("*.h")):
        text = hdr.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(emu_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_the_header():
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_status_strings():
    assert _lib.strerror(_lib.EMU_OK) == "ok"
    assert "whole number of blocks" in _lib.strerror(_lib.EMU_E_SHORT)
    assert _lib.strerror(999) == "unknown status"


def test_block_layout_matches_gguf_table():  # spm-gguf/src/parse.rs:10-29
    for dtype, (e, b) in gguf.LAYOUT.items():
        assert gguf.layout(dtype) == (e, b)
    try:
        gguf.layout(2)  # Q4_0 has a size in the reference table but is not on this path
    except _lib.Unsupported:
        pass
    else:
        raise AssertionError("unsupported dtype accepted")


def test_row_bytes():
    assert gguf.row_bytes(_lib.Q6_K, 4096) == 16 * 210
    assert gguf.row_bytes(_lib.Q8_0, 576) == 18 * 34
    try:
        gguf.row_bytes(_lib.Q6_K, 100)
    except ValueError:
        pass
    else:
        raise AssertionError


def test_null_arguments_are_rejected_without_touching_a_device():
    lib = _lib.load()
    assert lib.emu_ctx_create(0, None) == _lib.EMU_E_ARG
    assert lib.emu_dequant(None, _lib.Q6_K, None, 0, None) == _lib.EMU_E_ARG
    assert lib.emu_qmatvec(None, _lib.Q6_K, None, 0, 1, 256, None, 0, 1, None, 0) == _lib.EMU_E_ARG
    assert np.isscalar(lib.emu_ctx_destroy(None))
