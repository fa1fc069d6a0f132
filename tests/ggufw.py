"""A GGUF v3 writer for tests: metadata of every scalar type, strings and
arrays, and tensors placed at aligned offsets (the layout spm-gguf reads,
components/cli/crates/spm-gguf/src/parse.rs:157-182)."""
from __future__ import annotations

import struct

# metadata value types (spm-gguf/src/wire.rs:55-90)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "B", U64: "Q", I64: "q", F64: "d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(ty: int, v) -> bytes:
    if ty == STR:
        return _str(v)
    if ty == ARR:
        inner, items = v
        return struct.pack("<IQ", inner, len(items)) + b"".join(_value(inner, x) for x in items)
    return struct.pack("<" + _FMT[ty], v)


def gguf_bytes(metadata, tensors, align: int = 32) -> bytes:
    """metadata: [(key, type, value)]; tensors: [(name, dims, dtype, data bytes)].
    Tensor data follows the directory at the next `align` boundary, each
    tensor at an `align`-aligned offset."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    for key, ty, v in metadata:
        out += _str(key) + struct.pack("<I", ty) + _value(ty, v)
    offs, at = [], 0
    for _, _, _, data in tensors:
        offs.append(at)
        at = (at + len(data) + align - 1) // align * align
    for (name, dims, dtype, _), off in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", dtype, off)
    base = (len(out) + align - 1) // align * align
    out += b"\0" * (base - len(out))
    for (_, _, _, data), off in zip(tensors, offs):
        out += b"\0" * (base + off - len(out)) + bytes(data)
    return bytes(out)


def _row_bytes(enc: int, cols: int) -> int:
    from emufpga_amd.gguf import row_bytes
    return row_bytes(enc, cols)


def model_file_tensors(cfg, w: dict, arch_metadata: bool = True):
    """A model's weights (Model.host_weights()) as GGUF (metadata, tensors)
    under llama.cpp's names, shapes in GGML order (row length first)."""
    from emufpga_amd import _lib
    H, QW, KW = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    enc, moe = cfg.encoding, cfg.style == _lib.EMU_STYLE_GRANITE
    rb_h, rb_q = _row_bytes(enc, H), _row_bytes(enc, QW)
    t = [("token_embd.weight", (H, cfg.vocab), enc, w["embed"].tobytes())]
    if not cfg.tied:
        t.append(("output.weight", (H, cfg.vocab), enc, w["output"].tobytes()))
    t.append(("output_norm.weight", (H,), 0, w["out_norm"].tobytes()))
    layers = w["layers"]
    if moe:
        rb_he, rb_fe = _row_bytes(cfg.expert_encoding, H), _row_bytes(cfg.expert_encoding, cfg.expert_ff)
        off_o = (QW + 2 * KW) * rb_h
        off_r = (off_o + H * rb_q + 15) // 16 * 16
        ge = cfg.n_experts * cfg.expert_ff * rb_he
        de = cfg.n_experts * H * rb_fe
        lb = (off_r + 4 * cfg.n_experts * H + 2 * ge + de + 15) // 16 * 16
    else:
        rb_f = _row_bytes(enc, cfg.ffn)
        lb = (QW + 2 * KW) * rb_h + H * rb_q + 2 * cfg.ffn * rb_h + H * rb_f
    assert layers.size == lb * cfg.layers
    for l in range(cfg.layers):
        blob = layers[l * lb:(l + 1) * lb]
        at = 0

        def take(name, dims, dtype, n):
            nonlocal at
            t.append((f"blk.{l}.{name}.weight", dims, dtype, blob[at:at + n].tobytes()))
            at += n

        t.append((f"blk.{l}.attn_norm.weight", (H,), 0, w["attn_norm"][l * H:(l + 1) * H].tobytes()))
        t.append((f"blk.{l}.ffn_norm.weight", (H,), 0, w["ffn_norm"][l * H:(l + 1) * H].tobytes()))
        if cfg.qk_norm:
            d = cfg.head_dim
            t.append((f"blk.{l}.attn_q_norm.weight", (d,), 0, w["q_norm"][l * d:(l + 1) * d].tobytes()))
            t.append((f"blk.{l}.attn_k_norm.weight", (d,), 0, w["k_norm"][l * d:(l + 1) * d].tobytes()))
        take("attn_q", (H, QW), enc, QW * rb_h)
        take("attn_k", (H, KW), enc, KW * rb_h)
        take("attn_v", (H, KW), enc, KW * rb_h)
        take("attn_output", (QW, H), enc, H * rb_q)
        if moe:
            at = off_r
            take("ffn_gate_inp", (H, cfg.n_experts), 0, 4 * cfg.n_experts * H)
            take("ffn_gate_exps", (H, cfg.expert_ff, cfg.n_experts), cfg.expert_encoding, ge)
            take("ffn_up_exps", (H, cfg.expert_ff, cfg.n_experts), cfg.expert_encoding, ge)
            take("ffn_down_exps", (cfg.expert_ff, H, cfg.n_experts), cfg.expert_encoding, de)
        else:
            take("ffn_gate", (H, cfg.ffn), enc, cfg.ffn * rb_h)
            take("ffn_up", (H, cfg.ffn), enc, cfg.ffn * rb_h)
            take("ffn_down", (cfg.ffn, H), enc, H * _row_bytes(enc, cfg.ffn))
    arch = {_lib.EMU_STYLE_QWEN3: "qwen3", _lib.EMU_STYLE_SMOL: "llama", _lib.EMU_STYLE_GRANITE: "granitemoe"}[cfg.style]
    meta = [("general.architecture", STR, arch), ("general.alignment", U32, 64),
            (f"{arch}.embedding_length", U32, H), (f"{arch}.block_count", U32, cfg.layers),
            (f"{arch}.attention.head_count", U32, cfg.heads), (f"{arch}.attention.head_count_kv", U32, cfg.kv_heads),
            (f"{arch}.attention.key_length", U32, cfg.head_dim), (f"{arch}.rope.freq_base", F32, cfg.rope_theta),
            (f"{arch}.attention.layer_norm_rms_epsilon", F32, cfg.eps)]
    if moe:
        meta += [(f"{arch}.expert_count", U32, cfg.n_experts), (f"{arch}.expert_used_count", U32, cfg.experts_used),
                 (f"{arch}.expert_feed_forward_length", U32, cfg.expert_ff),
                 (f"{arch}.embedding_scale", F32, cfg.embed_scale), (f"{arch}.residual_scale", F32, cfg.residual_scale),
                 (f"{arch}.logit_scale", F32, cfg.logit_div), (f"{arch}.attention.scale", F32, cfg.score_mul)]
    else:
        meta.append((f"{arch}.feed_forward_length", U32, cfg.ffn))
    return (meta if arch_metadata else []), t
