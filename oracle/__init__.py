"""Python binding of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

The oracle restates the reference's Rust CPU arithmetic in C (oracle.c) and is
the checker the HIP path is compared against.  Only tests, the smoke entry
point and the benchmark's CPU-baseline leg use it; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

OR_F32, OR_F16, OR_Q8_0, OR_Q2_K, OR_Q5_K, OR_Q6_K = 0, 1, 8, 10, 13, 14
STYLE_QWEN3, STYLE_SMOL = 0, 1


class DenseCfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("heads", C.c_uint32), ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32),
        ("layers", C.c_uint32), ("context", C.c_uint32), ("rope_theta", C.c_float),
        ("eps", C.c_float), ("style", C.c_int32), ("dtype", C.c_int32), ("kv_f16", C.c_int32),
        ("tied", C.c_int32), ("qk_norm", C.c_int32),
    ]


class MoeDesc(C.Structure):
    _fields_ = [("enc_gate_up", C.c_int32), ("enc_down", C.c_int32), ("gate", C.c_void_p), ("up", C.c_void_p),
                ("down", C.c_void_p), ("down_scale", C.c_void_p), ("n_experts", C.c_uint32),
                ("width", C.c_uint32), ("ff", C.c_uint32), ("k", C.c_uint32), ("act", C.c_int32)]


OR_ACT_SILU, OR_ACT_GELU_TANH = 0, 1


class DenseWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("layers", "embed", "output", "attn_norm", "ffn_norm", "q_norm", "k_norm", "out_norm")]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def load() -> C.CDLL:
    """The oracle library; ORACLE_LIB names another build of oracle.c (the
    planted-mistake tests load mutated copies that way, in a child process)."""
    global _lib
    if _lib is None:
        alt = os.environ.get("ORACLE_LIB")
        if alt is None and not LIB.exists():
            build()
        lib = C.CDLL(alt or str(LIB))
        P, U, I, F, SZ = C.c_void_p, C.c_uint32, C.c_int, C.c_float, C.c_size_t
        sig = {
            "or_f16_to_f32": ([C.c_uint16], F),
            "or_f32_to_f16": ([F], C.c_uint16),
            "or_decode": ([I, P, SZ, P], I),
            "or_decode_q6_k": ([P, SZ, P], I),
            "or_decode_q5_k": ([P, SZ, P], I),
            "or_decode_q8_0": ([P, SZ, P], I),
            "or_decode_q2_k": ([P, SZ, P], I),
            "or_matvec_m1": ([P, U, U, P, P], None),
            "or_matvec_m2": ([P, U, U, P, U, P], None),
            "or_qmatvec": ([I, P, U, U, P, U, P, I], I),
            "or_quantize_act_q8": ([P, U, P, P], None),
            "or_block_dots": ([I, P, U, U, P, U, P], I),
            "or_rms_norm": ([P, P, U, F, P], None),
            "or_rope_qwen3": ([P, U, U, F], None),
            "or_rope_fma": ([P, U, U, F], None),
            "or_rope_interleaved": ([P, U, U, F], None),
            "or_softmax_div": ([P, U], None),
            "or_softmax_recip": ([P, U], None),
            "or_silu": ([F], F),
            "or_top_k": ([P, U, U, P, P], None),
            "or_route": ([P, U, U, P, P], None),
            "or_attend": ([P, P, P, U, U, U, U, I, F, P], None),
            "or_dense_layer_bytes": ([C.POINTER(DenseCfg)], SZ),
            "or_dense_step": ([C.POINTER(DenseCfg), C.POINTER(DenseWeights), P, P, P, P, U, P, U], I),
            "or_argmax": ([P, U, I], U),
            "or_set_threads": ([I], None),
            "or_gelu_tanh": ([F], F),
            "or_moe_ffn": ([C.POINTER(MoeDesc), P, U, P, P, P], I),
            "or_moe_layer_bytes": ([C.POINTER(MoeModelCfg)], SZ),
            "or_moe_model_step": ([C.POINTER(MoeModelCfg), C.POINTER(MoeModelWeights), P, P, P, P, U, P, U], I),
        }
        # synth.c (absent from the planted-mistake builds of oracle.c alone)
        optional = {
            "or_synth_gauss": ([C.c_uint64, C.c_uint64, C.c_uint64, F], F),
            "or_synth_ln_int": ([U], C.c_double),
            "or_synth_cos_turn": ([U], C.c_double),
            "or_synth_sqrt": ([C.c_double], C.c_double),
            "or_synth_blocks": ([I, P, SZ, C.c_uint64, C.c_uint64, F], I),
            "or_synth_f32": ([P, SZ, C.c_uint64, C.c_uint64, F], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        for name, (args, res) in optional.items():
            if hasattr(lib, name):
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


BLOCK = {OR_Q8_0: (32, 34), OR_Q2_K: (256, 84), OR_Q5_K: (256, 176), OR_Q6_K: (256, 210), OR_F32: (1, 4)}


def set_threads(n: int) -> None:
    """Threads for the oracle's row loops (1 = the reference's scalar path)."""
    load().or_set_threads(int(n))


def decode(dtype: int, data) -> np.ndarray:
    raw = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray)
                               else data.view(np.uint8).reshape(-1))
    e, b = BLOCK[dtype]
    out = np.empty(max(raw.size // b * e, 1), np.float32)
    st = load().or_decode(dtype, _p(raw), raw.size, _p(out))
    if st != 0:
        raise ValueError(f"oracle decode failed ({st}): partial block")
    return out[: raw.size // b * e]


def matvec_m1(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(w.shape[0], np.float32)
    load().or_matvec_m1(_p(w), w.shape[0], w.shape[1], _p(x), _p(y))
    return y


def matvec_m2(w: np.ndarray, x: np.ndarray, positions: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(w.shape[0] * positions, np.float32)
    load().or_matvec_m2(_p(w), w.shape[0], w.shape[1], _p(x), positions, _p(y))
    return y


def qmatvec(dtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, n_tok: int, mode: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.empty(rows * n_tok, np.float32)
    st = load().or_qmatvec(dtype, _p(w), rows, cols, _p(x), n_tok, _p(y), mode)
    if st != 0:
        raise ValueError(f"oracle qmatvec failed ({st})")
    return y


def quantize_act(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    q = np.empty(x.size, np.int8)
    s = np.empty(x.size // 32, np.float32)
    load().or_quantize_act_q8(_p(x), x.size, _p(q), _p(s))
    return q, s


def block_dots(dtype: int, w: np.ndarray, rows: int, cols: int, xq: np.ndarray, n_tok: int) -> np.ndarray:
    sub = 16 if dtype in (OR_Q6_K, OR_Q2_K) else 32
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    xq = np.ascontiguousarray(xq, np.int8).reshape(-1)
    out = np.empty(n_tok * rows * (cols // sub), np.int32)
    st = load().or_block_dots(dtype, _p(w), rows, cols, _p(xq), n_tok, _p(out))
    if st != 0:
        raise ValueError(f"oracle block_dots failed ({st})")
    return out


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    load().or_rms_norm(_p(x), _p(w), x.size, eps, _p(y))
    return y


def rope(kind: str, head: np.ndarray, position: int, theta: float) -> np.ndarray:
    h = np.array(head, np.float32, copy=True)
    fn = {"qwen3": load().or_rope_qwen3, "fma": load().or_rope_fma,
          "interleaved": load().or_rope_interleaved}[kind]
    fn(_p(h), h.size, position, theta)
    return h


def softmax(v: np.ndarray, recip: bool = False) -> np.ndarray:
    v = np.array(v, np.float32, copy=True)
    (load().or_softmax_recip if recip else load().or_softmax_div)(_p(v), v.size)
    return v


def gelu_tanh(x: float) -> float:
    return float(load().or_gelu_tanh(x))


def moe_ffn(enc_gate_up: int, enc_down: int, gate, up, down, down_scale, n_experts: int, width: int, ff: int,
            k: int, act: int, x: np.ndarray, ids: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """Selected-expert FFN (moe::run after routing); x is n_tok x width."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, width)
    n_tok = x.shape[0]
    ids = np.ascontiguousarray(ids, np.uint32).reshape(n_tok, k)
    weights = np.ascontiguousarray(weights, np.float32).reshape(n_tok, k)
    bufs = [np.ascontiguousarray(a).view(np.uint8) if a is not None else None for a in (gate, up, down)]
    sc = np.ascontiguousarray(down_scale, np.float32) if down_scale is not None else None
    d = MoeDesc(enc_gate_up, enc_down, *[b.ctypes.data if b is not None else None for b in bufs],
                sc.ctypes.data if sc is not None else None, n_experts, width, ff, k, act)
    out = np.empty((n_tok, width), np.float32)
    st = load().or_moe_ffn(C.byref(d), _p(x), n_tok, _p(ids), _p(weights), _p(out))
    if st != 0:
        raise ValueError(f"oracle moe_ffn failed ({st})")
    return out


def silu(x: float) -> float:
    return load().or_silu(x)


def top_k(v: np.ndarray, k: int) -> list[tuple[int, float]]:
    v = np.ascontiguousarray(v, np.float32)
    idx = np.empty(k, np.uint32)
    val = np.empty(k, np.float32)
    load().or_top_k(_p(v), v.size, k, _p(idx), _p(val))
    return [(int(i), float(x)) for i, x in zip(idx, val)]


def route(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.uint32)
    w = np.empty(k, np.float32)
    load().or_route(_p(logits), logits.size, k, _p(ids), _p(w))
    return ids, w


def attend(q, keys, values, positions, heads, kv_heads, hd, variant, c=0.0) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(heads * hd, np.float32)
    load().or_attend(_p(q), _p(keys), _p(values), positions, heads, kv_heads, hd, variant, c, _p(out))
    return out


def argmax(v: np.ndarray, tie_last: bool) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(load().or_argmax(_p(v), v.size, int(tie_last)))


class MoeModelCfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("vocab", C.c_uint32), ("layers", C.c_uint32), ("context", C.c_uint32), ("n_experts", C.c_uint32),
        ("experts_used", C.c_uint32), ("expert_ff", C.c_uint32), ("rope_theta", C.c_float), ("eps", C.c_float),
        ("embed_scale", C.c_float), ("residual_scale", C.c_float), ("logit_div", C.c_float),
        ("score_mul", C.c_float), ("dtype", C.c_int32), ("expert_dtype", C.c_int32), ("kv_f16", C.c_int32),
        ("qk_norm", C.c_int32), ("rope_neox", C.c_int32), ("untied", C.c_int32), ("gemma", C.c_int32),
        ("expert_down_dtype", C.c_int32), ("shared_ff", C.c_uint32), ("window", C.c_uint32),
        ("global_every", C.c_uint32), ("rope_theta_global", C.c_float), ("softcap", C.c_float),
    ]


MOE_WEIGHT_KEYS = ("layers", "embed", "attn_norm", "ffn_norm", "q_norm", "k_norm", "out_norm", "output", "ffn_norm2")


class MoeModelWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in MOE_WEIGHT_KEYS]


def moe_layer_bytes(cfg: MoeModelCfg) -> int:
    return int(load().or_moe_layer_bytes(C.byref(cfg)))


class MoeModelOracle:
    """Reference decode steps for a mixture-of-experts decoder (or_moe_model_step)."""

    def __init__(self, cfg: MoeModelCfg, weights: dict, n_clients: int):
        self.cfg = cfg
        self.w = {k: np.ascontiguousarray(v) for k, v in weights.items()}
        self.ws = MoeModelWeights(*[_p(self.w[k]) if k in self.w else None for k in MOE_WEIGHT_KEYS])
        kw = cfg.kv_heads * cfg.head_dim
        self.n = n_clients
        self.k = np.zeros(n_clients * cfg.layers * cfg.context * kw, np.float32)
        self.v = np.zeros_like(self.k)
        self.pos = np.zeros(n_clients, np.uint32)

    def step(self, tokens, layers_limit: int = 0, want_logits: bool = True):
        """One decode step; without want_logits the output projection is
        skipped (the cache is filled the same) and None is returned."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.n * self.cfg.vocab, np.float32) if want_logits else None
        st = load().or_moe_model_step(C.byref(self.cfg), C.byref(self.ws), _p(self.k), _p(self.v), _p(self.pos),
                                      _p(toks), self.n, _p(logits) if logits is not None else None, layers_limit)
        if st != 0:
            raise ValueError(f"oracle MoE step failed ({st})")
        self.pos += 1
        return logits.reshape(self.n, self.cfg.vocab) if logits is not None else None


class DenseOracle:
    """Reference decode steps for a dense decoder (or_dense_step)."""

    def __init__(self, cfg: DenseCfg, weights: dict, n_clients: int):
        self.cfg = cfg
        self.w = {k: np.ascontiguousarray(v) for k, v in weights.items()}
        self.ws = DenseWeights(*[_p(self.w[k]) for k in
                                 ("layers", "embed", "output", "attn_norm", "ffn_norm", "q_norm", "k_norm",
                                  "out_norm")])
        kw = cfg.kv_heads * cfg.head_dim
        self.n = n_clients
        self.k = np.zeros(n_clients * cfg.layers * cfg.context * kw, np.float32)
        self.v = np.zeros_like(self.k)
        self.pos = np.zeros(n_clients, np.uint32)

    def step(self, tokens, layers_limit: int = 0, want_logits: bool = True):
        """One decode step; without want_logits the output projection is
        skipped (the cache is filled the same) and None is returned."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.n * self.cfg.vocab, np.float32) if want_logits else None
        st = load().or_dense_step(C.byref(self.cfg), C.byref(self.ws), _p(self.k), _p(self.v), _p(self.pos),
                                  _p(toks), self.n, _p(logits) if logits is not None else None, layers_limit)
        if st != 0:
            raise ValueError(f"oracle dense step failed ({st})")
        self.pos += 1
        return logits.reshape(self.n, self.cfg.vocab) if logits is not None else None

    def cache(self, client: int, layer: int, values: bool) -> np.ndarray:
        c = self.cfg
        kw = c.kv_heads * c.head_dim
        buf = self.v if values else self.k
        base = (client * c.layers + layer) * c.context * kw
        return buf[base: base + c.context * kw].reshape(c.context, kw)


def synth_blocks(dtype: int, nbytes: int, seed: int, stream: int, sd: float = 0.02) -> np.ndarray:
    """The bytes emu_model_synth writes for one quantized tensor (synth.c)."""
    be, bb = BLOCK[dtype]
    if nbytes % bb:
        raise ValueError(f"{nbytes} bytes is not whole {bb}-byte blocks")
    out = np.empty(nbytes, np.uint8)
    if load().or_synth_blocks(dtype, _p(out), nbytes // bb, seed, stream, sd) != 0:
        raise ValueError(f"dtype {dtype} has no synthesis")
    return out


def synth_f32(n: int, seed: int, stream: int, sd: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().or_synth_f32(_p(out), n, seed, stream, sd)
    return out


def synth_dense_weights(cfg: DenseCfg, seed: int) -> dict:
    """A dense decoder's weights as emu_model_synth writes them and
    Model.host_weights() reads them back: per layer q, k, v, o, gate, up,
    down (tensor t of layer l from stream 16 (l + 1) + t), the embedding
    (stream 1), the output matrix (stream 2, unless tied) and every norm gain
    1.0."""
    be, bb = BLOCK[cfg.dtype]
    qw, kw = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim

    def rb(cols):
        return cols // be * bb

    shapes = [(qw, cfg.hidden), (kw, cfg.hidden), (kw, cfg.hidden), (cfg.hidden, qw), (cfg.ffn, cfg.hidden),
              (cfg.ffn, cfg.hidden), (cfg.hidden, cfg.ffn)]
    layer_bytes = sum(r * rb(c) for r, c in shapes)
    layers = np.empty(cfg.layers * layer_bytes, np.uint8)
    for l in range(cfg.layers):
        off = l * layer_bytes
        for t, (r, c) in enumerate(shapes):
            n = r * rb(c)
            layers[off:off + n] = synth_blocks(cfg.dtype, n, seed, 16 * (l + 1) + t)
            off += n
    embed = synth_blocks(cfg.dtype, cfg.vocab * rb(cfg.hidden), seed, 1)
    ones = lambda n: np.ones(n, np.float32)  # noqa: E731
    return {
        "layers": layers, "embed": embed,
        "output": embed if cfg.tied else synth_blocks(cfg.dtype, cfg.vocab * rb(cfg.hidden), seed, 2),
        "attn_norm": ones(cfg.layers * cfg.hidden), "ffn_norm": ones(cfg.layers * cfg.hidden),
        "q_norm": ones(cfg.layers * cfg.head_dim), "k_norm": ones(cfg.layers * cfg.head_dim),
        "out_norm": ones(cfg.hidden),
    }


def _align(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def moe_layer_pieces(c, layer: int) -> list[tuple[int, int, str, int, int]]:
    """The pieces of one mixture-of-experts layer in the layer layout of
    emu_model_create, as (offset in the layer, bytes, kind, encoding or 0,
    synthesis stream): q, k, v, o, the f32 router at 16-byte alignment, then
    Granite/OLMoE: gate, up, down experts; Gemma form: router scale and
    per-expert down scales (1.0), the shared FFN's gate, up and down, the
    fused gate|up experts and the down experts.  `c` carries the model's
    shape (serve.DenseConfig's field names).  Alignment padding between
    pieces belongs to no piece."""
    enc = c.encoding

    def rb(e, cols):
        return cols // BLOCK[e][0] * BLOCK[e][1]

    H, QW, KW, E, FF = c.hidden, c.heads * c.head_dim, c.kv_heads * c.head_dim, c.n_experts, c.expert_ff
    rb_h, rb_q, rb_he = rb(enc, H), rb(enc, QW), rb(c.expert_encoding, H)
    down_enc = c.expert_down_encoding if c.gemma else c.expert_encoding
    rb_fe = rb(down_enc, FF)
    st = 16 * (layer + 1)
    pieces, off = [], 0
    for t, rows in enumerate((QW, KW, KW)):
        pieces.append((off, rows * rb_h, "blocks", enc, st + t))
        off += rows * rb_h
    pieces.append((off, H * rb_q, "blocks", enc, st + 3))
    off_r = _align(off + H * rb_q, 16)
    pieces.append((off_r, 4 * E * H, "f32", 0, st + 4))
    if c.gemma:
        off_rs = off_r + 4 * E * H
        pieces.append((off_rs, 4 * H, "ones", 0, 0))
        off_ds = _align(off_rs + 4 * H, 16)
        pieces.append((off_ds, 4 * E, "ones", 0, 0))
        off_ge = _align(off_ds + 4 * E, 16)
        if c.shared_ff:
            rb_sf, sff = rb(enc, c.shared_ff), c.shared_ff
            pieces.append((off_ge, sff * rb_h, "blocks", enc, st + 8))
            pieces.append((off_ge + sff * rb_h, sff * rb_h, "blocks", enc, st + 9))
            pieces.append((off_ge + 2 * sff * rb_h, H * rb_sf, "blocks", enc, st + 10))
            off_ge += 2 * sff * rb_h + H * rb_sf
        ge = E * 2 * FF * rb_he
        pieces.append((off_ge, ge, "blocks", c.expert_encoding, st + 5))
        pieces.append((off_ge + ge, E * H * rb_fe, "blocks", down_enc, st + 7))
    else:
        off_ge = off_r + 4 * E * H
        ge = E * FF * rb_he
        pieces.append((off_ge, ge, "blocks", c.expert_encoding, st + 5))
        pieces.append((off_ge + ge, ge, "blocks", c.expert_encoding, st + 6))
        pieces.append((off_ge + 2 * ge, E * H * rb_fe, "blocks", down_enc, st + 7))
    return pieces


def synth_moe_layer(c, seed: int, layer: int) -> list[tuple[int, np.ndarray]]:
    """The pieces (offset in the layer, bytes) of one mixture-of-experts layer
    as emu_model_synth writes them (moe_layer_pieces)."""
    out = []
    for off, n, kind, enc, stream in moe_layer_pieces(c, layer):
        if kind == "blocks":
            data = synth_blocks(enc, n, seed, stream)
        elif kind == "f32":
            data = synth_f32(n // 4, seed, stream).view(np.uint8)
        else:
            data = np.ones(n // 4, np.float32).view(np.uint8)
        out.append((off, data))
    return out


def synth_moe_weights(c, mcfg: "MoeModelCfg", seed: int) -> dict:
    """A mixture-of-experts decoder's weights as emu_model_synth writes them,
    in the layout the oracle's MoE step reads (padding zero): the layers, the
    embedding (stream 1), the output matrix (stream 2) when untied, every
    norm gain 1.0."""
    lb = moe_layer_bytes(mcfg)
    layers = np.zeros(c.layers * lb, np.uint8)
    for l in range(c.layers):
        for off, data in synth_moe_layer(c, seed, l):
            layers[l * lb + off:l * lb + off + data.size] = data
    be, bb = BLOCK[c.encoding]
    embed = synth_blocks(c.encoding, c.vocab * (c.hidden // be) * bb, seed, 1)
    ones = lambda n: np.ones(n, np.float32)  # noqa: E731
    w = {"layers": layers, "embed": embed,
         "attn_norm": ones(c.layers * c.hidden), "ffn_norm": ones(c.layers * c.hidden),
         "q_norm": ones(c.layers * c.head_dim), "k_norm": ones(c.layers * c.head_dim), "out_norm": ones(c.hidden)}
    if not c.tied:
        w["output"] = synth_blocks(c.encoding, c.vocab * (c.hidden // be) * bb, seed, 2)
    if c.gemma:
        w["ffn_norm2"] = ones(c.layers * c.hidden)
    return w
