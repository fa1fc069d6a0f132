"""Independent numpy restatements used to pin the C oracle.

Written from the block layouts the reference documents (spm-gguf/src/
tensor.rs:103-210; the public GGML block_q2_K layout for Q2_K), in a different
form from the oracle: every decoded weight is the *exact* real value computed
in float64 and rounded once to float32, so a decoder that drops a term, swaps
a nibble or mis-indexes a scale disagrees bit-for-bit.  Also random-block
generators and integer-code extraction for brute-force block dots.
"""
from __future__ import annotations

import numpy as np


def f16(raw: np.ndarray) -> np.ndarray:
    """Little-endian f16 bytes (..., 2) -> float64 (exact)."""
    return np.ascontiguousarray(raw).view("<f2").astype(np.float64)[..., 0]


def q6_k_codes(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(codes q-32 [n,256], sub-block scale index [256], d [n])."""
    n = blocks.shape[0]
    e = np.arange(256)
    h, r = e // 128, e % 128
    lane, l = r // 32, r % 32
    ql_idx = 64 * h + l + 32 * (lane & 1)
    ql = blocks[:, ql_idx].astype(np.int64)
    nib = np.where((lane >> 1) == 1, ql >> 4, ql & 15)
    qh = blocks[:, 128 + 32 * h + l].astype(np.int64)
    hi = (qh >> (2 * lane)) & 3
    codes = (nib | (hi << 4)) - 32
    d = f16(blocks[:, 208:210])
    return codes, e // 16, d


def decode_q6_k(raw: np.ndarray) -> np.ndarray:
    blocks = raw.reshape(-1, 210)
    codes, si, d = q6_k_codes(blocks)
    sc = blocks[:, 192:208].view(np.int8).astype(np.float64)
    exact = d[:, None] * sc[:, si] * codes
    return exact.astype(np.float32).reshape(-1)


def q5_k_scales(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    s = blocks[:, 4:16].astype(np.int64)
    sc = np.zeros((blocks.shape[0], 8), np.int64)
    m = np.zeros_like(sc)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            m[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
            m[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, m


def q5_k_codes(blocks: np.ndarray) -> np.ndarray:
    e = np.arange(256)
    g, half, l = e // 64, (e // 32) & 1, e % 32
    qs = blocks[:, 48 + 32 * g + l].astype(np.int64)
    low = np.where(half == 1, qs >> 4, qs & 15)
    qh = blocks[:, 16 + l].astype(np.int64)
    return low + ((qh >> (2 * g + half)) & 1) * 16


def decode_q5_k(raw: np.ndarray) -> np.ndarray:
    blocks = raw.reshape(-1, 176)
    d, dmin = f16(blocks[:, 0:2]), f16(blocks[:, 2:4])
    sc, m = q5_k_scales(blocks)
    j = np.arange(256) // 32
    exact = d[:, None] * sc[:, j] * q5_k_codes(blocks) - dmin[:, None] * m[:, j]
    return exact.astype(np.float32).reshape(-1)


def decode_q8_0(raw: np.ndarray) -> np.ndarray:
    blocks = raw.reshape(-1, 34)
    d = f16(blocks[:, 0:2])
    q = blocks[:, 2:].view(np.int8).astype(np.float64)
    return (d[:, None] * q).astype(np.float32).reshape(-1)


def q2_k_codes(blocks: np.ndarray) -> np.ndarray:
    e = np.arange(256)
    N, j, s, l = e // 128, (e // 32) & 3, (e // 16) & 1, e % 16
    qs = blocks[:, 16 + 32 * N + 16 * s + l].astype(np.int64)
    return (qs >> (2 * j)) & 3


def decode_q2_k(raw: np.ndarray) -> np.ndarray:
    blocks = raw.reshape(-1, 84)
    d, dmin = f16(blocks[:, 80:82]), f16(blocks[:, 82:84])
    sc = blocks[:, 0:16].astype(np.int64)
    si = np.arange(256) // 16
    exact = d[:, None] * (sc[:, si] & 15) * q2_k_codes(blocks) - dmin[:, None] * (sc[:, si] >> 4)
    return exact.astype(np.float32).reshape(-1)


DECODERS = {14: decode_q6_k, 13: decode_q5_k, 8: decode_q8_0, 10: decode_q2_k}
BLOCK_BYTES = {14: 210, 13: 176, 8: 34, 10: 84}
BLOCK_ELEMS = {14: 256, 13: 256, 8: 32, 10: 256}
SUB = {14: 16, 13: 32, 8: 32, 10: 16}


def codes(dtype: int, raw: np.ndarray) -> np.ndarray:
    """Signed integer code of every element (the int8-mode weight code)."""
    blocks = raw.reshape(-1, BLOCK_BYTES[dtype])
    if dtype == 14:
        return q6_k_codes(blocks)[0].reshape(-1)
    if dtype == 13:
        return q5_k_codes(blocks).reshape(-1)
    if dtype == 8:
        return blocks[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
    return q2_k_codes(blocks).reshape(-1)


def random_blocks(dtype: int, nblocks: int, rng: np.random.Generator, scale_exp=(-12, -6)) -> np.ndarray:
    """Random block bytes with finite, moderate f16 scales (every byte pattern
    of the code fields is a valid block)."""
    bb = BLOCK_BYTES[dtype]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)

    def put_f16(col: int):
        v = (rng.uniform(0.5, 1.0, nblocks) * 2.0 ** rng.integers(*scale_exp, size=nblocks)).astype(np.float16)
        raw[:, col:col + 2] = v.view(np.uint8).reshape(nblocks, 2)

    if dtype == 14:
        put_f16(208)
    elif dtype == 13:
        put_f16(0)
        put_f16(2)
    elif dtype == 8:
        put_f16(0)
    elif dtype == 10:
        put_f16(80)
        put_f16(82)
    return raw.reshape(-1)


def q6_pipeline_fixture(blocks: int) -> np.ndarray:
    """fabric/crates/q6-pipeline/tests/pipeline.rs:11-20: byte i = (i%256)*73+19 mod 256."""
    i = np.arange(blocks * 210)
    return (((i % 256) * 73 + 19) % 256).astype(np.uint8)


def dyadic(rng: np.random.Generator, shape, lo=-8, hi=8, denom=16) -> np.ndarray:
    """Multiples of 1/denom: sums and products of these stay exact in f32 at test sizes."""
    return (rng.integers(lo, hi + 1, size=shape) / denom).astype(np.float32)


def gelu_tanh_f64(v):
    v = np.asarray(v, np.float64)
    return 0.5 * v * (1.0 + np.tanh(0.7978846 * v * (1.0 + 0.044715 * v * v)))


def silu_f64(v):
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


def moe_ffn_f64(enc_in, enc_down, gate, up, down, down_scale, n_experts, width, ff, k, gelu, x, ids, weights):
    """The selected-expert FFN in float64 from this module's own decoders:
    out[t] = sum over the token's slots of w * down_e(act(gate_e x) * up_e x) (* scale_e)."""
    dec_in, dec_dn = DECODERS[enc_in], DECODERS[enc_down]
    g_all = dec_in(gate).astype(np.float64)
    g_all = g_all.reshape(n_experts, (1 if up is not None else 2) * ff, width)
    u_all = dec_in(up).astype(np.float64).reshape(n_experts, ff, width) if up is not None else g_all[:, ff:]
    g_all = g_all[:, :ff]
    d_all = dec_dn(down).astype(np.float64).reshape(n_experts, width, ff)
    x = np.asarray(x, np.float64).reshape(-1, width)
    out = np.zeros_like(x)
    act = gelu_tanh_f64 if gelu else silu_f64
    for t in range(x.shape[0]):
        for s in range(k):
            e = int(ids[t][s])
            h = act(g_all[e] @ x[t]) * (u_all[e] @ x[t])
            v = d_all[e] @ h
            if down_scale is not None:
                v = v * float(down_scale[e])
            out[t] += float(weights[t][s]) * v
    return out
