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


def moe_model_f64(cfg, w: dict, tokens_per_step, layers_limit=0, router_eps=1e-6):
    """A mixture-of-experts decoder in float64 from this module's own
    decoders, for one client: the logits of every step.  Granite
    (spm-granite-moe model.rs:330-411: interleaved RoPE, scores x score_mul,
    residual x residual_scale, embeddings x embed_scale, logits / logit_div),
    OLMoE (half-split RoPE, QK-norm, untied output) and the Gemma-4 form
    (windowed local layers, a shared GeGLU FFN, the router input of
    gemma_smoke.rs:57-86, fused Q5_K gate|up experts with a Q8_0 down and a
    per-expert scale, logit soft-cap).  w holds the byte blobs and gains the
    oracle takes; cfg an oracle MoeModelCfg."""
    H, hd, NH, NKV = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads
    QW, KW, E, K, F = NH * hd, NKV * hd, cfg.n_experts, cfg.experts_used, cfg.expert_ff
    gemma = bool(cfg.gemma)
    dt, et = cfg.dtype, cfg.expert_dtype
    dn_t = cfg.expert_down_dtype if gemma else et
    SF = cfg.shared_ff if gemma else 0
    dec = DECODERS[dt]
    rbH, rbQ, rbHe, rbFd = _rb(dt, H), _rb(dt, QW), _rb(et, H), _rb(dn_t, F)
    if gemma:
        layer_bytes = ((QW + 2 * KW) * rbH + H * rbQ + 4 * (E * H + H + E) + (2 * SF * rbH + H * _rb(dt, SF)
                       if SF else 0) + E * (2 * F * rbHe + H * rbFd))
    else:
        layer_bytes = (QW + 2 * KW) * rbH + H * rbQ + 4 * E * H + E * (2 * F * rbHe + H * rbFd)
    embed = dec(np.asarray(w["embed"]).view(np.uint8).reshape(-1)).astype(np.float64).reshape(-1, H)
    out_w = dec(np.asarray(w["output"]).view(np.uint8).reshape(-1)).astype(np.float64).reshape(-1, H) \
        if cfg.untied else embed
    L = cfg.layers if not layers_limit else min(layers_limit, cfg.layers)
    blob_all = np.asarray(w["layers"]).view(np.uint8).reshape(-1)
    mats = []
    for layer in range(L):
        blob = blob_all[layer * layer_bytes:(layer + 1) * layer_bytes]
        o = 0

        def take(n):
            nonlocal o
            part = blob[o:o + n]
            o += n
            return part
        m = {"q": dec(take(QW * rbH)).astype(np.float64).reshape(QW, H),
             "k": dec(take(KW * rbH)).astype(np.float64).reshape(KW, H),
             "v": dec(take(KW * rbH)).astype(np.float64).reshape(KW, H),
             "o": dec(take(H * rbQ)).astype(np.float64).reshape(H, QW),
             "r": take(4 * E * H).view(np.float32).astype(np.float64).reshape(E, H)}
        if gemma:
            m["rscale"] = take(4 * H).view(np.float32).astype(np.float64)
            m["dscale"] = take(4 * E).view(np.float32).astype(np.float64)
            if SF:
                m["sg"] = dec(take(SF * rbH)).astype(np.float64).reshape(SF, H)
                m["su"] = dec(take(SF * rbH)).astype(np.float64).reshape(SF, H)
                m["sd"] = dec(take(H * _rb(dt, SF))).astype(np.float64).reshape(H, SF)
            m["gu"], m["d"] = take(E * 2 * F * rbHe), take(E * H * rbFd)
        else:
            m["g"], m["u"], m["d"] = take(E * F * rbHe), take(E * F * rbHe), take(E * H * rbFd)
        mats.append(m)

    eps = float(np.float32(cfg.eps))

    def gains(name, layer, n):
        return np.asarray(w[name], np.float64)[layer * n:(layer + 1) * n]

    def norm(x, gain, e=eps):
        return x / np.sqrt(np.mean(x * x) + e) * gain

    def heads_norm(x, gain):
        x = x.reshape(-1, hd)
        return (x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * gain).reshape(-1)

    def rope(x, pos, theta):
        if cfg.rope_neox:
            return rope_neox_f64(x, pos, theta, hd)
        x = x.reshape(-1, hd).copy()
        i = np.arange(hd // 2)
        ang = pos * np.power(float(np.float32(theta)), -2.0 * i / hd)
        c, s = np.cos(ang), np.sin(ang)
        a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
        x[:, 0::2], x[:, 1::2] = a * c - b * s, a * s + b * c
        return x.reshape(-1)

    def cache_round(x):
        return x.astype(np.float16).astype(np.float64) if cfg.kv_f16 else x.astype(np.float32).astype(np.float64)

    res = cfg.residual_scale if cfg.residual_scale else 1.0
    keys = [[] for _ in range(L)]
    vals = [[] for _ in range(L)]
    out = []
    for pos, tok in enumerate(tokens_per_step):
        h = embed[int(tok)] * (float(np.float32(cfg.embed_scale)) if cfg.embed_scale else 1.0)
        for layer in range(L):
            m = mats[layer]
            glob = (not gemma) or cfg.window == 0 or (layer + 1) % cfg.global_every == 0
            theta = cfg.rope_theta_global if gemma and glob else cfg.rope_theta
            xn = norm(h, gains("attn_norm", layer, H))
            q, k, v = m["q"] @ xn, m["k"] @ xn, m["v"] @ xn
            if cfg.qk_norm:
                q, k = heads_norm(q, gains("q_norm", layer, hd)), heads_norm(k, gains("k_norm", layer, hd))
            q, k = rope(q, pos, theta), rope(k, pos, theta)
            keys[layer].append(cache_round(k))
            vals[layer].append(cache_round(v))
            lo = 0 if glob else max(0, pos + 1 - cfg.window)
            att = attend_f64(q, np.stack(keys[layer][lo:]), np.stack(vals[layer][lo:]), NH, NKV, hd,
                             float(np.float32(cfg.score_mul)))
            h = h + (m["o"] @ att) * res
            if gemma:
                rin = h * m["rscale"] / np.sqrt(np.mean(h * h) + router_eps) / np.sqrt(H)
                xe = norm(h, gains("ffn_norm2", layer, H), 1e-6)
                if SF:
                    xs = norm(h, gains("ffn_norm", layer, H))
                    h = h + (m["sd"] @ (gelu_tanh_f64(m["sg"] @ xs) * (m["su"] @ xs))) * res
                lg = m["r"] @ rin
            else:
                xe = norm(h, gains("ffn_norm", layer, H))
                lg = m["r"] @ xe
            pr = np.exp(lg - lg.max())
            pr /= pr.sum()
            ids = sorted(range(E), key=lambda e: (-pr[e], e))[:K]
            wts = pr[ids] / pr[ids].sum()
            if gemma:
                moe = moe_ffn_f64(et, dn_t, m["gu"], None, m["d"], m["dscale"], E, H, F, K, True, xe,
                                  [ids], [wts])[0]
            else:
                moe = moe_ffn_f64(et, et, m["g"], m["u"], m["d"], None, E, H, F, K, False, xe, [ids], [wts])[0]
            h = h + moe * res
        lo = out_w @ norm(h, np.asarray(w["out_norm"], np.float64))
        lo = lo / (cfg.logit_div if cfg.logit_div else 1.0)
        if gemma and cfg.softcap:
            lo = cfg.softcap * np.tanh(lo / cfg.softcap)
        out.append(lo)
    return out


def _rb(dtype: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


def rope_neox_f64(x, pos: int, theta: float, hd: int):
    """Half-split rotation of each head of x by angle pos * theta^(-2i/hd),
    i = 0..hd/2-1 (the rotation both the Qwen3 slice, spm-qwen3-slice/src/
    attention.rs:11-25, and spm_ops::rope, spm-ops/src/attention.rs:20-32,
    apply): x_i' = x_i cos - x_{i+hd/2} sin, x_{i+hd/2}' = x_i sin + x_{i+hd/2} cos."""
    x = np.asarray(x, np.float64).reshape(-1, hd).copy()
    i = np.arange(hd // 2)
    ang = pos * np.power(float(np.float32(theta)), -2.0 * i / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[:, :hd // 2].copy(), x[:, hd // 2:].copy()
    x[:, :hd // 2], x[:, hd // 2:] = a * c - b * s, a * s + b * c
    return x.reshape(-1)


def attend_f64(q, keys, values, heads: int, kv_heads: int, hd: int, scale: float):
    """softmax(q_h . K_g * scale) V_g for each query head h, g = h / (heads/kv_heads)."""
    q = np.asarray(q, np.float64)
    K, V = np.asarray(keys, np.float64), np.asarray(values, np.float64)
    out = np.empty(heads * hd)
    for h in range(heads):
        g = h // (heads // kv_heads)
        sc = K[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd] * scale
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h * hd:(h + 1) * hd] = p @ V[:, g * hd:(g + 1) * hd]
    return out


def dense_model_f64(cfg, w: dict, tokens_per_step):
    """A dense decoder in float64 from this module's own decoders, one client:
    the logits of every step.  The composition of spm-qwen3-slice/src/
    model.rs:35-171 and of spm-batch/src/inner.rs:16-105 (they differ only in
    rounding order and tie rule, which float64 does not see):
      h = embed[tok]
      per layer: xn = rms(h)*g_attn; q,k,v = W xn; per head q,k: rms*g_qk
        (if qk_norm) then the half-split RoPE at the position; K/V appended
        (rounded to fp16 if the cache is fp16); att = softmax(q.k/sqrt(hd)) V;
        h += Wo att; xn = rms(h)*g_ffn; h += Wd (silu(Wg xn) * (Wu xn))
      logits = (tied ? embed : output) (rms(h)*g_out).
    cfg is an oracle DenseCfg; w holds the byte blobs and gains it takes."""
    H, hd, NH, NKV, F = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.ffn
    QW, KW, L = NH * hd, NKV * hd, cfg.layers
    dt = cfg.dtype
    dec = DECODERS[dt]
    rbH, rbQ, rbF = _rb(dt, H), _rb(dt, QW), _rb(dt, F)
    layer_bytes = (QW + 2 * KW) * rbH + H * rbQ + 2 * F * rbH + H * rbF
    blob = np.asarray(w["layers"]).view(np.uint8).reshape(-1)
    mats = []
    for layer in range(L):
        o = layer * layer_bytes
        shapes = [(QW, H, rbH), (KW, H, rbH), (KW, H, rbH), (H, QW, rbQ), (F, H, rbH), (F, H, rbH), (H, F, rbF)]
        ms = []
        for rows, cols, rb in shapes:
            ms.append(dec(blob[o:o + rows * rb]).astype(np.float64).reshape(rows, cols))
            o += rows * rb
        mats.append(ms)
    embed = dec(np.asarray(w["embed"]).view(np.uint8).reshape(-1)).astype(np.float64).reshape(-1, H)
    out_w = embed if cfg.tied else dec(np.asarray(w["output"]).view(np.uint8).reshape(-1)).astype(
        np.float64).reshape(-1, H)

    def gains(name, layer, n):
        return np.asarray(w[name], np.float64)[layer * n:(layer + 1) * n]

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + float(np.float32(cfg.eps))) * g

    def heads_rms(x, g):
        x = x.reshape(-1, hd)
        return (x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + float(np.float32(cfg.eps))) * g).reshape(-1)

    def cache_round(x):
        return x.astype(np.float16).astype(np.float64) if cfg.kv_f16 else x.astype(np.float32).astype(np.float64)

    keys = [[] for _ in range(L)]
    vals = [[] for _ in range(L)]
    out = []
    for pos, tok in enumerate(tokens_per_step):
        h = embed[int(tok)].copy()
        for layer in range(L):
            wq, wk, wv, wo, wg, wu, wd = mats[layer]
            xn = rms(h, gains("attn_norm", layer, H))
            q, k, v = wq @ xn, wk @ xn, wv @ xn
            if cfg.qk_norm:
                q, k = heads_rms(q, gains("q_norm", layer, hd)), heads_rms(k, gains("k_norm", layer, hd))
            q, k = rope_neox_f64(q, pos, cfg.rope_theta, hd), rope_neox_f64(k, pos, cfg.rope_theta, hd)
            keys[layer].append(cache_round(k))
            vals[layer].append(cache_round(v))
            att = attend_f64(q, np.stack(keys[layer]), np.stack(vals[layer]), NH, NKV, hd, 1.0 / np.sqrt(hd))
            h = h + wo @ att
            xn = rms(h, gains("ffn_norm", layer, H))
            h = h + wd @ (silu_f64(wg @ xn) * (wu @ xn))
        out.append(out_w @ rms(h, np.asarray(w["out_norm"], np.float64)))
    return out


def lane_major_q6k(raw: np.ndarray) -> np.ndarray:
    """The Q6_K lane-major layout: the block stream in chunks of 16 blocks
    (the last may hold n < 16); within a chunk unit L = 4*block + 2*half +
    slot gets three 16-byte code words at 16L, 64n + 16L and 128n + 16L, made
    from its ql-low bytes a, ql-high bytes b and qh bytes q as
      W0 = (a & 15) | (q & 3) << 4 | (b >> 4 & 3) << 6
      W1 = (b & 15) | (q >> 2 & 3) << 4 | (b >> 6) << 6
      W2 = (a >> 4) | (q & 0xf0)
    then the n blocks' 16 scale bytes (256 B for n = 16), then their d
    values."""
    blocks = np.asarray(raw, np.uint8).reshape(-1, 210)
    out = []
    for c0 in range(0, blocks.shape[0], 16):
        ch = blocks[c0:c0 + 16]
        n = ch.shape[0]
        units = np.arange(4 * n)
        j, h, m = units // 4, (units // 2) % 2, units % 2
        col = np.arange(16)
        a = ch[j[:, None], (64 * h + 16 * m)[:, None] + col]
        b = ch[j[:, None], (64 * h + 32 + 16 * m)[:, None] + col]
        q = ch[j[:, None], (128 + 32 * h + 16 * m)[:, None] + col]
        w0 = (a & 15) | (q & 3) << 4 | (b >> 4 & 3) << 6
        w1 = (b & 15) | (q >> 2 & 3) << 4 | (b >> 6) << 6
        w2 = (a >> 4) | (q & 0xF0)
        out += [w0.reshape(-1), w1.reshape(-1), w2.reshape(-1), ch[:, 192:208].reshape(-1), ch[:, 208:210].reshape(-1)]
    return np.concatenate(out) if out else np.zeros(0, np.uint8)


def mfma_major_q6k(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The Q6_K matrix-core operand layout of a rows x cols matrix: 32-row
    tiles (the last padded by repeating the last row) by 256-column blocks,
    one 6720-byte chunk each, chunk (t, k) at 6720 (t cols/256 + k).  Lane
    l = 32 kh + j owns row j's codes for columns 8 kh + 4 p + b (p, b in
    0..1, 0..3) of each 16-column sub-block s; word 6 (s/4) + 3 p + w of the
    lane (w in 0..2), at 1024 (word // 4) + 16 l + 4 (word % 4), holds in
    byte b the code of sub-block 4 (s/4) + w in its low six bits and bits
    2w, 2w + 1 of sub-block 4 (s/4) + 3's code in its top two.  Then the 32
    rows' scale bytes (16 per row) and their d (2 bytes per row)."""
    nblk = cols // 256
    blocks = np.asarray(raw, np.uint8).reshape(rows, nblk, 210)
    ntile = (rows + 31) // 32
    blocks = blocks[np.minimum(np.arange(32 * ntile), rows - 1)].reshape(ntile, 32, nblk, 210)
    code = (q6_k_codes(blocks.reshape(-1, 210))[0] + 32).reshape(ntile, 32, nblk, 256)  # 0..63
    out = np.zeros((ntile, nblk, 6720), np.uint8)
    lane = np.arange(64)
    j, kh = lane % 32, lane // 32
    for g in range(4):
        for p in range(2):
            for b in range(4):
                col = 8 * kh + 4 * p + b  # per lane
                c3 = code[:, j, :, 16 * (4 * g + 3) + col]  # (64, ntile, nblk): lanes first
                for w in range(3):
                    cw = code[:, j, :, 16 * (4 * g + w) + col]
                    byte = cw | ((c3 >> (2 * w)) & 3) << 6
                    word = 6 * g + 3 * p + w
                    off = 1024 * (word // 4) + 16 * lane + 4 * (word % 4) + b  # (64,)
                    out[:, :, off] = byte.transpose(1, 2, 0)
    out[:, :, 6144:6656] = blocks[:, :, :, 192:208].transpose(0, 2, 1, 3).reshape(ntile, nblk, 512)
    out[:, :, 6656:6720] = blocks[:, :, :, 208:210].transpose(0, 2, 1, 3).reshape(ntile, nblk, 64)
    return out.reshape(-1)
