"""Pins the CPU oracle (CPU only, no GPU).

Each check is independent of the oracle's own code: the reference's own
known-answer tests (cited), closed forms computed exactly in float64, an
independent numpy restatement (tests/npref.py), brute force on small inputs,
and invariants.  A mistake planted in the oracle (dropped term, swapped
nibble, wrong scale index, wrong tie order) fails at least one of these.
"""
import math

import numpy as np
import pytest

import oracle
from tests import npref

Q6, Q5, Q8, Q2 = oracle.OR_Q6_K, oracle.OR_Q5_K, oracle.OR_Q8_0, oracle.OR_Q2_K


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---- f16 ----------------------------------------------------------------

def test_f16_exhaustive_matches_ieee_half():
    lib = oracle.load()
    codes = np.arange(65536, dtype=np.uint16)
    ours = np.array([lib.or_f16_to_f32(int(c)) for c in codes], np.float32)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(bits(ours[~nan]), bits(ref[~nan]))
    # NaN payload kept (tensor.rs:94): fraction shifted into the f32 mantissa.
    # Only quiet NaNs survive the ctypes float -> double round trip unchanged.
    assert np.all(np.isnan(ours[nan]))
    quiet = nan & ((codes & 0x200) != 0)
    assert np.array_equal(bits(ours[quiet]) & 0x7FFFFF, (codes[quiet].astype(np.uint32) & 0x3FF) << 13)


def test_f32_to_f16_round_nearest_even():
    lib = oracle.load()
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.normal(0, 1, 4000), rng.normal(0, 1e-5, 2000), rng.normal(0, 7e4, 500),
        [0.0, -0.0, 65504.0, 65520.0, 65519.99, 6e-8, 2.98e-8, 5.96e-8, np.inf, -np.inf],
        (np.arange(1, 2048) * 2.0 ** -24),  # subnormal grid and half-way points
        (np.arange(1, 2048) * 2.0 ** -25),
    ]).astype(np.float32)
    ours = np.array([lib.or_f32_to_f16(float(x)) for x in xs], np.uint16)
    ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ---- decoders: reference KATs (spm-gguf/tests/decode.rs) -----------------

def test_q6_k_zero_code_with_unit_scale_is_minus_32():  # decode.rs:8-14
    block = np.zeros(210, np.uint8)
    block[192:208] = 1
    block[208:210] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    assert np.array_equal(oracle.decode(Q6, block), np.full(256, -32.0, np.float32))


def test_q6_k_lane_bit_packing_matches_reference_layout():  # decode.rs:16-28
    block = np.zeros(210, np.uint8)
    block[192:208] = 1
    block[208:210] = np.frombuffer(np.uint16(0x4000).tobytes(), np.uint8)
    block[0], block[32], block[128] = 0xA5, 0xC7, 0b11_10_01_00
    d = oracle.decode(Q6, block)
    assert np.array_equal(bits(d[[0, 32, 64, 96]]), bits([-54.0, -18.0, 20.0, 56.0]))


def test_q6_k_rejects_partial_block():  # decode.rs:30-33
    with pytest.raises(ValueError):
        oracle.decode(Q6, np.zeros(209, np.uint8))


def test_q5_k_known_low_nibbles_and_rejects_partial_block():  # decode.rs:35-46
    block = np.zeros(176, np.uint8)
    block[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    block[4] = 1
    block[5] = 1
    block[48:80] = 0x32
    d = oracle.decode(Q5, block)
    assert np.array_equal(d[:32], np.full(32, 2.0, np.float32))
    assert np.array_equal(d[32:64], np.full(32, 3.0, np.float32))
    with pytest.raises(ValueError):
        oracle.decode(Q5, block[:175])


def test_q8_0_signed_values_and_rejects_partial_block():  # decode.rs:48-58
    block = np.zeros(34, np.uint8)
    block[0:2] = np.frombuffer(np.uint16(0x3800).tobytes(), np.uint8)
    block[2] = 4
    block[3] = np.uint8(np.int8(-6).view(np.uint8))
    d = oracle.decode(Q8, block)
    assert abs(d[0] - 2.0) < np.finfo(np.float32).eps
    assert abs(d[1] + 3.0) < np.finfo(np.float32).eps
    with pytest.raises(ValueError):
        oracle.decode(Q8, block[:33])


def test_q6_pipeline_fixture_matches_independent_decoder():  # q6-pipeline/tests/pipeline.rs:22-35
    raw = npref.q6_pipeline_fixture(3)
    assert np.array_equal(bits(oracle.decode(Q6, raw)), bits(npref.decode_q6_k(raw)))


@pytest.mark.parametrize("dtype", [Q6, Q5, Q8, Q2])
def test_decoders_equal_exact_closed_form(dtype):
    rng = np.random.default_rng(dtype)
    raw = npref.random_blocks(dtype, 257, rng)
    ours = oracle.decode(dtype, raw)
    ref = npref.DECODERS[dtype](raw)
    assert np.array_equal(bits(ours), bits(ref))


@pytest.mark.parametrize("dtype", [Q6, Q5, Q8, Q2])
def test_decoders_with_extreme_scales(dtype):
    # subnormal and near-max f16 scales still give the single-rounding value
    rng = np.random.default_rng(100 + dtype)
    raw = npref.random_blocks(dtype, 64, rng, scale_exp=(-24, -14))
    assert np.array_equal(bits(oracle.decode(dtype, raw)), bits(npref.DECODERS[dtype](raw)))
    raw = npref.random_blocks(dtype, 64, rng, scale_exp=(4, 8))
    assert np.array_equal(bits(oracle.decode(dtype, raw)), bits(npref.DECODERS[dtype](raw)))


def test_q2_k_single_field_blocks():
    # published GGML block_q2_K: element 128N+32j+16s+l reads bits 2j of qs[32N+16s+l]
    block = np.zeros(84, np.uint8)
    block[80:82] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    block[82:84] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    block[0:16] = 1  # scale 1, min 0
    block[16 + 32 * 1 + 16 * 1 + 3] = 0b10_01_11_00  # N=1, s=1, l=3
    d = oracle.decode(Q2, block)
    for j, code in enumerate([0, 3, 1, 2]):
        assert d[128 + 32 * j + 16 + 3] == code
    assert np.count_nonzero(d) == 3
    block[0:16] = 0x20  # scale 0, min 2 -> every weight -0.5*2 = -1
    assert np.array_equal(oracle.decode(Q2, block), np.full(256, -1.0, np.float32))


# ---- matvec -------------------------------------------------------------

def test_matvec_known_matrix():  # spm-qwen3-slice/src/math.rs:62-71
    w = np.array([[1, 2], [3, 4]], np.float32)
    assert np.array_equal(oracle.matvec_m1(w, np.array([5, 6], np.float32)), [17.0, 39.0])
    assert np.array_equal(oracle.matvec_m2(w, np.array([5, 6], np.float32), 1), [17.0, 39.0])


def test_matvec_dyadic_exact_in_any_order():
    rng = np.random.default_rng(7)
    w = npref.dyadic(rng, (37, 300))
    x = npref.dyadic(rng, (300,))
    exact = (w.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(oracle.matvec_m1(w, x), exact)
    assert np.array_equal(oracle.matvec_m2(w, x, 1), exact)


def test_matvec_m1_is_sequential_separately_rounded_fold():
    rng = np.random.default_rng(8)
    w = rng.normal(size=(5, 64)).astype(np.float32)
    x = rng.normal(size=64).astype(np.float32)
    ref = []
    for r in range(5):
        acc = np.float32(-0.0)
        for c in range(64):
            acc = np.float32(acc + np.float32(w[r, c] * x[c]))
        ref.append(acc)
    assert np.array_equal(bits(oracle.matvec_m1(w, x)), bits(ref))


def test_matvec_m2_is_fma_chain():
    rng = np.random.default_rng(9)
    w = rng.normal(size=(4, 48)).astype(np.float32)
    x = rng.normal(size=(2, 48)).astype(np.float32)
    ref = np.empty(8, np.float32)
    for p in range(2):
        for r in range(4):
            acc = 0.0
            for c in range(48):  # fma = exact product + one rounding
                acc = float(np.float32(float(w[r, c]) * float(x[p, c]) + acc))
            ref[p * 4 + r] = acc
    assert np.array_equal(bits(oracle.matvec_m2(w, x, 2)), bits(ref))


@pytest.mark.parametrize("dtype", [Q6, Q5, Q8, Q2])
def test_qmatvec_is_decode_then_m1(dtype):
    rng = np.random.default_rng(20 + dtype)
    rows, cols = 7, 512
    raw = npref.random_blocks(dtype, rows * cols // npref.BLOCK_ELEMS[dtype], rng)
    x = rng.normal(size=(3, cols)).astype(np.float32)
    w = npref.DECODERS[dtype](raw).reshape(rows, cols)
    y = oracle.qmatvec(dtype, raw, rows, cols, x, 3, mode=1)
    ref = np.concatenate([oracle.matvec_m1(w, x[t]) for t in range(3)])
    assert np.array_equal(bits(y), bits(ref))


# ---- integer block dots -------------------------------------------------

def test_quantize_act_closed_form():
    rng = np.random.default_rng(11)
    x = rng.normal(size=256).astype(np.float32)
    x[32:64] = 0.0
    q, s = oracle.quantize_act(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    s_ref = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(bits(s), bits(s_ref))
    inv = np.where(s_ref != 0, np.float32(1) / np.where(s_ref != 0, s_ref, 1), 0).astype(np.float32)
    prod = (xb * inv[:, None]).astype(np.float32)
    q_ref = np.clip(np.sign(prod) * np.floor(np.abs(prod) + 0.5), -127, 127).astype(np.int8)
    assert np.array_equal(q, q_ref.reshape(-1))
    assert np.all(q[32:64] == 0)


@pytest.mark.parametrize("dtype", [Q6, Q5, Q8, Q2])
def test_block_dots_brute_force(dtype):
    rng = np.random.default_rng(30 + dtype)
    rows, cols = 5, 512
    raw = npref.random_blocks(dtype, rows * cols // npref.BLOCK_ELEMS[dtype], rng)
    xq = rng.integers(-127, 128, size=(2, cols), dtype=np.int8)
    got = oracle.block_dots(dtype, raw, rows, cols, xq, 2)
    codes = npref.codes(dtype, raw).reshape(rows, cols)
    sub = npref.SUB[dtype]
    ref = np.einsum("rc,tc->trc", codes, xq.astype(np.int64)).reshape(2, rows, cols // sub, sub).sum(-1)
    assert np.array_equal(got, ref.reshape(-1).astype(np.int32))


# ---- norms, rope, softmax, attention, routing ---------------------------

def test_rms_norm_known_vector():  # spm-qwen3-slice/src/math.rs:54-60
    r = oracle.rms_norm(np.array([3, 4], np.float32), np.array([1, 2], np.float32), 1e-6)
    assert abs(r[0] - 0.848528) < 1e-5 and abs(r[1] - 2.2627416) < 1e-5


def test_rope_identity_and_known_pair():  # spm-qwen3-slice/src/attention.rs:85-99
    head = np.arange(128, dtype=np.float32)
    for kind in ("qwen3", "fma", "interleaved"):
        assert np.array_equal(bits(oracle.rope(kind, head, 0, 1e6)), bits(head))
    h = np.zeros(128, np.float32)
    h[0] = 1.0
    r = oracle.rope("qwen3", h, 1, 1e6)
    assert abs(r[0] - math.cos(1.0)) < 1e-6 and abs(r[64] - math.sin(1.0)) < 1e-6
    r = oracle.rope("fma", h, 1, 1e5)
    assert abs(r[0] - math.cos(1.0)) < 1e-6 and abs(r[64] - math.sin(1.0)) < 1e-6
    r = oracle.rope("interleaved", h, 1, 1.5e6)
    assert abs(r[0] - math.cos(1.0)) < 1e-6 and abs(r[1] - math.sin(1.0)) < 1e-6


def test_rope_preserves_pair_norms():
    rng = np.random.default_rng(12)
    h = rng.normal(size=64).astype(np.float32)
    r = oracle.rope("qwen3", h, 517, 1e6)
    n0 = h[:32] ** 2 + h[32:] ** 2
    n1 = r[:32] ** 2 + r[32:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5)


def test_softmax_equal_large_values_exact_half():  # attention.rs:96-98, granite math.rs:46-54
    assert np.array_equal(bits(oracle.softmax([1000.0, 1000.0])), bits([0.5, 0.5]))
    assert np.array_equal(bits(oracle.softmax([1000.0, 1000.0], recip=True)), bits([0.5, 0.5]))


def test_top_k_tie_order():  # spm-qwen3-slice/src/math.rs:67-70
    assert oracle.top_k(np.array([1, 3, 3, 2], np.float32), 3) == [(1, 3.0), (2, 3.0), (3, 2.0)]


def test_olmoe_route_picks_top_eight():  # spm-granite-moe/src/moe.rs:183-191
    ids, w = oracle.route(np.arange(64, dtype=np.float32), 8)
    assert list(ids) == [63, 62, 61, 60, 59, 58, 57, 56]
    assert abs(float(w.sum()) - 1.0) < 1e-6 and np.all(np.diff(w) <= 0)


def test_gqa_maps_four_query_heads_to_each_kv_head():  # attention.rs:101-118
    heads, kvh, hd = 32, 8, 128
    q = np.zeros(heads * hd, np.float32)
    keys = np.zeros((1, kvh * hd), np.float32)
    values = np.repeat(np.arange(kvh, dtype=np.float32), hd)[None, :]
    for variant in (0, 1, 2):
        out = oracle.attend(q, keys, values, 1, heads, kvh, hd, variant, 11.313708)
        for h in range(heads):
            assert abs(out[h * hd] - h // 4) < np.finfo(np.float32).eps


def test_later_key_cannot_affect_earlier_output():  # attention.rs:120-131
    heads, kvh, hd = 4, 2, 64
    q = np.zeros(heads * hd, np.float32)
    keys = np.zeros((2, kvh * hd), np.float32)
    values = np.ones((2, kvh * hd), np.float32)
    values[1] = 99.0
    out = oracle.attend(q, keys, values, 1, heads, kvh, hd, 0, 8.0)  # prefix of one position
    assert np.array_equal(out, np.ones(heads * hd, np.float32))


def test_argmax_tie_rules():  # math.rs:38-48 vs batching.rs:111-123
    v = np.array([0.5, 2.0, 1.0, 2.0, -1.0], np.float32)
    assert oracle.argmax(v, tie_last=False) == 1
    assert oracle.argmax(v, tie_last=True) == 3


def test_dense_step_batched_equals_alone():  # spm-batch/tests/batching.rs:128-145
    rng = np.random.default_rng(5)
    cfg = oracle.DenseCfg(hidden=64, heads=2, kv_heads=1, head_dim=32, ffn=96, vocab=50, layers=2, context=8,
                          rope_theta=1e5, eps=1e-5, style=oracle.STYLE_SMOL, dtype=Q8, kv_f16=0, tied=1,
                          qk_norm=0)
    lb = oracle.load().or_dense_layer_bytes(cfg)
    w = {
        "layers": npref.random_blocks(Q8, lb * 2 // 34, rng),
        "embed": npref.random_blocks(Q8, 50 * 64 // 32, rng),
        "attn_norm": np.ones(128, np.float32), "ffn_norm": np.ones(128, np.float32),
        "q_norm": np.ones(64, np.float32), "k_norm": np.ones(64, np.float32), "out_norm": np.ones(64, np.float32),
    }
    w["output"] = w["embed"]
    both = oracle.DenseOracle(cfg, w, 2)
    alone = oracle.DenseOracle(cfg, w, 1)
    toks = [(3, 7), (11, 2), (5, 5)]
    for a, b in toks:
        lb2 = both.step([a, b])
        la = alone.step([a])
        assert np.array_equal(bits(lb2[0]), bits(la[0]))


def test_gelu_tanh_closed_form_and_odd_part():  # spm-granite-moe/src/gemma_smoke.rs:88-90
    v = np.linspace(-8, 8, 2001).astype(np.float32)
    got = np.array([oracle.gelu_tanh(float(a)) for a in v], np.float64)
    ref = npref.gelu_tanh_f64(v)
    # f32 evaluation: a few ulp relative, plus the cancellation of 1 + tanh(..) for v < 0,
    # worth at most one ulp of 1.0 times 0.5|v|
    assert np.all(np.abs(got - ref) <= 4e-7 * np.abs(ref) + 6e-8 * np.abs(v) + 1e-30)
    assert oracle.gelu_tanh(0.0) == 0.0
    # tanh is odd: gelu(v) - gelu(-v) == v in exact arithmetic
    odd = np.array([oracle.gelu_tanh(float(a)) - oracle.gelu_tanh(float(-a)) for a in v], np.float64)
    assert np.all(np.abs(odd - v) <= 2e-7 * np.maximum(np.abs(v), 1.0))


def _moe_case(rng, enc_in, enc_down, n_experts, width, ff, fused):
    n_in = n_experts * (2 if fused else 1) * ff * width // npref.BLOCK_ELEMS[enc_in]
    gate = npref.random_blocks(enc_in, n_in, rng)
    up = None if fused else npref.random_blocks(enc_in, n_in, rng)
    down = npref.random_blocks(enc_down, n_experts * width * ff // npref.BLOCK_ELEMS[enc_down], rng)
    return gate, up, down


@pytest.mark.parametrize("enc_in,enc_down,fused,gelu", [(oracle.OR_Q6_K, oracle.OR_Q6_K, False, False),
                                                        (oracle.OR_Q2_K, oracle.OR_Q2_K, False, False),
                                                        (oracle.OR_Q5_K, oracle.OR_Q8_0, True, True)])
def test_moe_ffn_against_float64_composition(enc_in, enc_down, fused, gelu):
    """moe::run (moe.rs:37-159) against an independent float64 restatement
    built from numpy decoders: per-token weighted sum of the routed experts."""
    rng = np.random.default_rng(enc_in * 7 + enc_down)
    E, W, FF, K, T = 6, 256, 256 if enc_down != oracle.OR_Q8_0 else 64, 3, 4
    gate, up, down = _moe_case(rng, enc_in, enc_down, E, W, FF, fused)
    x = rng.normal(size=(T, W)).astype(np.float32)
    logits = rng.normal(size=(T, E)).astype(np.float32)
    ids, wts = zip(*[oracle.route(logits[t], K) for t in range(T)])
    ids, wts = np.array(ids), np.array(wts)
    scale = rng.uniform(0.5, 2.0, E).astype(np.float32) if fused else None
    act = oracle.OR_ACT_GELU_TANH if gelu else oracle.OR_ACT_SILU
    got = oracle.moe_ffn(enc_in, enc_down, gate, up, down, scale, E, W, FF, K, act, x, ids, wts)
    ref = npref.moe_ffn_f64(enc_in, enc_down, gate, up, down, scale, E, W, FF, K, gelu, x, ids, wts)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_moe_ffn_single_expert_is_plain_swiglu_ffn():
    rng = np.random.default_rng(5)
    E, W, FF = 3, 256, 512
    gate, up, down = _moe_case(rng, oracle.OR_Q6_K, oracle.OR_Q6_K, E, W, FF, False)
    x = rng.normal(size=(2, W)).astype(np.float32)
    ids, wts = np.array([[1], [2]]), np.ones((2, 1), np.float32)
    got = oracle.moe_ffn(oracle.OR_Q6_K, oracle.OR_Q6_K, gate, up, down, None, E, W, FF, 1, oracle.OR_ACT_SILU,
                         x, ids, wts)
    rb_in, rb_dn = W // 256 * 210, FF // 256 * 210
    for t, e in enumerate([1, 2]):
        g = oracle.qmatvec(oracle.OR_Q6_K, gate[e * FF * rb_in:(e + 1) * FF * rb_in], FF, W, x[t], 1)
        u = oracle.qmatvec(oracle.OR_Q6_K, up[e * FF * rb_in:(e + 1) * FF * rb_in], FF, W, x[t], 1)
        h = (np.array([oracle.silu(float(a)) for a in g], np.float32) * u).astype(np.float32)
        y = oracle.qmatvec(oracle.OR_Q6_K, down[e * W * rb_dn:(e + 1) * W * rb_dn], W, FF, h, 1)
        assert np.array_equal(got[t], y)  # 0.0 + y * 1.0 == y


def test_moe_ffn_sums_experts_in_ascending_id_order():  # moe.rs:166-185
    """out = ((0 + v_lo * w_lo) + v_hi * w_hi) whatever order the route lists them in."""
    rng = np.random.default_rng(6)
    E, W, FF = 4, 256, 256
    gate, up, down = _moe_case(rng, oracle.OR_Q6_K, oracle.OR_Q6_K, E, W, FF, False)
    x = rng.normal(size=(1, W)).astype(np.float32)
    w = np.array([[0.3, 0.7]], np.float32)
    a = oracle.moe_ffn(oracle.OR_Q6_K, oracle.OR_Q6_K, gate, up, down, None, E, W, FF, 2, oracle.OR_ACT_SILU,
                       x, np.array([[3, 0]]), w)
    one = [oracle.moe_ffn(oracle.OR_Q6_K, oracle.OR_Q6_K, gate, up, down, None, E, W, FF, 1, oracle.OR_ACT_SILU,
                          x, np.array([[e]]), np.ones((1, 1), np.float32))[0] for e in (0, 3)]
    want = (np.float32(0.0) + one[0] * w[0, 1]).astype(np.float32) + (one[1] * w[0, 0]).astype(np.float32)
    assert np.array_equal(a[0], want.astype(np.float32))


def small_moe_model(seed, qk_norm=0, expert_dtype=oracle.OR_Q6_K):
    rng = np.random.default_rng(seed)
    cfg = oracle.MoeModelCfg(hidden=256, heads=4, kv_heads=2, head_dim=64, vocab=300, layers=2, context=16,
                             n_experts=8, experts_used=2, expert_ff=256, rope_theta=1.5e6, eps=1e-6,
                             embed_scale=12.0, residual_scale=0.22, logit_div=6.0, score_mul=0.015625,
                             dtype=oracle.OR_Q6_K, expert_dtype=expert_dtype, kv_f16=0, qk_norm=qk_norm)
    H, E, F = cfg.hidden, cfg.n_experts, cfg.expert_ff
    QW, KW = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    rb = {oracle.OR_Q6_K: 210, oracle.OR_Q2_K: 84}
    parts = []
    for _ in range(cfg.layers):
        parts.append(npref.random_blocks(14, (QW + 2 * KW) * H // 256, rng, scale_exp=(-12, -10)).view(np.uint8).reshape(-1))
        parts.append(npref.random_blocks(14, H * QW // 256, rng, scale_exp=(-12, -10)).view(np.uint8).reshape(-1))
        parts.append((rng.normal(size=E * H) * 0.05).astype(np.float32).view(np.uint8))
        nb = E * F * H // 256
        for _ in range(3):
            parts.append(npref.random_blocks(expert_dtype, nb, rng, scale_exp=(-12, -10)).view(np.uint8).reshape(-1))
    layers = np.concatenate(parts)
    assert layers.size == cfg.layers * oracle.moe_layer_bytes(cfg)
    w = {"layers": layers,
         "embed": npref.random_blocks(14, cfg.vocab * H // 256, rng, scale_exp=(-10, -8)).view(np.uint8).reshape(-1),
         "attn_norm": rng.uniform(0.5, 1.5, cfg.layers * H).astype(np.float32),
         "ffn_norm": rng.uniform(0.5, 1.5, cfg.layers * H).astype(np.float32),
         "q_norm": rng.uniform(0.5, 1.5, cfg.layers * cfg.head_dim).astype(np.float32),
         "k_norm": rng.uniform(0.5, 1.5, cfg.layers * cfg.head_dim).astype(np.float32),
         "out_norm": rng.uniform(0.5, 1.5, H).astype(np.float32)}
    return cfg, w


@pytest.mark.parametrize("expert_dtype", [oracle.OR_Q6_K, oracle.OR_Q2_K])
def test_moe_model_step_matches_float64_composition(expert_dtype):
    """The oracle's mixture-of-experts decode step (embedding x 12, interleaved
    RoPE, score x 1/64, residual adds x 0.22, f32 router, top-2 of 8 SwiGLU
    experts, tied output / 6) against an independent float64 composition."""
    cfg, w = small_moe_model(81, expert_dtype=expert_dtype)
    orc = oracle.MoeModelOracle(cfg, w, 1)
    toks = [5, 17, 299, 0, 42, 7]
    ref = npref.moe_model_f64(cfg, w, toks)
    for t, want in zip(toks, ref):
        got = orc.step([t])[0].astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), t


def test_moe_model_step_residual_scale_matters():
    """A planted change of the residual scale moves the logits: the composition
    test above can see it (the scale is not a no-op in the restatement)."""
    cfg, w = small_moe_model(82)
    a = oracle.MoeModelOracle(cfg, w, 1).step([3])[0]
    cfg.residual_scale = 0.25
    b = oracle.MoeModelOracle(cfg, w, 1).step([3])[0]
    assert np.max(np.abs(a - b)) > 1e-3 * np.max(np.abs(a))


# ---- closed forms at positions past the KATs ------------------------------

@pytest.mark.parametrize("kind,theta,hd", [("qwen3", 1e6, 128), ("fma", 1e5, 64), ("interleaved", 1.5e6, 64),
                                           ("qwen3", 1e6, 256)])
@pytest.mark.parametrize("pos", [1, 517, 2047])
def test_rope_matches_float64_rotation_at_every_index(kind, theta, hd, pos):
    """Every pair i turns by pos * theta^(-2i/hd) (spm-qwen3-slice/src/
    attention.rs:11-25, spm-ops/src/attention.rs:20-32, spm-granite-moe/src/
    attention.rs:12-26); half-split pairs (i, i+hd/2) or adjacent pairs
    (2i, 2i+1).  The f32 angle carries at most ~2 ulp of pos, hence the bound."""
    rng = np.random.default_rng(pos + hd)
    h = rng.normal(size=hd).astype(np.float32)
    got = oracle.rope(kind, h, pos, theta).astype(np.float64)
    i = np.arange(hd // 2)
    ang = pos * np.power(float(np.float32(theta)), -2.0 * i / hd)
    c, s = np.cos(ang), np.sin(ang)
    if kind == "interleaved":
        a, b = h[0::2].astype(np.float64), h[1::2].astype(np.float64)
        ga, gb = got[0::2], got[1::2]
    else:
        a, b = h[:hd // 2].astype(np.float64), h[hd // 2:].astype(np.float64)
        ga, gb = got[:hd // 2], got[hd // 2:]
    norm = np.sqrt(a * a + b * b)
    tol = norm * (3e-7 * pos + 1e-6)
    assert np.all(np.abs(ga - (a * c - b * s)) <= tol)
    assert np.all(np.abs(gb - (a * s + b * c)) <= tol)


@pytest.mark.parametrize("variant", [0, 1, 2])
def test_attend_with_nonzero_queries_matches_float64(variant):
    """Scores scaled as each reference form states -- dot / c (spm-qwen3-slice/
    src/attention.rs:63), dot * (1/sqrt(hd)) (spm-kv/src/attend.rs:37-60),
    dot * c (spm-granite-moe/src/attention.rs:44) -- then softmax and the
    probability-weighted sum of values, in float64 at a real spread of scores."""
    rng = np.random.default_rng(40 + variant)
    heads, kvh, hd, positions = 8, 2, 64, 37
    q = rng.normal(size=heads * hd).astype(np.float32)
    keys = rng.normal(size=(positions, kvh * hd)).astype(np.float32)
    values = rng.normal(size=(positions, kvh * hd)).astype(np.float32)
    c = {0: 8.0, 1: 0.0, 2: 0.125}[variant]
    got = oracle.attend(q, keys, values, positions, heads, kvh, hd, variant, c)
    scale = {0: 1.0 / 8.0, 1: 1.0 / math.sqrt(hd), 2: 0.125}[variant]
    ref = npref.attend_f64(q, keys, values, heads, kvh, hd, scale)
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))
    # the scores are far from uniform, so a wrong scale cannot hide
    flat = npref.attend_f64(q, keys, values, heads, kvh, hd, scale * 0.5)
    assert np.max(np.abs(flat - ref)) > 1e-2 * np.max(np.abs(ref))


def small_dense_model(seed, style, dtype, tied, qk_norm, kv_f16, hidden=256, heads=4, kv_heads=2, head_dim=64,
                      ffn=512, vocab=300, layers=2, context=16):
    rng = np.random.default_rng(seed)
    theta, eps = (1e6, 1e-6) if style == oracle.STYLE_QWEN3 else (1e5, 1e-5)
    cfg = oracle.DenseCfg(hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=ffn, vocab=vocab,
                          layers=layers, context=context, rope_theta=theta, eps=eps, style=style, dtype=dtype,
                          kv_f16=kv_f16, tied=tied, qk_norm=qk_norm)
    lb = oracle.load().or_dense_layer_bytes(cfg)
    bb, be = npref.BLOCK_BYTES[dtype], npref.BLOCK_ELEMS[dtype]
    sexp = (-12, -10) if dtype == Q6 else (-8, -6)
    w = {
        "layers": npref.random_blocks(dtype, layers * lb // bb, rng, scale_exp=sexp),
        "embed": npref.random_blocks(dtype, vocab * hidden // be, rng, scale_exp=sexp),
        "output": npref.random_blocks(dtype, vocab * hidden // be, rng, scale_exp=sexp),
        "attn_norm": rng.uniform(0.5, 1.5, layers * hidden).astype(np.float32),
        "ffn_norm": rng.uniform(0.5, 1.5, layers * hidden).astype(np.float32),
        "q_norm": rng.uniform(0.5, 1.5, layers * head_dim).astype(np.float32),
        "k_norm": rng.uniform(0.5, 1.5, layers * head_dim).astype(np.float32),
        "out_norm": rng.uniform(0.5, 1.5, hidden).astype(np.float32),
    }
    return cfg, w


DENSE_FORMS = {
    "qwen3": dict(style=oracle.STYLE_QWEN3, dtype=Q6, tied=0, qk_norm=1, kv_f16=0),
    "qwen3_f16kv": dict(style=oracle.STYLE_QWEN3, dtype=Q6, tied=0, qk_norm=1, kv_f16=1),
    "smol": dict(style=oracle.STYLE_SMOL, dtype=Q8, tied=1, qk_norm=0, kv_f16=0),
    "smol_f16kv_untied": dict(style=oracle.STYLE_SMOL, dtype=Q8, tied=0, qk_norm=0, kv_f16=1),
}


@pytest.mark.parametrize("form", list(DENSE_FORMS))
def test_dense_step_matches_float64_composition(form):
    """or_dense_step (the Qwen3 slice's layer, spm-qwen3-slice/src/model.rs:35-171,
    and spm-batch's, inner.rs:16-105) against an independent float64
    composition: QK-norm, the RoPE schedule at positions 0..7, the score scale,
    SwiGLU, both residual adds, the final norm, tied or untied logits.  A
    planted mistake in any of these moves the logits well past the bound."""
    cfg, w = small_dense_model(70 + len(form), **DENSE_FORMS[form])
    orc = oracle.DenseOracle(cfg, w, 1)
    toks = [5, 17, 299, 0, 42, 7, 123, 5]
    ref = npref.dense_model_f64(cfg, w, toks)
    for t, want in zip(toks, ref):
        got = orc.step([t])[0].astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), (form, t)



def test_qmatvec_threads_give_identical_bits():
    """Rows are independent and keep their own sequential fold, so the
    multi-threaded oracle equals the single-threaded one bit for bit."""
    rng = np.random.default_rng(90)
    rows, cols = 1024, 4096
    raw = npref.random_blocks(Q6, rows * cols // 256, rng)
    x = rng.normal(size=(2, cols)).astype(np.float32)
    try:
        oracle.set_threads(1)
        one = oracle.qmatvec(Q6, raw, rows, cols, x, 2, mode=1)
        one_m2 = oracle.qmatvec(Q6, raw, rows, cols, x, 2, mode=2)
        oracle.set_threads(8)
        many = oracle.qmatvec(Q6, raw, rows, cols, x, 2, mode=1)
        many_m2 = oracle.qmatvec(Q6, raw, rows, cols, x, 2, mode=2)
    finally:
        oracle.set_threads(1)
    assert np.array_equal(bits(one), bits(many))
    assert np.array_equal(bits(one_m2), bits(many_m2))


def test_lane_major_layout_gives_each_unit_its_codes():
    """The lane-major Q6_K layout (the batch-1 device copy) read at the offsets
    the kernel's loader uses -- code words at 16L, 1024 + 16L, 2048 + 16L,
    scales at 3072 + 8(L/2), d at 3328 + 2(L/4) in each 16-block chunk -- and
    decoded as the kernel decodes (sub-blocks 0-2: the low six bits of W0, W1,
    W2; sub-block 3: their top two bits, in that order) dequantizes, weight for
    weight, to the oracle's GGUF decoder (spm-gguf/src/tensor.rs:103-139):
    d * scales[8h + 2j + m] * (code - 32) at column 128h + 32j + 16m + i."""
    rng = np.random.default_rng(95)
    raw = rng.integers(0, 256, size=48 * 210, dtype=np.uint8)  # three chunks: one 12288-column row
    raw.reshape(-1, 210)[:, 208:210] = np.frombuffer(rng.uniform(0.5, 2.0, 48).astype(np.float16).tobytes(),
                                                     np.uint8).reshape(-1, 2)  # finite d
    lm = npref.lane_major_q6k(raw)
    assert lm.size == raw.size
    ref = oracle.decode(Q6, raw).reshape(-1, 256)
    checked = 0
    for chunk in range(3):
        c = lm[3360 * chunk:3360 * (chunk + 1)]
        for L in range(64):
            blk, h, m = L // 4, (L // 2) % 2, L % 2
            w0, w1, w2 = (c[o + 16 * L:o + 16 * L + 16].astype(np.int32) for o in (0, 1024, 2048))
            codes = [w0 & 63, w1 & 63, w2 & 63, (w0 >> 6) | (w1 >> 6) << 2 | (w2 >> 6) << 4]
            sc = c[3072 + 8 * (L // 2):3080 + 8 * (L // 2)].view(np.int8)
            d = c[3328 + 2 * (L // 4):3330 + 2 * (L // 4)].view(np.float16)[0].astype(np.float32)
            for j in range(4):
                w = (d * np.float32(sc[2 * j + m])) * (codes[j].astype(np.float32) - np.float32(32))
                cols = 128 * h + 32 * j + 16 * m + np.arange(16)
                assert np.array_equal(w, ref[16 * chunk + blk, cols]), (chunk, L, j)
                checked += 16
    assert checked == 48 * 256


def test_mfma_major_layout_gives_each_lane_its_operand_codes():
    """The matrix-core operand layout of Q6_K (the multi-token device copy),
    read where the kernel's loader reads -- lane l = 32 kh + j's 24 code words
    at 1024 (w // 4) + 16 l + 4 (w % 4), the row's scales at 6144 + 16 j and
    d at 6656 + 2 j of each 6720-byte (tile, block) chunk -- and decoded as
    the kernel decodes (sub-blocks 4g..4g+2: the low six bits of words 6g+3p,
    6g+3p+1, 6g+3p+2; sub-block 4g+3: their top two bits, in that order),
    dequantizes, weight for weight, to the oracle's GGUF decoder
    (spm-gguf/src/tensor.rs:103-139), the padding rows of the last tile
    repeating the last row."""
    rng = np.random.default_rng(96)
    rows, cols = 37, 512  # two tiles, the second padded
    raw = rng.integers(0, 256, size=rows * cols // 256 * 210, dtype=np.uint8)
    raw.reshape(-1, 210)[:, 208:210] = np.frombuffer(
        rng.uniform(0.5, 2.0, raw.size // 210).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    mm = npref.mfma_major_q6k(raw, rows, cols)
    nblk, ntile = cols // 256, (rows + 31) // 32
    assert mm.size == ntile * nblk * 6720
    ref = oracle.decode(Q6, raw).reshape(rows, cols)
    checked = 0
    for t in range(ntile):
        for k in range(nblk):
            c = mm[6720 * (t * nblk + k):6720 * (t * nblk + k + 1)]
            for lane in range(64):
                j, kh = lane % 32, lane // 32
                row = min(32 * t + j, rows - 1)
                words = [c[1024 * (w // 4) + 16 * lane + 4 * (w % 4):][:4].astype(np.int32) for w in range(24)]
                sc = c[6144 + 16 * j:6160 + 16 * j].view(np.int8)
                d = c[6656 + 2 * j:6658 + 2 * j].view(np.float16)[0].astype(np.float32)
                for sb in range(16):
                    g, jj = sb // 4, sb % 4
                    for p in range(2):
                        w0, w1, w2 = words[6 * g + 3 * p:6 * g + 3 * p + 3]
                        code = [w0 & 63, w1 & 63, w2 & 63, (w0 >> 6) | (w1 >> 6) << 2 | (w2 >> 6) << 4][jj]
                        wt = (d * np.float32(sc[sb])) * (code.astype(np.float32) - np.float32(32))
                        cols_here = 256 * k + 16 * sb + 8 * kh + 4 * p + np.arange(4)
                        assert np.array_equal(wt, ref[row, cols_here]), (t, k, lane, sb, p)
                        checked += 4
    assert checked == ntile * 32 * cols


def _moe_weights(cfg, rng, w_extra=None):
    """Seeded blobs in the layer layout of or_moe_layer_bytes for cfg."""
    H, E, F = cfg.hidden, cfg.n_experts, cfg.expert_ff
    QW, KW = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    dt, et = cfg.dtype, cfg.expert_dtype

    def blocks(dtype, n_elems, sexp=(-12, -10)):
        return npref.random_blocks(dtype, n_elems // npref.BLOCK_ELEMS[dtype], rng,
                                   scale_exp=sexp).view(np.uint8).reshape(-1)

    parts = []
    for _ in range(cfg.layers):
        parts.append(blocks(dt, (QW + 2 * KW) * H))
        parts.append(blocks(dt, H * QW))
        parts.append((rng.normal(size=E * H) * 0.05).astype(np.float32).view(np.uint8))
        if cfg.gemma:
            parts.append(rng.uniform(0.5, 1.5, H).astype(np.float32).view(np.uint8))  # router scale
            parts.append(rng.uniform(0.5, 2.0, E).astype(np.float32).view(np.uint8))  # down scale
            if cfg.shared_ff:
                parts += [blocks(dt, cfg.shared_ff * H), blocks(dt, cfg.shared_ff * H), blocks(dt, H * cfg.shared_ff)]
            parts.append(blocks(et, E * 2 * F * H, (-8, -6) if et == Q5 else (-12, -10)))
            parts.append(blocks(cfg.expert_down_dtype, E * H * F, (-8, -6)))
        else:
            for _ in range(3):
                parts.append(blocks(et, E * F * H))
    layers = np.concatenate(parts)
    assert layers.size == cfg.layers * oracle.moe_layer_bytes(cfg)
    w = {"layers": layers, "embed": blocks(dt, cfg.vocab * H, (-10, -8)),
         "output": blocks(dt, cfg.vocab * H, (-10, -8)),
         "attn_norm": rng.uniform(0.5, 1.5, cfg.layers * H).astype(np.float32),
         "ffn_norm": rng.uniform(0.5, 1.5, cfg.layers * H).astype(np.float32),
         "ffn_norm2": rng.uniform(0.5, 1.5, cfg.layers * H).astype(np.float32),
         "q_norm": rng.uniform(0.5, 1.5, cfg.layers * cfg.head_dim).astype(np.float32),
         "k_norm": rng.uniform(0.5, 1.5, cfg.layers * cfg.head_dim).astype(np.float32),
         "out_norm": rng.uniform(0.5, 1.5, H).astype(np.float32)}
    return w


def small_olmoe_model(seed):
    """OLMoE form: Q6_K attention with per-head QK-norm and half-split RoPE,
    16/16-style equal head counts, Q2_K SwiGLU experts, untied output, no
    Granite constants."""
    rng = np.random.default_rng(seed)
    cfg = oracle.MoeModelCfg(hidden=256, heads=4, kv_heads=4, head_dim=64, vocab=300, layers=2, context=16,
                             n_experts=8, experts_used=3, expert_ff=256, rope_theta=1e4, eps=1e-5, embed_scale=0.0,
                             residual_scale=0.0, logit_div=0.0, score_mul=0.125, dtype=Q6, expert_dtype=Q2,
                             kv_f16=0, qk_norm=1, rope_neox=1, untied=1)
    return cfg, _moe_weights(cfg, rng)


def small_gemma_model(seed, kv_f16=0):
    """Gemma-4 form: head_dim 256, local layers with a 4-position window and
    global ones at a second RoPE base, a shared GeGLU FFN, fused Q5_K
    gate|up experts and Q8_0 downs with per-expert scales, the scaled router
    input, x sqrt(hidden) embeddings, logits soft-capped at 30."""
    rng = np.random.default_rng(seed)
    cfg = oracle.MoeModelCfg(hidden=512, heads=2, kv_heads=1, head_dim=256, vocab=300, layers=2, context=16,
                             n_experts=8, experts_used=3, expert_ff=64, rope_theta=1e4, eps=1e-6,
                             embed_scale=float(np.float32(np.sqrt(512.0))), residual_scale=0.0, logit_div=0.0,
                             score_mul=1.0 / 16, dtype=Q6, expert_dtype=Q5, kv_f16=kv_f16, qk_norm=1, rope_neox=1,
                             untied=0, gemma=1, expert_down_dtype=Q8, shared_ff=256, window=4, global_every=2,
                             rope_theta_global=1e6, softcap=30.0)
    return cfg, _moe_weights(cfg, rng)


@pytest.mark.parametrize("form", ["olmoe", "gemma", "gemma_f16kv"])
def test_moe_model_forms_match_float64_composition(form):
    cfg, w = small_olmoe_model(83) if form == "olmoe" else small_gemma_model(84, kv_f16=int(form.endswith("kv")))
    orc = oracle.MoeModelOracle(cfg, w, 1)
    toks = [5, 17, 299, 0, 42, 7, 123, 5, 9]  # positions 0..8 pass the 4-position window
    ref = npref.moe_model_f64(cfg, w, toks)
    for t, want in zip(toks, ref):
        got = orc.step([t])[0].astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), (form, t)
    if form.startswith("gemma"):
        assert np.max(np.abs(ref[-1])) < 30.0  # the soft-cap bounds the logits


def test_moe_model_gemma_router_eps_pinned():  # spm-granite-moe/src/gemma_smoke.rs:62
    """The Gemma router input's eps (1e-6 in x * scale / sqrt(mean x^2 +
    eps) / sqrt(W)) only shows where mean x^2 is near it: here the o
    projection is zero and the embeddings are scaled by 2^-10, so the first
    layer's residual has mean x^2 of about 1e-6.  The float64 composition with
    eps 1e-5 must differ from the one with 1e-6 far beyond the bar (so this
    case sees the constant), and the oracle must follow 1e-6."""
    cfg, w = small_gemma_model(87)
    cfg.embed_scale = 2.0 ** -10
    H, QW, KW = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    per_layer = w["layers"].size // cfg.layers
    o_off = (QW + 2 * KW) * H // 256 * 210
    layers = w["layers"].copy()
    for layer in range(cfg.layers):
        base = layer * per_layer + o_off
        layers[base:base + H * QW // 256 * 210] = 0  # d = 0: the o projection adds exact zeros
    w = {**w, "layers": layers}
    toks = [5, 17, 299, 42]
    e6 = npref.moe_model_f64(cfg, w, toks)
    e5 = npref.moe_model_f64(cfg, w, toks, router_eps=1e-5)
    for a, b in zip(e6, e5):
        assert np.max(np.abs(a - b)) > 10 * 1e-4 * np.max(np.abs(a))
    orc = oracle.MoeModelOracle(cfg, w, 1)
    for t, want in zip(toks, e6):
        got = orc.step([t])[0].astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), t


def test_moe_model_batched_equals_alone():  # spm-batch/tests/batching.rs:128-145
    for cfg, w in (small_olmoe_model(85), small_gemma_model(86)):
        both, alone = oracle.MoeModelOracle(cfg, w, 2), oracle.MoeModelOracle(cfg, w, 1)
        for a, b in [(3, 7), (11, 2), (5, 5), (1, 0), (2, 2), (9, 8)]:
            assert np.array_equal(bits(both.step([a, b])[0]), bits(alone.step([a])[0]))


def test_steps_without_logits_fill_the_same_cache():
    """A prompt step without a logits buffer skips only the output
    projection: the following step's logits are the same bits."""
    for make in (lambda: small_olmoe_model(88), lambda: small_gemma_model(89)):
        cfg, w = make()
        a, b = oracle.MoeModelOracle(cfg, w, 1), oracle.MoeModelOracle(cfg, w, 1)
        for t in (3, 7, 11):
            a.step([t])
            assert b.step([t], want_logits=False) is None
        assert np.array_equal(bits(a.step([5])[0]), bits(b.step([5])[0]))
    cfg = oracle.DenseCfg(hidden=256, heads=2, kv_heads=1, head_dim=128, ffn=256, vocab=300, layers=2, context=8,
                          rope_theta=1e6, eps=1e-6, style=0, dtype=Q6, kv_f16=1, tied=0, qk_norm=1)
    w = oracle.synth_dense_weights(cfg, 17)
    a, b = oracle.DenseOracle(cfg, w, 1), oracle.DenseOracle(cfg, w, 1)
    a.step([4])
    assert b.step([4], want_logits=False) is None
    assert np.array_equal(bits(a.step([9])[0]), bits(b.step([9])[0]))
