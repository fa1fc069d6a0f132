"""Kernel parity on the GPU, through the C ABI, against the oracle.

Bars: dequant, integer block dots, activation quantisation and RoPE are
bit-exact.  Matvec is bit-exact on dyadic inputs (every summation order is
exact) and otherwise within |gpu - ref| <= 1e-5 * sum_c |w_c x_c| + 1e-30
(the reference's own sequential fold differs from any reordering by far less).
Softmax-based kernels (attention, router weights) are within 2e-6 relative
per element; router ids are identical.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from emufpga_amd import _lib, gguf
from emufpga_amd.linear import QuantMatrix, streamed
from tests import npref

pytestmark = pytest.mark.gpu

FORMATS = [_lib.Q6_K, _lib.Q5_K, _lib.Q8_0, _lib.Q2_K]


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def p(buf, off=0):
    return C.c_void_p(buf.addr + off)


def abs_scale(dtype, raw, rows, cols, x):
    w = npref.DECODERS[dtype](raw).reshape(rows, cols).astype(np.float64)
    return np.abs(w) @ np.abs(x.astype(np.float64)).T  # rows x n_tok


def close_to(got, ref, scale):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = 1e-5 * scale + 1e-30
    assert np.all(err <= bound), f"max err {err.max()} vs bound at argmax {bound.reshape(-1)[err.argmax()]}"


@pytest.mark.parametrize("dtype", FORMATS)
@pytest.mark.parametrize("offset", [0, 2, 6, 34])
def test_dequant_bit_exact(ctx, dtype, offset):
    rng = np.random.default_rng(dtype * 7 + offset)
    nblk = 333
    raw = npref.random_blocks(dtype, nblk, rng)
    padded = np.concatenate([np.zeros(offset, np.uint8), raw])
    src = ctx.upload(padded)
    out = ctx.alloc(nblk * npref.BLOCK_ELEMS[dtype] * 4)
    ctx.check(ctx.lib.emu_dequant(ctx.h, dtype, p(src, offset), raw.size, out.ptr), "dequant")
    got = out.read(np.float32)
    assert np.array_equal(bits(got), bits(oracle.decode(dtype, raw)))


def test_dequant_reference_kats(ctx):
    block = np.zeros(210, np.uint8)  # spm-gguf/tests/decode.rs:16-28
    block[192:208] = 1
    block[208:210] = np.frombuffer(np.uint16(0x4000).tobytes(), np.uint8)
    block[0], block[32], block[128] = 0xA5, 0xC7, 0b11_10_01_00
    d = gguf.decode_q6_k(block, ctx)
    assert np.array_equal(bits(d[[0, 32, 64, 96]]), bits([-54.0, -18.0, 20.0, 56.0]))
    raw = npref.q6_pipeline_fixture(3)  # q6-pipeline/tests/pipeline.rs:11-35
    assert np.array_equal(bits(gguf.decode_q6_k(raw, ctx)), bits(oracle.decode(oracle.OR_Q6_K, raw)))


@pytest.mark.parametrize("dtype", FORMATS)
def test_dequant_partial_block_is_short(ctx, dtype):
    bb = npref.BLOCK_BYTES[dtype]
    with pytest.raises(_lib.Short):
        gguf.decode(dtype, np.zeros(bb + 1, np.uint8), ctx)


def dyadic_blocks(dtype, nblk, rng):
    """Random codes, power-of-two d / dmin and small sub-block scales: every
    weight, product and partial sum is exact in f32 at the test sizes."""
    raw = npref.random_blocks(dtype, nblk, rng).reshape(nblk, -1)
    h = lambda v: np.frombuffer(np.float16(v).tobytes(), np.uint8)
    if dtype == _lib.Q6_K:
        raw[:, 192:208] = rng.integers(-2, 3, size=(nblk, 16)).astype(np.int8).view(np.uint8)
        raw[:, 208:210] = h(2.0 ** -4)
    elif dtype == _lib.Q8_0:
        raw[:, 0:2] = h(2.0 ** -6)
    elif dtype == _lib.Q5_K:
        raw[:, 0:2] = h(2.0 ** -6)
        raw[:, 2:4] = h(2.0 ** -6)
        raw[:, 4:16] = 1
    else:
        raw[:, 80:82] = h(2.0 ** -4)
        raw[:, 82:84] = h(2.0 ** -4)
        raw[:, 0:16] = rng.integers(0, 4, size=(nblk, 16)) | (rng.integers(0, 4, size=(nblk, 16)) << 4)
    return raw.reshape(-1)


@pytest.mark.parametrize("dtype", FORMATS)
@pytest.mark.parametrize("n_tok", [1, 2, 3, 8])
def test_qmatvec_dyadic_bit_exact(ctx, dtype, n_tok):
    rng = np.random.default_rng(100 * dtype + n_tok)
    rows, cols = 67, 2048
    raw = dyadic_blocks(dtype, rows * cols // npref.BLOCK_ELEMS[dtype], rng)
    x = npref.dyadic(rng, (n_tok, cols))
    m = QuantMatrix(ctx, dtype, rows, cols, raw)
    got = streamed(ctx, m, (x, n_tok))
    ref = oracle.qmatvec(dtype, raw, rows, cols, x, n_tok, mode=1)
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("dtype", FORMATS)
@pytest.mark.parametrize("n_tok", [1, 4, 5, 8])
@pytest.mark.parametrize("cols", [256, 1024, 2816])
def test_qmatvec_random_within_tolerance(ctx, dtype, n_tok, cols):
    rng = np.random.default_rng(dtype + 10 * n_tok + cols)
    rows = 45
    raw = npref.random_blocks(dtype, rows * cols // npref.BLOCK_ELEMS[dtype], rng)
    x = rng.normal(size=(n_tok, cols)).astype(np.float32)
    m = QuantMatrix(ctx, dtype, rows, cols, raw)
    got = streamed(ctx, m, (x, n_tok)).reshape(n_tok, rows)
    ref = oracle.qmatvec(dtype, raw, rows, cols, x, n_tok, mode=1).reshape(n_tok, rows)
    close_to(got, ref, abs_scale(dtype, raw, rows, cols, x).T)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288)])
def test_qmatvec_qwen3_shapes(ctx, rows, cols):
    rng = np.random.default_rng(rows + cols)
    raw = npref.random_blocks(_lib.Q6_K, rows * cols // 256, rng, scale_exp=(-14, -12))
    x = rng.normal(size=(1, cols)).astype(np.float32)
    m = QuantMatrix(ctx, _lib.Q6_K, rows, cols, raw)
    got = streamed(ctx, m, (x, 1)).reshape(1, rows)
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1).reshape(1, rows)
    close_to(got, ref, abs_scale(_lib.Q6_K, raw, rows, cols, x).T)


def test_qmatvec_output_shape_sampled_rows(ctx):
    """151936 x 4096 Q6_K (the Qwen3 output matrix): every row computed on the
    GPU, 2048 sampled rows checked against the oracle."""
    rows, cols = 151936, 4096
    rng = np.random.default_rng(3)
    raw = npref.random_blocks(_lib.Q6_K, rows * cols // 256, rng, scale_exp=(-14, -12))
    x = rng.normal(size=(1, cols)).astype(np.float32)
    m = QuantMatrix(ctx, _lib.Q6_K, rows, cols, raw)
    got = streamed(ctx, m, (x, 1))
    pick = np.sort(rng.choice(rows, 2048, replace=False))
    rb = cols // 256 * 210
    sub = raw.reshape(rows, rb)[pick].reshape(-1)
    ref = oracle.qmatvec(oracle.OR_Q6_K, sub, len(pick), cols, x, 1)
    close_to(got[pick], ref, abs_scale(_lib.Q6_K, sub, len(pick), cols, x)[:, 0])


def test_qmatvec_accumulate(ctx):
    rng = np.random.default_rng(4)
    rows, cols = 33, 512
    raw = dyadic_blocks(_lib.Q6_K, rows * cols // 256, rng)
    x = npref.dyadic(rng, (1, cols))
    base = npref.dyadic(rng, (rows,))
    m = QuantMatrix(ctx, _lib.Q6_K, rows, cols, raw)
    got = streamed(ctx, m, (x, 1), accumulate_into=base)
    ref = base + oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1)
    assert np.array_equal(bits(got), bits(ref))


def test_qmatvec_shape_errors(ctx):
    raw = np.zeros(4 * 210, np.uint8)
    m = QuantMatrix(ctx, _lib.Q6_K, 4, 256, raw)
    xb = ctx.upload(np.zeros(256, np.float32))
    yb = ctx.alloc(64)
    lib = ctx.lib
    assert lib.emu_qmatvec(ctx.h, _lib.Q6_K, m.ptr, m.nbytes - 1, 4, 256, xb.ptr, 256, 1, yb.ptr, 0) == _lib.EMU_E_SHAPE
    assert lib.emu_qmatvec(ctx.h, _lib.Q6_K, m.ptr, m.nbytes, 4, 256, xb.ptr, 255, 1, yb.ptr, 0) == _lib.EMU_E_ACTIVATION_LEN
    assert lib.emu_qmatvec(ctx.h, _lib.Q6_K, m.ptr, m.nbytes, 4, 250, xb.ptr, 256, 1, yb.ptr, 0) == _lib.EMU_E_SHORT
    assert lib.emu_qmatvec(ctx.h, 2, m.ptr, m.nbytes, 4, 256, xb.ptr, 256, 1, yb.ptr, 0) == _lib.EMU_E_UNSUPPORTED
    with pytest.raises(_lib.ActivationLen):
        streamed(ctx, m, (np.zeros(100, np.float32), 1))


@pytest.mark.parametrize("dtype", [_lib.Q6_K, _lib.Q8_0])
def test_fused_norm_and_swiglu(ctx, dtype):
    rng = np.random.default_rng(50 + dtype)
    rows, cols, eps = 96, 1024, 1e-6
    nb = rows * cols // npref.BLOCK_ELEMS[dtype]
    wg = npref.random_blocks(dtype, nb, rng)
    wu = npref.random_blocks(dtype, nb, rng)
    x = rng.normal(size=(2, cols)).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    bg, bu, bx, bgn = ctx.upload(wg), ctx.upload(wu), ctx.upload(x), ctx.upload(gain)
    y = ctx.alloc(2 * rows * 4)
    ctx.check(ctx.lib.emu_qmatvec_fused(ctx.h, dtype, bg.ptr, None, rows, cols, bx.ptr, 2, bgn.ptr, eps, y.ptr, 0),
              "fused norm")
    got = y.read(np.float32).reshape(2, rows)
    xn = np.stack([oracle.rms_norm(x[t], gain, eps) for t in range(2)])
    ref = oracle.qmatvec(dtype, wg, rows, cols, xn, 2).reshape(2, rows)
    close_to(got, ref, abs_scale(dtype, wg, rows, cols, xn).T)
    ctx.check(ctx.lib.emu_qmatvec_fused(ctx.h, dtype, bg.ptr, bu.ptr, rows, cols, bx.ptr, 2, bgn.ptr, eps, y.ptr, 0),
              "fused swiglu")
    got = y.read(np.float32).reshape(2, rows)
    g = oracle.qmatvec(dtype, wg, rows, cols, xn, 2).reshape(2, rows)
    u = oracle.qmatvec(dtype, wu, rows, cols, xn, 2).reshape(2, rows)
    ref = np.vectorize(oracle.silu)(g).astype(np.float32) * u
    sg = abs_scale(dtype, wg, rows, cols, xn).T
    su = abs_scale(dtype, wu, rows, cols, xn).T
    # silu is 1-Lipschitz-ish (|silu'| <= 1.1): propagate both operand bounds
    bound = 1.1e-5 * sg * np.abs(u) + 1e-5 * su * np.abs(g) + 1e-6 * np.abs(ref) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)


@pytest.mark.parametrize("dtype", FORMATS)
def test_block_dots_bit_exact(ctx, dtype):
    rng = np.random.default_rng(60 + dtype)
    rows, cols, n_tok = 19, 1536, 3
    raw = npref.random_blocks(dtype, rows * cols // npref.BLOCK_ELEMS[dtype], rng)
    x = rng.normal(size=(n_tok, cols)).astype(np.float32)
    bx = ctx.upload(x)
    bq = ctx.alloc(x.size)
    bs = ctx.alloc(x.size // 32 * 4)
    ctx.check(ctx.lib.emu_quantize_act(ctx.h, bx.ptr, n_tok, cols, bq.ptr, bs.ptr), "quantize_act")
    q = bq.read(np.int8)
    s = bs.read(np.float32)
    q_ref, s_ref = oracle.quantize_act(x)
    assert np.array_equal(q, q_ref) and np.array_equal(bits(s), bits(s_ref))
    bw = ctx.upload(raw)
    sub = npref.SUB[dtype]
    out = ctx.alloc(n_tok * rows * (cols // sub) * 4)
    ctx.check(ctx.lib.emu_block_dots(ctx.h, dtype, bw.ptr, raw.size, rows, cols, bq.ptr, n_tok, out.ptr), "dots")
    assert np.array_equal(out.read(np.int32), oracle.block_dots(dtype, raw, rows, cols, q_ref, n_tok))
    # int8-mode matvec equals the exact-integer formula up to f32 rounding
    y = ctx.alloc(n_tok * rows * 4)
    ctx.check(ctx.lib.emu_qmatvec_i8(ctx.h, dtype, bw.ptr, raw.size, rows, cols, bq.ptr, bs.ptr, n_tok, y.ptr),
              "qmatvec_i8")
    w = npref.DECODERS[dtype](raw).reshape(rows, cols).astype(np.float64)
    xd = (q_ref.reshape(n_tok, cols).astype(np.float64) * np.repeat(s_ref.astype(np.float64), 32).reshape(n_tok, cols))
    ref = (w @ xd.T).T
    scale = np.abs(w) @ np.abs(xd).T
    assert np.all(np.abs(y.read(np.float32).reshape(n_tok, rows) - ref) <= 1e-5 * scale.T + 1e-30)


def test_rms_norm(ctx):
    rng = np.random.default_rng(70)
    x = rng.normal(size=(3, 4096)).astype(np.float32)
    g = rng.uniform(0.5, 2, 4096).astype(np.float32)
    bx, bg, by = ctx.upload(x), ctx.upload(g), ctx.alloc(x.nbytes)
    ctx.check(ctx.lib.emu_rms_norm(ctx.h, bx.ptr, bg.ptr, 3, 4096, 1e-6, by.ptr), "rms")
    got = by.read(np.float32).reshape(3, 4096)
    ref = np.stack([oracle.rms_norm(x[i], g, 1e-6) for i in range(3)])
    assert np.allclose(got, ref, rtol=4e-6, atol=0)


@pytest.mark.parametrize("style,kind,theta,hd", [(0, "qwen3", 1e6, 128), (1, "interleaved", 1.5e6, 128),
                                                 (2, "fma", 1e5, 64), (2, "fma", 1e5, 128)])
def test_rope_bit_exact(ctx, style, kind, theta, hd):
    """All three RoPE forms, table and rotation, bit for bit against the
    oracle; style 2 is spm_ops::rope's fma form (SmolLM2)."""
    rng = np.random.default_rng(80 + style)
    heads, n_tok, table_pos = 8, 4, 2048
    x = rng.normal(size=(n_tok, heads, hd)).astype(np.float32)
    pos = np.array([0, 1, 777, 2047], np.uint32)
    tb = ctx.alloc(table_pos * hd * 4)
    if style == 2:
        ctx.check(ctx.lib.emu_rope_table_style(ctx.h, style, table_pos, hd, theta, tb.ptr), "rope_table_style")
    else:
        ctx.check(ctx.lib.emu_rope_table(ctx.h, table_pos, hd, theta, tb.ptr), "rope_table")
    bx, bp = ctx.upload(x), ctx.upload(pos)
    ctx.check(ctx.lib.emu_rope(ctx.h, bx.ptr, n_tok, heads, hd, bp.ptr, tb.ptr, table_pos, style), "rope")
    got = bx.read(np.float32).reshape(n_tok, heads, hd)
    ref = np.stack([np.stack([oracle.rope(kind, x[t, h], int(pos[t]), theta) for h in range(heads)])
                    for t in range(n_tok)])
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("kv_f16", [0, 1])
def test_attend_cached(ctx, kv_f16):
    rng = np.random.default_rng(90 + kv_f16)
    heads, kvh, hd, positions = 32, 8, 128, 700
    q = rng.normal(size=heads * hd).astype(np.float32)
    keys = rng.normal(size=(positions, kvh * hd)).astype(np.float32)
    values = rng.normal(size=(positions, kvh * hd)).astype(np.float32)
    if kv_f16:
        keys = keys.astype(np.float16).astype(np.float32)
        values = values.astype(np.float16).astype(np.float32)
        bk, bv = ctx.upload(keys.astype(np.float16)), ctx.upload(values.astype(np.float16))
    else:
        bk, bv = ctx.upload(keys), ctx.upload(values)
    bq, bo = ctx.upload(q), ctx.alloc(heads * hd * 4)
    scale = 1.0 / np.sqrt(np.float32(hd))
    ctx.check(ctx.lib.emu_attend_cached(ctx.h, bq.ptr, bk.ptr, bv.ptr, kv_f16, positions, heads, kvh, hd,
                                        float(np.float32(scale)), bo.ptr), "attend")
    got = bo.read(np.float32)
    ref = oracle.attend(q, keys, values, positions, heads, kvh, hd, 1)
    assert np.allclose(got, ref, rtol=2e-5, atol=2e-6)
    assert ctx.lib.emu_attend_cached(ctx.h, bq.ptr, bk.ptr, bv.ptr, kv_f16, 4, 6, 4, hd, 1.0, bo.ptr) \
        == _lib.EMU_E_CONFIG  # heads must group evenly (spm-kv/src/attend.rs:82-85)


@pytest.mark.parametrize("experts,k", [(256, 64), (256, 8), (128, 8), (65, 1), (40, 8), (3, 3)])
def test_route_shapes_match_oracle(ctx, experts, k):
    """The register-resident route at every expert count it takes (up to 256
    experts, 64 routed): entries past a 64-expert boundary, ties across the
    boundary (lowest id first), and all experts routed."""
    rng = np.random.default_rng(experts * 100 + k)
    n_tok = 5
    logits = rng.normal(size=(n_tok, experts)).astype(np.float32)
    logits[1, :] = 0.5  # all tied
    logits[2, ::3] = 2.0  # ties spread over every 64-expert word
    logits[3] = -logits[3] * 40.0  # probabilities far apart (underflow to zero)
    bl, bi, bw = ctx.upload(logits), ctx.alloc(n_tok * k * 4), ctx.alloc(n_tok * k * 4)
    ctx.check(ctx.lib.emu_route(ctx.h, bl.ptr, n_tok, experts, k, bi.ptr, bw.ptr), "route")
    ids = bi.read(np.int32).reshape(n_tok, k)
    w = bw.read(np.float32).reshape(n_tok, k)
    for t in range(n_tok):
        rid, rw = oracle.route(logits[t], k)
        assert list(ids[t]) == list(rid), t
        assert np.allclose(w[t], rw, rtol=2e-6, atol=1e-30), t
    assert list(ids[1]) == list(range(k))


def test_route_matches_oracle(ctx):
    rng = np.random.default_rng(95)
    n_tok, experts, k = 8, 64, 8
    logits = rng.normal(size=(n_tok, experts)).astype(np.float32)
    logits[0] = np.arange(64, dtype=np.float32)  # moe.rs:183-191
    logits[1, :] = 1.0  # all ties -> lowest ids
    bl, bi, bw = ctx.upload(logits), ctx.alloc(n_tok * k * 4), ctx.alloc(n_tok * k * 4)
    ctx.check(ctx.lib.emu_route(ctx.h, bl.ptr, n_tok, experts, k, bi.ptr, bw.ptr), "route")
    ids = bi.read(np.int32).reshape(n_tok, k)
    w = bw.read(np.float32).reshape(n_tok, k)
    for t in range(n_tok):
        rid, rw = oracle.route(logits[t], k)
        assert list(ids[t]) == list(rid)
        assert np.allclose(w[t], rw, rtol=2e-6, atol=0)
    assert list(ids[0]) == list(range(63, 55, -1))
    assert list(ids[1]) == list(range(8))


def test_argmax_tie_rules(ctx):
    v = np.zeros((2, 151936), np.float32)
    v[:, [5, 77, 150000]] = 3.5
    v[1, 9] = -0.0
    bv, bo = ctx.upload(v), ctx.alloc(8)
    ctx.check(ctx.lib.emu_argmax(ctx.h, bv.ptr, 2, 151936, 0, bo.ptr), "argmax")
    assert list(bo.read(np.int32)) == [5, 5]
    ctx.check(ctx.lib.emu_argmax(ctx.h, bv.ptr, 2, 151936, 1, bo.ptr), "argmax")
    assert list(bo.read(np.int32)) == [150000, 150000]
    for t in range(2):
        assert oracle.argmax(v[t], False) == 5 and oracle.argmax(v[t], True) == 150000


def test_session_time_layers_and_hbm_read_rate(ctx):
    """emu_session_time_layers: one step timed interval by interval (the
    embedding, each layer, the output), consuming one position; and the HBM
    read-rate probe returns a plausible rate."""
    from emufpga_amd.serve import Model, Session
    from tests.test_gpu_model import SMALL_QWEN3
    model = Model(ctx, SMALL_QWEN3)
    model.synth(5)
    sess = Session(model, 1, 8)
    sess.decode_step([3])
    us = sess.time_layers()
    assert us.shape == (SMALL_QWEN3.layers + 2,) and np.all(us > 0.0) and np.all(us < 1e5)
    assert list(sess.positions()) == [2]
    sess.close()
    model.close()
    gbs = ctx.hbm_read_rate(512 << 20, 2)
    assert 500.0 < gbs < 8000.0, gbs
