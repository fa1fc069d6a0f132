"""Batch-1 integer-limb matvec (Q6_K rows of 4096 and 12288 columns) on the
GPU, through the C ABI, against the oracle.

The kernel carries the activation as s * (16384*L0 + 128*L1 + L2) per
16-column sub-block, exact to 2^-20 of the sub-block's largest |x|, and sums
codes times limbs exactly in int32.  Bar per row:

    |gpu - ref| <= 1e-5 * sum_c |w_c x_c|  +  2^-19 * sum_c |w_c| * amax_sb(c)

(the first term is the matvec bar of the other kernels, the second twice the
limb representation's bound).  Non-finite activations give non-finite rows,
as the reference's f32 fold does.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from emufpga_amd import _lib
from emufpga_amd.linear import QuantMatrix, streamed
from tests import npref

pytestmark = pytest.mark.gpu

Q6 = _lib.Q6_K


def weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    return npref.random_blocks(Q6, rows * cols // 256, rng, scale_exp=(-14, -12))


def limb_bound(raw, rows, cols, x):
    w = np.abs(npref.DECODERS[Q6](raw).reshape(rows, cols).astype(np.float64))
    xa = np.abs(x.astype(np.float64)).reshape(-1)
    amax = np.repeat(xa.reshape(-1, 16).max(axis=1), 16)
    return 1e-5 * (w @ xa) + 2.0 ** -19 * (w @ amax) + 1e-30


def check(got, ref, bound):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= bound), f"max err {err.max():.3e}, bound there {bound[err.argmax()]:.3e}"


@pytest.mark.parametrize("rows,cols", [(1, 4096), (7, 4096), (4099, 4096), (6144, 4096), (24576, 4096),
                                       (1, 12288), (37, 12288), (4096, 12288)])
def test_plain_matches_oracle(ctx, rows, cols):
    raw = weights(rows, cols, rows * 7 + cols)
    x = np.random.default_rng(rows).normal(size=(1, cols)).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, 1)).reshape(rows)
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1)
    check(got, ref, limb_bound(raw, rows, cols, x))


@pytest.mark.parametrize("rows,cols", [(300, 4096), (97, 12288)])
def test_dyadic_inputs_bit_exact(ctx, rows, cols):
    """Power-of-two d, sub-block scales in -2..2 and activations k/16 with
    |k| <= 32: the three limbs hold every activation exactly (k * 2^(16-e) <
    2^21), each sub-block's integer dot is a multiple of 2^12 below 2^30 (so
    its float conversion is exact), and every product and partial sum is a
    multiple of 2^-8 (the row sums of these random rows stay far below 2^15,
    inside f32's 24 bits).  So the limb kernel must equal the oracle's f32
    fold bit for bit."""
    rng = np.random.default_rng(rows + cols)
    nblk = rows * cols // 256
    raw = npref.random_blocks(Q6, nblk, rng).reshape(nblk, 210)
    raw[:, 192:208] = rng.integers(-2, 3, size=(nblk, 16)).astype(np.int8).view(np.uint8)
    raw[:, 208:210] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)
    raw = raw.reshape(-1)
    x = npref.dyadic(rng, (1, cols), lo=-32, hi=32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, 1)).reshape(rows)
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1).reshape(rows)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("cols", [4096, 12288])
def test_accumulate_matches_oracle(ctx, cols):
    rows = 515
    raw = weights(rows, cols, 11 + cols)
    rng = np.random.default_rng(12)
    x = rng.normal(size=(1, cols)).astype(np.float32)
    base = rng.normal(size=rows).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, 1), accumulate_into=base)
    ref = base + oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1)
    check(got, ref, limb_bound(raw, rows, cols, x) + 1e-7 * np.abs(ref))


def fused(ctx, wg, wu, rows, cols, x, gain, eps):
    bg = ctx.upload(wg)
    bu = ctx.upload(wu) if wu is not None else None
    bx, bgn = ctx.upload(x), ctx.upload(gain)
    y = ctx.alloc(rows * 4)
    ctx.check(ctx.lib.emu_qmatvec_fused(ctx.h, Q6, bg.ptr, bu.ptr if bu else None, rows, cols, bx.ptr, 1, bgn.ptr,
                                        eps, y.ptr, 0), "fused")
    return y.read(np.float32)


def test_norm_and_swiglu_match_oracle(ctx):
    rows, cols, eps = 12288, 4096, 1e-6
    wg, wu = weights(rows, cols, 21), weights(rows, cols, 22)
    rng = np.random.default_rng(23)
    x = (rng.normal(size=cols) * 7).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    xn = oracle.rms_norm(x, gain, eps)
    got = fused(ctx, wg, None, rows, cols, x, gain, eps)
    ref = oracle.qmatvec(oracle.OR_Q6_K, wg, rows, cols, xn, 1)
    # the normalisation's own rounding (scale from a tree sum) adds ~1e-6 relative
    check(got, ref, limb_bound(wg, rows, cols, xn) + 2e-6 * np.abs(ref))
    got = fused(ctx, wg, wu, rows, cols, x, gain, eps)
    g = ref
    u = oracle.qmatvec(oracle.OR_Q6_K, wu, rows, cols, xn, 1)
    want = np.vectorize(oracle.silu)(g).astype(np.float64) * u
    bg = limb_bound(wg, rows, cols, xn) + 2e-6 * np.abs(g)
    bu = limb_bound(wu, rows, cols, xn) + 2e-6 * np.abs(u)
    bound = 1.1 * bg * np.abs(u) + bu * np.abs(g) * 1.1 + 1e-6 * np.abs(want) + 1e-30
    check(got, want, bound)


def test_wide_dynamic_range(ctx):
    """Sub-blocks mixing magnitudes 1e-20..1e20: the bound scales with each
    sub-block's largest value, and tiny sub-blocks keep their own scale."""
    rows, cols = 300, 4096
    raw = weights(rows, cols, 31)
    rng = np.random.default_rng(32)
    x = (rng.normal(size=cols) * 10.0 ** rng.uniform(-20, 20, cols)).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x[None], 1)).reshape(rows)
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1)
    check(got, ref, limb_bound(raw, rows, cols, x))
    # an all-tiny activation is scale-invariant: 2^-100 * x gives 2^-100 * y
    tiny = (x / np.float32(1e20) * np.float32(2.0 ** -60)).astype(np.float32)
    got_t = streamed(ctx, m, (tiny[None], 1)).reshape(rows)
    ref_t = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, tiny, 1)
    check(got_t, ref_t, limb_bound(raw, rows, cols, tiny))


def test_zero_and_non_finite_activations(ctx):
    rows, cols = 64, 4096
    raw = weights(rows, cols, 41)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    zero = np.zeros((1, cols), np.float32)
    assert np.all(streamed(ctx, m, (zero, 1)) == 0.0)
    for bad in (np.nan, np.inf, -np.inf):
        x = np.random.default_rng(42).normal(size=(1, cols)).astype(np.float32)
        x[0, 1234] = bad
        got = streamed(ctx, m, (x, 1))
        ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1)
        assert not np.any(np.isfinite(ref))
        assert not np.any(np.isfinite(got)), f"{bad}: finite rows {np.isfinite(got).sum()}"


def test_large_magnitudes_do_not_overflow_early(ctx):
    """|x| near 1e33: code-times-x partial sums would pass FLT_MAX; the block
    scale is applied before them, so finite dots stay finite."""
    rows, cols = 128, 4096
    raw = weights(rows, cols, 51)
    x = (np.random.default_rng(52).normal(size=(1, cols)) * 1e33).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, 1)).reshape(rows)
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, 1)
    assert np.all(np.isfinite(ref))
    check(got, ref, limb_bound(raw, rows, cols, x))


def test_repeatable(ctx):
    """Fixed reduction order: two launches give identical bits."""
    rows, cols = 4096, 12288
    raw = weights(rows, cols, 61)
    x = np.random.default_rng(62).normal(size=(1, cols)).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    a = streamed(ctx, m, (x, 1))
    b = streamed(ctx, m, (x, 1))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- the lane-major device layout ------------------------------------------

@pytest.mark.parametrize("nblocks", [16, 48, 16 * 5 + 7, 3])
def test_lane_major_permutation_matches_numpy(ctx, nblocks):
    raw = np.random.default_rng(nblocks).integers(0, 256, size=nblocks * 210, dtype=np.uint8)
    src, dst = ctx.upload(raw), ctx.alloc(raw.size)
    ctx.check(ctx.lib.emu_weights_lane_major(ctx.h, Q6, src.ptr, raw.size, dst.ptr), "lane_major")
    assert np.array_equal(dst.read(np.uint8), npref.lane_major_q6k(raw))


def test_lane_major_refusals(ctx):
    raw = np.zeros(210 * 16, np.uint8)
    src, dst = ctx.upload(raw), ctx.alloc(raw.size)
    L = ctx.lib
    assert L.emu_weights_lane_major(ctx.h, _lib.Q8_0, src.ptr, raw.size, dst.ptr) == _lib.EMU_E_UNSUPPORTED
    assert L.emu_weights_lane_major(ctx.h, Q6, src.ptr, raw.size - 1, dst.ptr) == _lib.EMU_E_SHORT
    assert L.emu_weights_lane_major(ctx.h, Q6, src.ptr, raw.size, src.ptr) == _lib.EMU_E_ARG
    # the flag is for one token at 4096 / 12288 columns only
    x, y = ctx.upload(np.zeros(2 * 4096, np.float32)), ctx.alloc(16 * 2 * 4)
    w = ctx.upload(np.zeros(16 * 210, np.uint8))
    assert L.emu_qmatvec(ctx.h, Q6, w.ptr, 16 * 210, 1, 4096, x.ptr, 8192, 2, y.ptr,
                         _lib.EMU_MV_LANE_MAJOR) == _lib.EMU_E_UNSUPPORTED
    assert L.emu_qmatvec(ctx.h, Q6, w.ptr, 16 * 210, 4, 1024, x.ptr, 8192, 1, y.ptr,
                         _lib.EMU_MV_LANE_MAJOR) == _lib.EMU_E_UNSUPPORTED


@pytest.mark.parametrize("rows,cols", [(1, 4096), (4099, 4096), (37, 12288), (4096, 12288)])
def test_lane_major_matvec_equals_gguf_order_bit_for_bit(ctx, rows, cols):
    """Same register contents, same arithmetic: the lane-major copy gives the
    GGUF-order kernel's bits, plain, accumulated, normalised and SwiGLU."""
    raw = weights(rows, cols, 3 * rows + cols)
    rng = np.random.default_rng(rows + 1)
    x = rng.normal(size=cols).astype(np.float32)
    base = rng.normal(size=rows).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    w = ctx.upload(raw)
    lm = ctx.alloc(raw.size)
    ctx.check(ctx.lib.emu_weights_lane_major(ctx.h, Q6, w.ptr, raw.size, lm.ptr), "lane_major")
    bx, bg = ctx.upload(x), ctx.upload(gain)

    def run(wp, flags, acc):
        y = ctx.upload(base.copy()) if acc else ctx.alloc(rows * 4)
        ctx.check(ctx.lib.emu_qmatvec(ctx.h, Q6, wp, raw.size, rows, cols, bx.ptr, cols, 1, y.ptr,
                                      flags | (_lib.EMU_MV_ACCUMULATE if acc else 0)), "qmatvec")
        return y.read(np.uint32)

    for acc in (False, True):
        assert np.array_equal(run(w.ptr, 0, acc), run(lm.ptr, _lib.EMU_MV_LANE_MAJOR, acc))

    def run_fused(wp, up, flags):
        y = ctx.alloc(rows * 4)
        ctx.check(ctx.lib.emu_qmatvec_fused(ctx.h, Q6, wp, up, rows, cols, bx.ptr, 1, bg.ptr, 1e-6, y.ptr, flags),
                  "fused")
        return y.read(np.uint32)

    assert np.array_equal(run_fused(w.ptr, None, 0), run_fused(lm.ptr, None, _lib.EMU_MV_LANE_MAJOR))
    assert np.array_equal(run_fused(w.ptr, w.ptr, 0), run_fused(lm.ptr, lm.ptr, _lib.EMU_MV_LANE_MAJOR))
