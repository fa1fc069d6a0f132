"""Multi-token (2..8) Q6_K matvec on the int8 matrix cores, through the C ABI,
against the oracle.

The kernels carry each token's activation as s * (16384*L0 + 128*L1 + L2) per
16-column sub-block (exact to 2^-20 of the sub-block's largest |x|) and form
the integer sub-block dots exactly on v_mfma_i32_32x32x16_i8.  Bar per token
and row, as for the batch-1 limb kernel:

    |gpu - ref| <= 1e-5 * sum_c |w_c x_c|  +  2^-19 * sum_c |w_c| * amax_sb(c)

Tokens do not interact: a token's row sums are the same bits whichever tokens
share its launch.
"""
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
    """Per-token bound, shape (n_tok, rows)."""
    w = np.abs(npref.DECODERS[Q6](raw).reshape(rows, cols).astype(np.float64))
    xa = np.abs(x.astype(np.float64)).reshape(-1, cols)
    amax = np.repeat(xa.reshape(xa.shape[0], -1, 16).max(axis=2), 16, axis=1)
    return 1e-5 * (xa @ w.T) + 2.0 ** -19 * (amax @ w.T) + 1e-30


def check(got, ref, bound):
    got = got.reshape(bound.shape)
    ref = ref.reshape(bound.shape)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= bound), f"max err {err.max():.3e}, bound there {bound.reshape(-1)[err.argmax()]:.3e}"


@pytest.mark.parametrize("rows,cols,n_tok", [(1, 4096, 2), (31, 4096, 8), (33, 4096, 3), (4099, 4096, 8),
                                             (6144, 4096, 5), (37, 12288, 2), (4096, 12288, 8), (100, 2048, 7),
                                             # widths that end in a partly empty slice
                                             (77, 2816, 8), (40, 2304, 2), (300, 3328, 5)])
def test_plain_matches_oracle(ctx, rows, cols, n_tok):
    raw = weights(rows, cols, rows * 7 + cols + n_tok)
    x = np.random.default_rng(rows + n_tok).normal(size=(n_tok, cols)).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, n_tok))
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, n_tok)
    check(got, ref, limb_bound(raw, rows, cols, x))


@pytest.mark.parametrize("cols", [4096, 12288])
def test_accumulate_matches_oracle(ctx, cols):
    rows, n_tok = 515, 6
    raw = weights(rows, cols, 11 + cols)
    rng = np.random.default_rng(12)
    x = rng.normal(size=(n_tok, cols)).astype(np.float32)
    base = rng.normal(size=(n_tok, rows)).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, n_tok), accumulate_into=base)
    ref = base.reshape(-1) + oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, n_tok)
    check(got, ref, limb_bound(raw, rows, cols, x) + 1e-7 * np.abs(ref.reshape(n_tok, rows)))


def fused(ctx, wg, wu, rows, cols, x, n_tok, gain, eps):
    bg = ctx.upload(wg)
    bu = ctx.upload(wu) if wu is not None else None
    bx, bgn = ctx.upload(x), ctx.upload(gain)
    y = ctx.alloc(n_tok * rows * 4)
    ctx.check(ctx.lib.emu_qmatvec_fused(ctx.h, Q6, bg.ptr, bu.ptr if bu else None, rows, cols, bx.ptr, n_tok,
                                        bgn.ptr, eps, y.ptr, 0), "fused")
    return y.read(np.float32).reshape(n_tok, rows)


def test_norm_and_swiglu_match_oracle(ctx):
    rows, cols, eps, n_tok = 2048, 4096, 1e-6, 8
    wg, wu = weights(rows, cols, 21), weights(rows, cols, 22)
    rng = np.random.default_rng(23)
    x = (rng.normal(size=(n_tok, cols)) * rng.uniform(0.1, 10, (n_tok, 1))).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    xn = np.stack([oracle.rms_norm(x[t], gain, eps) for t in range(n_tok)])
    got = fused(ctx, wg, None, rows, cols, x, n_tok, gain, eps)
    g = oracle.qmatvec(oracle.OR_Q6_K, wg, rows, cols, xn, n_tok).reshape(n_tok, rows)
    # the normalisation's own rounding (scale from a tree sum) adds ~1e-6 relative
    check(got, g, limb_bound(wg, rows, cols, xn) + 2e-6 * np.abs(g))
    got = fused(ctx, wg, wu, rows, cols, x, n_tok, gain, eps)
    u = oracle.qmatvec(oracle.OR_Q6_K, wu, rows, cols, xn, n_tok).reshape(n_tok, rows)
    want = np.vectorize(oracle.silu)(g).astype(np.float64) * u
    bg = limb_bound(wg, rows, cols, xn) + 2e-6 * np.abs(g)
    bu = limb_bound(wu, rows, cols, xn) + 2e-6 * np.abs(u)
    bound = 1.1 * bg * np.abs(u) + bu * np.abs(g) * 1.1 + 1e-6 * np.abs(want) + 1e-30
    check(got, want, bound)


def test_tokens_do_not_interact(ctx):
    """Token 0's outputs are bit-identical whatever its batch partners are, and
    a non-finite value in one token leaves the others finite."""
    rows, cols = 200, 4096
    raw = weights(rows, cols, 71)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    rng = np.random.default_rng(72)
    x = rng.normal(size=(8, cols)).astype(np.float32)
    a = streamed(ctx, m, (x, 8)).reshape(8, rows)
    y = x.copy()
    y[1:] = rng.normal(size=(7, cols)) * 1e3
    b = streamed(ctx, m, (y[:3], 3)).reshape(3, rows)
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    y[2, 77] = np.nan
    c = streamed(ctx, m, (y[:3], 3)).reshape(3, rows)
    assert np.array_equal(a[0].view(np.uint32), c[0].view(np.uint32))
    assert np.all(np.isfinite(c[1])) and not np.any(np.isfinite(c[2]))


def test_wide_dynamic_range(ctx):
    rows, cols, n_tok = 300, 4096, 4
    raw = weights(rows, cols, 31)
    rng = np.random.default_rng(32)
    x = (rng.normal(size=(n_tok, cols)) * 10.0 ** rng.uniform(-20, 20, (n_tok, cols))).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, n_tok))
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, n_tok)
    check(got, ref, limb_bound(raw, rows, cols, x))


def test_large_magnitudes_do_not_overflow_early(ctx):
    rows, cols, n_tok = 128, 12288, 2
    raw = weights(rows, cols, 51)
    x = (np.random.default_rng(52).normal(size=(n_tok, cols)) * 1e33).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    got = streamed(ctx, m, (x, n_tok))
    ref = oracle.qmatvec(oracle.OR_Q6_K, raw, rows, cols, x, n_tok)
    assert np.all(np.isfinite(ref))
    check(got, ref, limb_bound(raw, rows, cols, x))


def test_repeatable(ctx):
    rows, cols, n_tok = 4096, 12288, 8
    raw = weights(rows, cols, 61)
    x = np.random.default_rng(62).normal(size=(n_tok, cols)).astype(np.float32)
    m = QuantMatrix(ctx, Q6, rows, cols, raw)
    a = streamed(ctx, m, (x, n_tok))
    b = streamed(ctx, m, (x, n_tok))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- the matrix-core operand device layout ---------------------------------

@pytest.mark.parametrize("rows,cols", [(32, 256), (37, 1024), (96, 4096), (5, 2816)])
def test_mfma_major_layout_matches_numpy(ctx, rows, cols):
    raw = np.random.default_rng(rows * cols).integers(0, 256, size=rows * cols // 256 * 210, dtype=np.uint8)
    n = ctx.lib.emu_weights_mfma_major_bytes(rows, cols)
    assert n == (rows + 31) // 32 * cols // 256 * 6720
    src, dst = ctx.upload(raw), ctx.alloc(n)
    ctx.check(ctx.lib.emu_weights_mfma_major(ctx.h, Q6, src.ptr, raw.size, rows, cols, dst.ptr), "mfma_major")
    assert np.array_equal(dst.read(np.uint8), npref.mfma_major_q6k(raw, rows, cols))


def test_mfma_major_refusals(ctx):
    L = ctx.lib
    rows, cols = 32, 4096
    raw = np.zeros(rows * cols // 256 * 210, np.uint8)
    n = L.emu_weights_mfma_major_bytes(rows, cols)
    src, dst = ctx.upload(raw), ctx.alloc(n)
    assert L.emu_weights_mfma_major_bytes(rows, 1000) == 0
    assert L.emu_weights_mfma_major(ctx.h, _lib.Q8_0, src.ptr, raw.size, rows, cols, dst.ptr) == _lib.EMU_E_UNSUPPORTED
    assert L.emu_weights_mfma_major(ctx.h, Q6, src.ptr, raw.size - 210, rows, cols, dst.ptr) == _lib.EMU_E_SHAPE
    assert L.emu_weights_mfma_major(ctx.h, Q6, src.ptr, raw.size, rows, 1000, dst.ptr) == _lib.EMU_E_SHORT
    assert L.emu_weights_mfma_major(ctx.h, Q6, src.ptr, raw.size, rows, cols, src.ptr) == _lib.EMU_E_ARG
    x, y = ctx.upload(np.zeros(8 * cols, np.float32)), ctx.alloc(8 * rows * 4)
    ctx.check(L.emu_weights_mfma_major(ctx.h, Q6, src.ptr, raw.size, rows, cols, dst.ptr), "mfma_major")
    # the flag is for 2..8 tokens on the matrix-core widths, with the padded length
    assert L.emu_qmatvec(ctx.h, Q6, dst.ptr, n, rows, cols, x.ptr, cols, 1, y.ptr,
                         _lib.EMU_MV_MFMA_MAJOR) == _lib.EMU_E_UNSUPPORTED
    assert L.emu_qmatvec(ctx.h, Q6, dst.ptr, n - 1, rows, cols, x.ptr, 2 * cols, 2, y.ptr,
                         _lib.EMU_MV_MFMA_MAJOR) == _lib.EMU_E_SHAPE
    assert L.emu_qmatvec(ctx.h, Q6, dst.ptr, n, rows, cols, x.ptr, 2 * cols, 2, y.ptr,
                         _lib.EMU_MV_MFMA_MAJOR | _lib.EMU_MV_LANE_MAJOR) == _lib.EMU_E_ARG


@pytest.mark.parametrize("rows,cols,n_tok", [(33, 4096, 2), (4096, 4096, 8), (37, 12288, 5), (6144, 4096, 3),
                                             (77, 2816, 8), (100, 2048, 7)])
def test_mfma_major_matvec_equals_gguf_order_bit_for_bit(ctx, rows, cols, n_tok):
    """Same codes in the same operand registers: the operand-order copy gives
    the GGUF-order matrix-core kernel's bits, plain, accumulated, normalised
    and SwiGLU."""
    raw = weights(rows, cols, 5 * rows + cols + n_tok)
    rng = np.random.default_rng(rows + 2 * n_tok)
    x = rng.normal(size=(n_tok, cols)).astype(np.float32)
    base = rng.normal(size=(n_tok, rows)).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    L = ctx.lib
    n = L.emu_weights_mfma_major_bytes(rows, cols)
    w = ctx.upload(raw)
    mm = ctx.alloc(n)
    ctx.check(L.emu_weights_mfma_major(ctx.h, Q6, w.ptr, raw.size, rows, cols, mm.ptr), "mfma_major")
    bx, bg = ctx.upload(x), ctx.upload(gain)

    def run(wp, wlen, flags, acc):
        y = ctx.upload(base.copy()) if acc else ctx.alloc(n_tok * rows * 4)
        ctx.check(L.emu_qmatvec(ctx.h, Q6, wp, wlen, rows, cols, bx.ptr, n_tok * cols, n_tok, y.ptr,
                                flags | (_lib.EMU_MV_ACCUMULATE if acc else 0)), "qmatvec")
        return y.read(np.uint32)

    for acc in (False, True):
        assert np.array_equal(run(w.ptr, raw.size, 0, acc), run(mm.ptr, n, _lib.EMU_MV_MFMA_MAJOR, acc))

    def run_fused(wp, up, flags):
        y = ctx.alloc(n_tok * rows * 4)
        ctx.check(L.emu_qmatvec_fused(ctx.h, Q6, wp, up, rows, cols, bx.ptr, n_tok, bg.ptr, 1e-6, y.ptr, flags),
                  "fused")
        return y.read(np.uint32)

    assert np.array_equal(run_fused(w.ptr, None, 0), run_fused(mm.ptr, None, _lib.EMU_MV_MFMA_MAJOR))
    assert np.array_equal(run_fused(w.ptr, w.ptr, 0), run_fused(mm.ptr, mm.ptr, _lib.EMU_MV_MFMA_MAJOR))
