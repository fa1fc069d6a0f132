"""emu_attend_cached_noalloc (no reference counterpart: the entry point for
callers that cannot allocate device memory) against emu_attend_cached, bit
for bit, on two calls in a row with the second smaller, and its size limit."""
import numpy as np
import pytest

from emufpga_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH_SCORES = 1 << 20


def run_both(ctx, heads, kvh, hd, positions, kv_f16, seed):
    rng = np.random.default_rng(seed)
    q = rng.normal(size=heads * hd).astype(np.float32)
    dt = np.float16 if kv_f16 else np.float32
    keys = rng.normal(size=(positions, kvh * hd)).astype(dt)
    values = rng.normal(size=(positions, kvh * hd)).astype(dt)
    bq, bk, bv = ctx.upload(q), ctx.upload(keys), ctx.upload(values)
    outs = []
    for fn in (ctx.lib.emu_attend_cached, ctx.lib.emu_attend_cached_noalloc):
        bo = ctx.alloc(heads * hd * 4)
        ctx.check(fn(ctx.h, bq.ptr, bk.ptr, bv.ptr, kv_f16, positions, heads, kvh, hd,
                     float(1.0 / np.sqrt(hd)), bo.ptr), fn.__name__)
        outs.append(bo.read(np.uint32))
    return outs


def test_noalloc_attend_equals_the_allocating_entry_point(ctx):
    # two calls in a row on the shared scratch, the second with fewer scores
    a, b = run_both(ctx, 32, 8, 128, 1500, 1, 1)
    assert np.array_equal(a, b)
    a, b = run_both(ctx, 8, 2, 64, 37, 0, 2)
    assert np.array_equal(a, b)


def test_noalloc_attend_refuses_more_scores_than_its_scratch(ctx):
    heads, kvh, hd = 64, 8, 64
    positions = SCRATCH_SCORES // heads + 1
    q = ctx.upload(np.zeros(heads * hd, np.float32))
    kv = ctx.upload(np.zeros(positions * kvh * hd, np.float16))
    out = ctx.alloc(heads * hd * 4)
    st = ctx.lib.emu_attend_cached_noalloc(ctx.h, q.ptr, kv.ptr, kv.ptr, 1, positions, heads, kvh, hd, 0.125,
                                           out.ptr)
    assert st == _lib.EMU_E_CONFIG
    # the largest size it takes still runs
    st = ctx.lib.emu_attend_cached_noalloc(ctx.h, q.ptr, kv.ptr, kv.ptr, 1, positions - 1, heads, kvh, hd, 0.125,
                                           out.ptr)
    assert st == _lib.EMU_OK
    ctx.sync()
