"""The CPU twin of the weight synthesis (oracle/synth.c), checked on its own.

Its logarithm, cosine and square root are compared with libm, its draws with
the moments of N(0, 0.02), and its quantized blocks with the draws they
encode (each weight within half a quantization step of its draw).  That the
device synthesis writes the same bytes is a GPU test (test_gpu_synth.py).
"""
import math

import numpy as np
import pytest

import oracle


def test_log_cos_sqrt_agree_with_libm():
    lib = oracle.load()
    rng = np.random.default_rng(0)
    ks = [1, 2, 3, 1 << 23, (1 << 24) - 1, 1 << 24] + [int(v) for v in rng.integers(1, 1 << 24, 2000)]
    for k in ks:
        assert abs(lib.or_synth_ln_int(k) - math.log(k)) <= 4e-16 * max(1.0, math.log(k)), k
    assert lib.or_synth_ln_int(1 << 24) - 24 * 0.6931471805599453 == 0.0  # u1 = 1 gives r = 0 exactly
    js = [0, 1, 1 << 21, (1 << 21) + 1, 1 << 22, 1 << 23, 3 << 22, (1 << 24) - 1] + \
         [int(v) for v in rng.integers(0, 1 << 24, 2000)]
    for j in js:
        assert abs(lib.or_synth_cos_turn(j) - math.cos(2 * math.pi * j / (1 << 24))) <= 2e-15, j
    for y in [0.0, 1e-7, 1.0, 2.0, 33.3] + [float(v) for v in rng.uniform(1e-8, 34.0, 2000)]:
        assert abs(lib.or_synth_sqrt(y) - math.sqrt(y)) <= 4e-16 * math.sqrt(y), y


def test_draws_have_the_moments_of_n_0_002():
    x = oracle.synth_f32(4_000_000, 11, 5).astype(np.float64)
    assert abs(x.mean()) < 3 * 0.02 / math.sqrt(x.size) * 2
    assert abs(x.std() / 0.02 - 1.0) < 2e-3
    kurt = np.mean((x / x.std()) ** 4)
    assert abs(kurt - 3.0) < 0.02
    assert np.max(np.abs(x)) < 0.02 * 6.0  # r <= sqrt(-2 ln 2^-24) = 5.77
    # the same key gives the same draw; another stream or seed another one
    assert np.array_equal(oracle.synth_f32(1000, 11, 5), x[:1000].astype(np.float32))
    assert not np.array_equal(oracle.synth_f32(1000, 11, 6), x[:1000].astype(np.float32))
    assert not np.array_equal(oracle.synth_f32(1000, 12, 5), x[:1000].astype(np.float32))


@pytest.mark.parametrize("dtype,sub", [(oracle.OR_Q6_K, 16), (oracle.OR_Q8_0, 32), (oracle.OR_Q5_K, 32),
                                       (oracle.OR_Q2_K, 16)], ids=["q6k", "q8_0", "q5k", "q2k"])
def test_blocks_encode_their_draws(dtype, sub):
    be, bb = oracle.BLOCK[dtype]
    nblk = 64
    raw = oracle.synth_blocks(dtype, nblk * bb, 21, 9)
    got = oracle.decode(dtype, raw).astype(np.float64).reshape(-1, sub)
    want = oracle.synth_f32(nblk * be, 21, 9).astype(np.float64).reshape(-1, sub)
    levels = {oracle.OR_Q6_K: 31.0, oracle.OR_Q8_0: 127.0, oracle.OR_Q5_K: 31.0, oracle.OR_Q2_K: 3.0}[dtype]
    span = (np.max(np.abs(want), axis=1) if dtype in (oracle.OR_Q6_K, oracle.OR_Q8_0)
            else np.max(want, axis=1) - np.minimum(np.min(want, axis=1), 0.0))
    # half a code step of the sub-block's own scale, plus the scale's own
    # quantization (its int or 6/4-bit code and the f16 super-scale)
    step = span / levels
    err = np.max(np.abs(got - want), axis=1)
    assert np.all(err <= 0.5 * step * 1.6 + 1e-9), float(np.max(err / step))
