"""Selected-expert FFN (moe::run and the Gemma expert form) on the GPU,
through the C ABI, against the oracle.

Bar: max |gpu - ref| <= 1e-4 * max |ref| over the layer output (two
quantized matvecs of the reference's rounding bar, an activation and the
weighted expert sum, propagated).  Expert order of the weighted sum is the
reference's (ascending id); routing ids are identical.  Inputs of up to 4096
columns run on the int8 matrix cores with the activations carried as limbs
exact to 2^-20 of each 256-column span's largest |x| (well inside the bar);
wider ones run the vector kernels.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from emufpga_amd import _lib
from tests import npref

pytestmark = pytest.mark.gpu


def zipf_logits(rng, n_tok, n_experts, s):
    """Router logits whose top choices follow Zipf(s) over a random expert ranking."""
    rank = rng.permutation(n_experts) + 1
    gumbel = -np.log(-np.log(rng.uniform(1e-9, 1.0, size=(n_tok, n_experts))))
    return (-s * np.log(rank)[None, :] + gumbel).astype(np.float32)


def make_experts(rng, enc_in, enc_down, n_experts, width, ff, fused):
    n_in = n_experts * (2 if fused else 1) * ff * width // npref.BLOCK_ELEMS[enc_in]
    gate = npref.random_blocks(enc_in, n_in, rng)
    up = None if fused else npref.random_blocks(enc_in, n_in, rng)
    down = npref.random_blocks(enc_down, n_experts * width * ff // npref.BLOCK_ELEMS[enc_down], rng)
    return gate, up, down


def run_gpu(ctx, enc_in, enc_down, gate, up, down, scale, n_experts, width, ff, k, act, x, ids, wts,
            on_device_ids=None, flags=0):
    n_tok = x.shape[0]
    bufs = [ctx.upload(a) if a is not None else None for a in (gate, up, down)]
    bs = ctx.upload(scale) if scale is not None else None
    desc = _lib.MoeDesc(enc_in, enc_down, bufs[0].addr, bufs[1].addr if bufs[1] else None, bufs[2].addr,
                        bs.addr if bs else None, n_experts, width, ff, k, act, flags)
    bx = ctx.upload(x)
    if on_device_ids is None:
        bi, bw = ctx.upload(np.asarray(ids, np.int32)), ctx.upload(np.asarray(wts, np.float32))
    else:
        bi, bw = on_device_ids
    ws_bytes = ctx.lib.emu_moe_workspace_bytes(n_tok, k, width, ff)
    ws = ctx.alloc(ws_bytes)
    out = ctx.alloc(n_tok * width * 4)
    ctx.check(ctx.lib.emu_moe_ffn(ctx.h, C.byref(desc), bx.ptr, n_tok, bi.ptr, bw.ptr, ws.ptr, ws_bytes, out.ptr),
              "moe_ffn")
    return out.read(np.float32).reshape(n_tok, width)


def route(logits, k):
    ids, wts = zip(*[oracle.route(logits[t], k) for t in range(logits.shape[0])])
    return np.array(ids, np.int64), np.array(wts, np.float32)


SHAPES = [
    # (name, enc_in, enc_down, experts, width, ff, k, tokens, fused, act, zipf s)
    ("granite", _lib.Q6_K, _lib.Q6_K, 32, 1024, 512, 8, 4, False, _lib.EMU_ACT_SILU, 1.1),
    ("olmoe", _lib.Q2_K, _lib.Q2_K, 64, 2048, 1024, 8, 8, False, _lib.EMU_ACT_SILU, 1.0),
    ("gemma", _lib.Q5_K, _lib.Q8_0, 16, 2816, 704, 8, 8, True, _lib.EMU_ACT_GELU_TANH, 1.2),
    # rows shorter than 16 units: 4 rows per wavefront in both kernels
    ("short-rows", _lib.Q6_K, _lib.Q8_0, 8, 256, 96, 2, 3, True, _lib.EMU_ACT_SILU, 1.0),
    # inputs wider than 4096 columns take the direct (vector) kernels
    ("wide-rows", _lib.Q6_K, _lib.Q6_K, 4, 4352, 256, 2, 2, False, _lib.EMU_ACT_SILU, 1.0),
    # one token: every expert holds a single position of the matrix-core operands
    ("one-token-olmoe", _lib.Q2_K, _lib.Q2_K, 64, 2048, 1024, 8, 1, False, _lib.EMU_ACT_SILU, 1.0),
    # a partial last span of Q8_0 down input (ff = 704: 2.75 spans) and 128 experts
    ("gemma-b1", _lib.Q5_K, _lib.Q8_0, 128, 2816, 704, 8, 1, True, _lib.EMU_ACT_GELU_TANH, 1.2),
    # the span loop's forms: Q6_K rows of 5 and 3 spans (the register loop:
    # 210-byte spans start 2-byte aligned); Q2_K and Q5_K down rows of 6 and
    # 5 spans (rows staged straight into LDS); Q8_0 down rows whose last span
    # holds an odd number of 34-byte blocks (ff = 736: 23 blocks, so rows
    # and that span end 2 bytes past a dword: the register loop again)
    ("q6k-loop", _lib.Q6_K, _lib.Q6_K, 16, 1280, 768, 4, 5, False, _lib.EMU_ACT_SILU, 1.0),
    ("q2k-direct-down", _lib.Q2_K, _lib.Q2_K, 24, 2048, 1536, 4, 6, False, _lib.EMU_ACT_SILU, 1.0),
    ("q5k-direct-down", _lib.Q5_K, _lib.Q5_K, 12, 1024, 1280, 4, 4, True, _lib.EMU_ACT_GELU_TANH, 1.0),
    ("q8-unaligned-down", _lib.Q5_K, _lib.Q8_0, 12, 1024, 736, 4, 4, True, _lib.EMU_ACT_SILU, 1.0),
]


@pytest.mark.parametrize("f32", [False, True], ids=["limbs", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_moe_ffn_matches_oracle(ctx, shape, f32):
    """Both activation forms: the int8-limb matrix-core form (the default
    for inputs of up to 4096 columns) and, with EMU_MOE_F32_ACT, the f32
    vector form, which every shape takes."""
    name, enc_in, enc_down, E, W, FF, K, T, fused, act, s = shape
    rng = np.random.default_rng(sum(map(ord, name)))
    gate, up, down = make_experts(rng, enc_in, enc_down, E, W, FF, fused)
    scale = rng.uniform(0.5, 2.0, E).astype(np.float32) if fused else None
    x = rng.normal(size=(T, W)).astype(np.float32)
    ids, wts = route(zipf_logits(rng, T, E, s), K)
    got = run_gpu(ctx, enc_in, enc_down, gate, up, down, scale, E, W, FF, K, act, x, ids, wts,
                  flags=_lib.EMU_MOE_F32_ACT if f32 else 0)
    ref = oracle.moe_ffn(enc_in, enc_down, gate, up, down, scale, E, W, FF, K, act, x, ids, wts)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_more_than_256_experts(ctx):
    """A layer of 300 experts with routes to ids past 255: the matrix-core
    form finds experts in a 256-bit mask, so such layers take the vector
    form, and every route is computed (ids 256..299 included)."""
    E, W, FF, K, T = 300, 256, 256, 4, 3
    rng = np.random.default_rng(80)
    gate, up, down = make_experts(rng, _lib.Q6_K, _lib.Q6_K, E, W, FF, False)
    x = rng.normal(size=(T, W)).astype(np.float32)
    ids = np.array([[299, 256, 3, 17], [255, 280, 0, 299], [100, 257, 258, 1]])
    wts = rng.uniform(0.1, 1.0, (T, K)).astype(np.float32)
    got = run_gpu(ctx, _lib.Q6_K, _lib.Q6_K, gate, up, down, None, E, W, FF, K, _lib.EMU_ACT_SILU, x, ids, wts)
    ref = oracle.moe_ffn(_lib.Q6_K, _lib.Q6_K, gate, up, down, None, E, W, FF, K, oracle.OR_ACT_SILU, x, ids, wts)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_route_then_ffn_on_device(ctx):
    """emu_route feeding emu_moe_ffn on the device equals oracle route + ffn."""
    E, W, FF, K, T = 32, 1024, 512, 8, 6
    rng = np.random.default_rng(77)
    gate, up, down = make_experts(rng, _lib.Q6_K, _lib.Q6_K, E, W, FF, False)
    x = rng.normal(size=(T, W)).astype(np.float32)
    logits = zipf_logits(rng, T, E, 1.1)
    bl = ctx.upload(logits)
    bi, bw = ctx.alloc(T * K * 4), ctx.alloc(T * K * 4)
    ctx.check(ctx.lib.emu_route(ctx.h, bl.ptr, T, E, K, bi.ptr, bw.ptr), "route")
    ids_ref, wts_ref = route(logits, K)
    assert np.array_equal(bi.read(np.int32).reshape(T, K), ids_ref)
    got = run_gpu(ctx, _lib.Q6_K, _lib.Q6_K, gate, up, down, None, E, W, FF, K, _lib.EMU_ACT_SILU, x, None, None,
                  on_device_ids=(bi, bw))
    ref = oracle.moe_ffn(_lib.Q6_K, _lib.Q6_K, gate, up, down, None, E, W, FF, K, oracle.OR_ACT_SILU, x,
                         ids_ref, wts_ref)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_single_token_single_expert_is_plain_ffn(ctx):
    """k = 1, weight 1: the layer output is one expert's SwiGLU FFN."""
    E, W, FF = 4, 1024, 512
    rng = np.random.default_rng(78)
    gate, up, down = make_experts(rng, _lib.Q6_K, _lib.Q6_K, E, W, FF, False)
    x = rng.normal(size=(1, W)).astype(np.float32)
    ids, wts = np.array([[2]]), np.ones((1, 1), np.float32)
    got = run_gpu(ctx, _lib.Q6_K, _lib.Q6_K, gate, up, down, None, E, W, FF, 1, _lib.EMU_ACT_SILU, x, ids, wts)
    ref = oracle.moe_ffn(_lib.Q6_K, _lib.Q6_K, gate, up, down, None, E, W, FF, 1, oracle.OR_ACT_SILU, x, ids, wts)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_argument_errors(ctx):
    E, W, FF, K = 4, 256, 256, 2
    rng = np.random.default_rng(79)
    gate, up, down = make_experts(rng, _lib.Q6_K, _lib.Q6_K, E, W, FF, False)
    bg, bu, bd = ctx.upload(gate), ctx.upload(up), ctx.upload(down)
    desc = _lib.MoeDesc(_lib.Q6_K, _lib.Q6_K, bg.addr, bu.addr, bd.addr, None, E, W, FF, K, _lib.EMU_ACT_SILU)
    bx, bi, bw = ctx.alloc(9 * W * 4), ctx.alloc(9 * K * 4), ctx.alloc(9 * K * 4)
    out = ctx.alloc(9 * W * 4)
    need = ctx.lib.emu_moe_workspace_bytes(9, K, W, FF)
    ws = ctx.alloc(need)
    lib = ctx.lib
    # more than 8 tokens per call
    assert lib.emu_moe_ffn(ctx.h, C.byref(desc), bx.ptr, 9, bi.ptr, bw.ptr, ws.ptr, need, out.ptr) == _lib.EMU_E_ARG
    # workspace too small
    assert lib.emu_moe_ffn(ctx.h, C.byref(desc), bx.ptr, 2, bi.ptr, bw.ptr, ws.ptr, 16, out.ptr) == _lib.EMU_E_ARG
    # width not whole blocks
    bad = _lib.MoeDesc(_lib.Q6_K, _lib.Q6_K, bg.addr, bu.addr, bd.addr, None, E, 200, FF, K, _lib.EMU_ACT_SILU)
    assert lib.emu_moe_ffn(ctx.h, C.byref(bad), bx.ptr, 2, bi.ptr, bw.ptr, ws.ptr, need, out.ptr) == _lib.EMU_E_SHORT
