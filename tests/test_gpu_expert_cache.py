"""Experts behind the HBM expert cache on the GPU: the selected-expert FFN
through the cache gives the resident experts' bits exactly, call after call,
while experts stream through, get admitted and get evicted; the cache's
counters agree with its policy run on the CPU."""
import ctypes as C

import numpy as np
import pytest

from emufpga_amd import _lib
from emufpga_amd.expert_cache import ExpertCache, policy_trace
from emufpga_amd.gguf import row_bytes
from tests.test_gpu_moe import make_experts, route

pytestmark = pytest.mark.gpu
SLOTS = 20


def popular_logits(rng, rank, n_tok, s):
    """Router logits whose top choices follow Zipf(s) over a fixed expert
    ranking (the layer's popular experts stay popular from call to call)."""
    gumbel = -np.log(-np.log(rng.uniform(1e-9, 1.0, size=(n_tok, rank.size))))
    return (-s * np.log(rank)[None, :] + gumbel).astype(np.float32)


@pytest.mark.parametrize("enc_in,enc_down,fused,act,layer_aware",
                         [(_lib.Q6_K, _lib.Q6_K, False, _lib.EMU_ACT_SILU, False),
                          (_lib.Q5_K, _lib.Q8_0, True, _lib.EMU_ACT_GELU_TANH, True)],
                         ids=["granite-form-lru", "gemma-form-layer-aware"])
def test_cached_experts_equal_resident_experts_bit_for_bit(ctx, enc_in, enc_down, fused, act, layer_aware):
    rng = np.random.default_rng(5 + enc_in)
    E, W, FF, K, T, layers = 16, 512, 256 if enc_down != _lib.Q8_0 else 128, 4, 4, 2
    rb_in, rb_ff = row_bytes(enc_in, W), row_bytes(enc_down, FF)
    expert_bytes = 2 * FF * rb_in + W * rb_ff
    # per layer: resident expert-major tensors and the cache's host copies (gate rows, up rows, down rows)
    per_layer, ranks = [], [rng.permutation(E) + 1 for _ in range(layers)]
    cache = ExpertCache(ctx, layers, E, expert_bytes, n_slots=SLOTS, n_transient=T * K, layer_aware=layer_aware)
    for layer in range(layers):
        gate, up, down = make_experts(rng, enc_in, enc_down, E, W, FF, fused)
        g = gate.view(np.uint8).reshape(E, (1 if up is not None else 2) * FF * rb_in)
        u = up.view(np.uint8).reshape(E, FF * rb_in) if up is not None else np.zeros((E, 0), np.uint8)
        host = np.concatenate([g, u, down.view(np.uint8).reshape(E, W * rb_ff)], axis=1)
        assert host.shape == (E, expert_bytes)
        cache.set_layer(layer, host)
        scale = rng.uniform(0.5, 2.0, E).astype(np.float32) if fused else None
        bufs = [ctx.upload(a) if a is not None else None for a in (gate, up, down)]
        bs = ctx.upload(scale) if scale is not None else None
        desc = _lib.MoeDesc(enc_in, enc_down, bufs[0].addr, bufs[1].addr if bufs[1] else None, bufs[2].addr,
                            bs.addr if bs else None, E, W, FF, K, act)
        per_layer.append((desc, bufs, bs))
    ws_bytes = ctx.lib.emu_moe_workspace_bytes(T, K, W, FF)
    ws = ctx.alloc(ws_bytes)
    calls, trace_layers, trace_experts = [], [], []
    for call in range(12):
        layer = call % layers
        desc = per_layer[layer][0]
        x = rng.normal(size=(T, W)).astype(np.float32)
        ids, wts = route(popular_logits(rng, ranks[layer], T, 1.2), K)
        bx, bi, bw = ctx.upload(x), ctx.upload(ids.astype(np.int32)), ctx.upload(wts)
        want, got = ctx.alloc(T * W * 4), ctx.alloc(T * W * 4)
        ctx.check(ctx.lib.emu_moe_ffn(ctx.h, C.byref(desc), bx.ptr, T, bi.ptr, bw.ptr, ws.ptr, ws_bytes, want.ptr),
                  "moe_ffn")
        cache.moe_ffn(desc, layer, bx.ptr, T, ids, bi.ptr, bw.ptr, ws.ptr, ws_bytes, got.ptr)
        assert np.array_equal(got.read(np.uint32), want.read(np.uint32)), call
        for e in sorted(set(ids.reshape(-1).tolist())):
            calls.append(call)
            trace_layers.append(layer)
            trace_experts.append(e)
    outcome, slot = policy_trace(SLOTS, layer_aware, calls, trace_layers, trace_experts)
    st = cache.stats()
    assert st["hits"] == int(np.sum(outcome == 0))
    assert st["loads"] == int(np.sum(outcome == 1))
    assert st["streamed"] == int(np.sum(outcome == 2))
    assert st["misses"] == st["loads"] + st["streamed"] and st["loads"] > 0 and st["hits"] > 0
    assert st["bytes_uploaded"] == (st["loads"] + st["streamed"]) * expert_bytes
    assert st["evictions"] > 0 and st["resident"] == SLOTS
    cache.close()


def test_cache_refuses_mismatched_shapes_and_too_many_streams(ctx):
    rng = np.random.default_rng(9)
    E, W, FF, K, T = 8, 256, 256, 8, 2
    rb = row_bytes(_lib.Q6_K, W)
    expert_bytes = 3 * FF * rb
    cache = ExpertCache(ctx, 1, E, expert_bytes, n_slots=2, n_transient=4)
    cache.set_layer(0, rng.integers(0, 256, size=(E, expert_bytes), dtype=np.uint8))
    desc = _lib.MoeDesc(_lib.Q6_K, _lib.Q6_K, None, None, None, None, E, W, FF, K, _lib.EMU_ACT_SILU)
    x = ctx.upload(np.zeros((T, W), np.float32))
    ids = np.stack([np.arange(8), np.arange(8)]).astype(np.int32)  # 8 distinct experts, 4 transient slots
    bi, bw = ctx.upload(ids), ctx.upload(np.full((T, K), 1 / 8, np.float32))
    ws_bytes = ctx.lib.emu_moe_workspace_bytes(T, K, W, FF)
    ws, out = ctx.alloc(ws_bytes), ctx.alloc(T * W * 4)
    st = ctx.lib.emu_moe_ffn_cached(ctx.h, C.byref(desc), cache.h, 0, x.ptr, T, ids.ctypes.data_as(C.c_void_p),
                                    bi.ptr, bw.ptr, ws.ptr, ws_bytes, out.ptr)
    assert st == _lib.EMU_E_CONFIG
    bad = _lib.MoeDesc(_lib.Q6_K, _lib.Q6_K, None, None, None, None, E, W, 2 * FF, K, _lib.EMU_ACT_SILU)
    st = ctx.lib.emu_moe_ffn_cached(ctx.h, C.byref(bad), cache.h, 0, x.ptr, T, ids.ctypes.data_as(C.c_void_p),
                                    bi.ptr, bw.ptr, ws.ptr, ws_bytes, out.ptr)
    assert st == _lib.EMU_E_SHAPE
    cache.close()


# ---- the cache inside the decode step (device policy) ----------------------

def _moe_model(cfg_kind):
    from emufpga_amd.serve import DenseConfig
    if cfg_kind == "granite":
        return DenseConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=0, vocab=300, layers=3,
                           rope_theta=1.5e6, eps=1e-6, style=_lib.EMU_STYLE_GRANITE, encoding=_lib.Q6_K, tied=True,
                           qk_norm=False, n_experts=12, experts_used=3, expert_ff=256, expert_encoding=_lib.Q6_K,
                           embed_scale=12.0, residual_scale=0.22, logit_div=6.0, score_mul=0.015625)
    return DenseConfig(512, 4, 2, 256, 0, 300, 3, 1e4, 1e-6, _lib.EMU_STYLE_GRANITE, _lib.Q6_K, True, True,
                       n_experts=16, experts_used=4, expert_ff=256, expert_encoding=_lib.Q5_K, embed_scale=22.6,
                       score_mul=1.0 / 16, rope_neox=True, gemma=True, expert_down_encoding=_lib.Q8_0, shared_ff=256,
                       window=8, global_every=2, rope_theta_global=1e6, logit_softcap=30.0)


def _expert_bytes(cfg):
    down_enc = cfg.expert_down_encoding if cfg.gemma else cfg.expert_encoding
    return 2 * cfg.expert_ff * row_bytes(cfg.expert_encoding, cfg.hidden) + cfg.hidden * row_bytes(down_enc,
                                                                                                 cfg.expert_ff)


def _replay(routes_per_step, n_slots, layer_aware):
    """The host policy over the same calls: per step and layer, the distinct
    routed experts ascending."""
    calls, layers, experts = [], [], []
    call = 0
    for ids in routes_per_step:
        for layer in range(ids.shape[0]):
            for e in sorted(set(ids[layer].reshape(-1).tolist())):
                calls.append(call)
                layers.append(layer)
                experts.append(e)
            call += 1
    out, _ = policy_trace(n_slots, layer_aware, calls, layers, experts)
    return {"hits": int(np.sum(out == 0)), "loads": int(np.sum(out == 1)), "streamed": int(np.sum(out == 2)),
            "misses": int(np.sum(out != 0)), "calls": len(out)}


@pytest.mark.parametrize("kind,n_clients,n_slots,layer_aware",
                         [("granite", 2, 8, False), ("granite", 3, 0, False), ("gemma", 2, 10, True)],
                         ids=["granite-8-slots", "granite-no-slots", "gemma-10-slots-layer-aware"])
def test_decode_step_through_the_device_cache(ctx, kind, n_clients, n_slots, layer_aware):
    """A session whose experts come through the cache (hits from HBM slots,
    admissions copied into their slots first, other misses read from pinned
    host memory by the expert kernels), captured and replayed as a graph: logits bit for bit those of
    the resident experts at every step, and the device's counters equal to
    the host policy replayed over the traced routes.  Routing is Zipf(1.5)
    (the same draws in both sessions), so popular experts come back and hit."""
    from emufpga_amd.serve import Model, Session
    cfg = _moe_model(kind)
    model = Model(ctx, cfg)
    model.synth(404)
    rng = np.random.default_rng(9)
    steps = 24
    toks = rng.integers(0, cfg.vocab, size=(steps, n_clients)).astype(np.uint32)
    plain = Session(model, n_clients, 64)
    plain.route_zipf(1.5, 3)
    want = [plain.decode_step(toks[i], want_logits=True) for i in range(steps)]
    plain.close()
    cache = ExpertCache(ctx, cfg.layers, cfg.n_experts, _expert_bytes(cfg), n_slots=n_slots, n_transient=1,
                        layer_aware=layer_aware)
    cache.load_model(model)
    sess = Session(model, n_clients, 64)
    sess.route_zipf(1.5, 3)
    sess.route_trace(steps)
    sess.attach_cache(cache)
    for i in range(steps):
        nxt, lg = sess.decode_step(toks[i], want_logits=True)
        assert np.array_equal(nxt, want[i][0]), i
        assert np.array_equal(lg.view(np.uint32), want[i][1].view(np.uint32)), i
    got = cache.stats()
    rep = _replay([sess.read_routes(i)[0] for i in range(steps)], n_slots, layer_aware)
    for k in ("hits", "loads", "streamed", "misses"):
        assert got[k] == rep[k], (k, got, rep)
    eb = _expert_bytes(cfg)
    assert got["bytes_uploaded"] == rep["loads"] * eb and got["bytes_streamed"] == rep["streamed"] * eb
    assert got["resident"] == min(n_slots, rep["loads"])
    if n_slots:
        assert rep["hits"] > 0 and rep["loads"] > 0
    sess.close()
    cache.close()
    model.close()
