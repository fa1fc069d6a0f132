"""Mixture-of-experts decode step (spm-granite-moe/src/model.rs:330-411) on the
GPU against the oracle's or_moe_model_step, in its Granite, OLMoE and
Gemma-4 forms.

Same bars as the dense decoder: logits within ||gpu - ref||_inf <= 1e-3 *
||ref||_inf per step and greedy tokens identical (ties to the lowest index,
math.rs:35-40).  The step: embeddings x 12, RMSNorm, q|k|v, adjacent-pair RoPE
(theta 1.5e6), scores x 1/64, o projection added as r + 0.22 v, RMSNorm, f32
router, softmax top-k, the routed SwiGLU experts added as r + 0.22 v, tied
output / 6.
"""
import numpy as np
import pytest

import oracle
from emufpga_amd import _lib
from emufpga_amd.gguf import row_bytes
from emufpga_amd.serve import GEMMA4_MOE, GRANITE_MOE_Q6K, OLMOE_1B_7B, DenseConfig, Model, Session

pytestmark = pytest.mark.gpu


def small_granite(expert_encoding=_lib.Q6_K, experts=8, used=2):
    return DenseConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=0, vocab=300, layers=2,
                       rope_theta=1.5e6, eps=1e-6, style=_lib.EMU_STYLE_GRANITE, encoding=_lib.Q6_K, tied=True,
                       qk_norm=False, n_experts=experts, experts_used=used, expert_ff=256,
                       expert_encoding=expert_encoding, embed_scale=12.0, residual_scale=0.22, logit_div=6.0,
                       score_mul=0.015625)


def oracle_for(model: Model, context: int, kv_f16: bool, n_clients: int) -> oracle.MoeModelOracle:
    c = model.cfg
    cfg = oracle.MoeModelCfg(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                             vocab=c.vocab, layers=c.layers, context=context, n_experts=c.n_experts,
                             experts_used=c.experts_used, expert_ff=c.expert_ff, rope_theta=c.rope_theta, eps=c.eps,
                             embed_scale=c.embed_scale, residual_scale=c.residual_scale, logit_div=c.logit_div,
                             score_mul=c.score_mul, dtype=c.encoding, expert_dtype=c.expert_encoding,
                             kv_f16=int(kv_f16), qk_norm=int(c.qk_norm), rope_neox=int(c.rope_neox),
                             untied=int(not c.tied), gemma=int(c.gemma), expert_down_dtype=c.expert_down_encoding,
                             shared_ff=c.shared_ff, window=c.window, global_every=c.global_every,
                             rope_theta_global=c.rope_theta_global, softcap=c.logit_softcap)
    w = model.host_weights()
    assert w["layers"].size == c.layers * oracle.moe_layer_bytes(cfg)
    return oracle.MoeModelOracle(cfg, w, n_clients)


def rel_inf(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("expert_encoding,n_clients,f32", [(_lib.Q6_K, 1, False), (_lib.Q6_K, 3, False),
                                                            (_lib.Q2_K, 2, False), (_lib.Q6_K, 3, True),
                                                            (_lib.Q2_K, 2, True)],
                         ids=["q6k-1", "q6k-3", "q2k-2", "q6k-3-f32", "q2k-2-f32"])
def test_moe_decode_steps_match_oracle(ctx, expert_encoding, n_clients, f32):
    """f32: EMU_SESSION_F32_ACT (projections and experts on f32 activations)."""
    model = Model(ctx, small_granite(expert_encoding))
    model.synth(2024 + expert_encoding)
    context = 80  # two attention chunks: the split merge
    sess = Session(model, n_clients, context, kv_f16=True)
    sess.set_options(f32_act=f32)
    ref = oracle_for(model, context, True, n_clients)
    rng = np.random.default_rng(expert_encoding + n_clients)
    worst = 0.0
    for step in range(70):
        toks = rng.integers(0, model.cfg.vocab, size=n_clients).astype(np.uint32)
        nxt, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        for c in range(n_clients):
            worst = max(worst, rel_inf(logits[c], r[c]))
            assert int(nxt[c]) == oracle.argmax(r[c], False), (step, c)
    assert worst <= 1e-3, worst


def test_moe_batched_client_gets_what_it_would_alone(ctx):  # spm-batch/tests/batching.rs:128-145
    model = Model(ctx, small_granite())
    model.synth(77)
    prompts = np.array([[1, 2, 3, 4], [9, 8, 7, 6], [5, 5, 5, 5]], np.uint32)
    together = Session(model, 3, 64).generate(prompts, 16)
    for c in range(3):
        alone = Session(model, 1, 64).generate(prompts[c:c + 1], 16)
        assert np.array_equal(alone[0], together[c])


def test_granite_shape_batched_client_gets_what_it_would_alone(ctx):  # spm-batch/tests/batching.rs:128-145
    """At the Granite width (1024) one client takes the same chained
    matrix-core step as two or four together -- q|k|v, o, the experts and the
    output on the int8 matrix cores, the expert sums joining the residual in
    the next layer's link -- so its logits and tokens are the same bits."""
    model = Model(ctx, DenseConfig(**{**GRANITE_MOE_Q6K.__dict__, "layers": 3}))
    model.synth(31)
    rng = np.random.default_rng(4)
    prompts = rng.integers(0, GRANITE_MOE_Q6K.vocab, size=(4, 6)).astype(np.uint32)
    alone = [Session(model, 1, 64).generate(prompts[c:c + 1], 12)[0] for c in range(4)]
    for n in (2, 4):
        together = Session(model, n, 64).generate(prompts[:n], 12)
        for c in range(n):
            assert np.array_equal(together[c], alone[c]), (n, c)
    toks = prompts[:, 0].copy()
    _, l4 = Session(model, 4, 16).decode_step(toks, want_logits=True)
    for c in range(4):
        _, l1 = Session(model, 1, 16).decode_step(toks[c:c + 1], want_logits=True)
        assert np.array_equal(l1[0].view(np.uint32), l4[c].view(np.uint32)), c


@pytest.mark.parametrize("n_clients", [2, 4])
def test_granite_shape_decodes_and_matches_oracle(ctx, n_clients):
    """The Granite shape itself (24 layers cut to 2 for the oracle's speed):
    width 1024, 32 experts of 512 with 8 routed, 49155-row tied output.
    Several clients take the chained step: q|k|v and o on the matrix cores,
    the attention adding q|k|v's partial sums, the gate kernel o's."""
    cfg = GRANITE_MOE_Q6K
    small = DenseConfig(**{**cfg.__dict__, "layers": 2})
    model = Model(ctx, small)
    model.synth(5150)
    context = 40
    sess = Session(model, n_clients, context, kv_f16=True)
    ref = oracle_for(model, context, True, n_clients)
    rng = np.random.default_rng(9)
    for step in range(6):
        toks = rng.integers(0, cfg.vocab, size=n_clients).astype(np.uint32)
        nxt, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        for c in range(n_clients):
            assert rel_inf(logits[c], r[c]) <= 1e-3, (step, c)
            assert int(nxt[c]) == oracle.argmax(r[c], False), (step, c)


def test_moe_config_rejects_unsupported_forms(ctx):
    with pytest.raises(_lib.EmuError):
        Model(ctx, DenseConfig(**{**small_granite().__dict__, "experts_used": 9, "n_experts": 16}))
    with pytest.raises(_lib.EmuError):  # a sliding window needs the global-layer period
        Model(ctx, DenseConfig(**{**small_gemma().__dict__, "global_every": 0}))
    with pytest.raises(_lib.EmuError):  # the MoE forms are not dense-model options
        Model(ctx, DenseConfig(**{**small_granite().__dict__, "style": _lib.EMU_STYLE_QWEN3, "ffn": 512,
                                  "n_experts": 0, "experts_used": 0, "expert_ff": 0, "rope_neox": True}))


# ---- the OLMoE form -------------------------------------------------------

def small_olmoe():
    return DenseConfig(hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=0, vocab=300, layers=2, rope_theta=1e4,
                       eps=1e-5, style=_lib.EMU_STYLE_GRANITE, encoding=_lib.Q6_K, tied=False, qk_norm=True,
                       n_experts=8, experts_used=3, expert_ff=256, expert_encoding=_lib.Q2_K,
                       score_mul=0.125, rope_neox=True)


def run_against_oracle(ctx, cfg, n_clients, steps, context, seed, gains=None):
    model = Model(ctx, cfg)
    model.synth(seed)
    if gains:
        gains(model)
    sess = Session(model, n_clients, context, kv_f16=True)
    ref = oracle_for(model, context, True, n_clients)
    rng = np.random.default_rng(seed)
    worst = 0.0
    oracle.set_threads(16)
    try:
        for step in range(steps):
            toks = rng.integers(0, cfg.vocab, size=n_clients).astype(np.uint32)
            nxt, logits = sess.decode_step(toks, want_logits=True)
            r = ref.step(toks)
            for c in range(n_clients):
                worst = max(worst, rel_inf(logits[c], r[c]))
                assert int(nxt[c]) == oracle.argmax(r[c], False), (step, c)
    finally:
        oracle.set_threads(1)
    assert worst <= 1e-3, worst
    sess.close()
    model.close()
    return worst


def random_norm_gains(model):
    """Gains away from 1.0, so a gain that is dropped or misplaced shows."""
    c, rng = model.cfg, np.random.default_rng(3)
    kinds = [(_lib.EMU_T_ATTN_NORM, c.layers * c.hidden), (_lib.EMU_T_FFN_NORM, c.layers * c.hidden),
             (_lib.EMU_T_Q_NORM, c.layers * c.head_dim), (_lib.EMU_T_K_NORM, c.layers * c.head_dim),
             (_lib.EMU_T_OUT_NORM, c.hidden)]
    if c.gemma:
        kinds.append((_lib.EMU_T_FFN_NORM2, c.layers * c.hidden))
    for kind, n in kinds:
        model.write_tensor(kind, rng.uniform(0.5, 1.5, n).astype(np.float32))


@pytest.mark.parametrize("n_clients", [1, 3])
def test_olmoe_form_matches_oracle(ctx, n_clients):
    """Half-split RoPE, per-head QK-norm, equal query and KV heads, Q2_K
    experts, an untied output, no Granite constants."""
    run_against_oracle(ctx, small_olmoe(), n_clients, 70, 80, 31 + n_clients, random_norm_gains)


@pytest.mark.parametrize("n_clients", [1, 8])
def test_olmoe_shape_matches_oracle(ctx, n_clients):
    """The OLMoE-1B-7B shape (16 layers cut to 2): width 2048, 16 heads of
    128, 64 Q2_K experts of 1024 with 8 routed, 50304-row untied output;
    eight clients take the chained matrix-core step."""
    cfg = DenseConfig(**{**OLMOE_1B_7B.__dict__, "layers": 2})
    run_against_oracle(ctx, cfg, n_clients, 5, 24, 41 + n_clients, random_norm_gains)


# ---- the Gemma-4 form -----------------------------------------------------

def small_gemma(window=70):
    return DenseConfig(hidden=512, heads=2, kv_heads=1, head_dim=256, ffn=0, vocab=300, layers=2, rope_theta=1e4,
                       eps=1e-6, style=_lib.EMU_STYLE_GRANITE, encoding=_lib.Q6_K, tied=True, qk_norm=True,
                       n_experts=8, experts_used=3, expert_ff=64, expert_encoding=_lib.Q5_K,
                       embed_scale=float(np.float32(np.sqrt(512.0))), score_mul=1.0 / 16, rope_neox=True, gemma=True,
                       expert_down_encoding=_lib.Q8_0, shared_ff=256, window=window, global_every=2,
                       rope_theta_global=1e6, logit_softcap=30.0)


def gemma_layer_scales(model):
    """Random router and down scales written into each layer (the layer
    layout of emu_model_config's gemma form), and random gains."""
    random_norm_gains(model)
    c, rng = model.cfg, np.random.default_rng(4)
    rb = lambda enc, cols: row_bytes(enc, cols)  # noqa: E731
    QW, KW = c.heads * c.head_dim, c.kv_heads * c.head_dim
    off_r = -(-((QW + 2 * KW) * rb(c.encoding, c.hidden) + c.hidden * rb(c.encoding, QW)) // 16) * 16
    off_rs = off_r + 4 * c.n_experts * c.hidden
    off_ds = -(-(off_rs + 4 * c.hidden) // 16) * 16
    for layer in range(c.layers):
        blob = model.read_tensor(_lib.EMU_T_LAYER, layer)
        blob[off_rs:off_rs + 4 * c.hidden] = rng.uniform(0.5, 1.5, c.hidden).astype(np.float32).view(np.uint8)
        blob[off_ds:off_ds + 4 * c.n_experts] = rng.uniform(0.5, 2.0, c.n_experts).astype(np.float32).view(np.uint8)
        model.write_tensor(_lib.EMU_T_LAYER, blob, layer)


@pytest.mark.parametrize("n_clients", [1, 3])
def test_gemma_form_matches_oracle(ctx, n_clients):
    """head_dim 256; the local layer attends to the last 70 positions (its
    first live chunk moves past chunk 0 after position 127), the global one
    to all at its own RoPE base; the shared GeGLU FFN; fused Q5_K gate|up
    experts with Q8_0 downs and per-expert scales; the scaled router input;
    x sqrt(512) embeddings; logits soft-capped at 30."""
    run_against_oracle(ctx, small_gemma(), n_clients, 140, 150, 51 + n_clients, gemma_layer_scales)


def test_gemma_shape_batched_client_gets_what_it_would_alone(ctx):  # spm-batch/tests/batching.rs:128-145
    """The Gemma-4-style shape (3 layers): one client takes the same chained
    matrix-core step as two or four together -- the gate adding o's partial
    sums, the shared GeGLU FFN chained link -> gate|up -> link -> down, its
    partial sums and the expert sum joining the residual in the next layer's
    link (the last layer's finished before the output) -- so its logits and
    tokens are the same bits."""
    model = Model(ctx, DenseConfig(**{**GEMMA4_MOE.__dict__, "layers": 3}))
    model.synth(73)
    gemma_layer_scales(model)
    rng = np.random.default_rng(6)
    prompts = rng.integers(0, GEMMA4_MOE.vocab, size=(4, 5)).astype(np.uint32)
    alone = [Session(model, 1, 32).generate(prompts[c:c + 1], 8)[0] for c in range(4)]
    for n in (2, 4):
        together = Session(model, n, 32).generate(prompts[:n], 8)
        for c in range(n):
            assert np.array_equal(together[c], alone[c]), (n, c)
    toks = prompts[:, 0].copy()
    _, l4 = Session(model, 4, 16).decode_step(toks, want_logits=True)
    for c in range(4):
        _, l1 = Session(model, 1, 16).decode_step(toks[c:c + 1], want_logits=True)
        assert np.array_equal(l1[0].view(np.uint32), l4[c].view(np.uint32)), c


def test_gemma_shape_matches_oracle(ctx):
    """The Gemma-4-style shape (30 layers cut to 2): width 2816, 16 heads /
    8 KV heads of 256, 128 experts of 704 with 8 routed, a shared FFN of
    2048, the tied 262144-row output soft-capped at 30; two clients, on the
    chained matrix-core step."""
    cfg = DenseConfig(**{**GEMMA4_MOE.__dict__, "layers": 2})
    run_against_oracle(ctx, cfg, 2, 4, 16, 61, gemma_layer_scales)


# ---- Zipf routing for throughput runs, and the device route trace -----------

def zipf_inclusion(E, k, s, draws, rng):
    """Monte Carlo inclusion probability of each expert in a Gumbel-top-k
    sample with P(e) proportional to (e + 1)^-s."""
    logits = -s * np.log(np.arange(1, E + 1))
    g = rng.gumbel(size=(draws, E))
    top = np.argsort(-(logits + g), axis=1)[:, :k]
    return np.bincount(top.reshape(-1), minlength=E) / draws


def test_zipf_routing_and_route_trace(ctx):
    cfg = small_granite(experts=32, used=8)
    model = Model(ctx, cfg)
    model.synth(91)
    n, steps, cap = 4, 48, 64
    prompts = np.arange(n * 4, dtype=np.uint32).reshape(n, 4)

    def run(s, seed):
        sess = Session(model, n, 128)
        sess.route_trace(cap)
        sess.route_zipf(s, seed)
        sess.generate(prompts, steps)
        slots = [sess.read_routes(i) for i in range(4 + steps - 1)]
        sess.close()
        return slots

    traced = run(1.1, 7)
    ids = np.stack([t[0] for t in traced])       # steps x layers x clients x k
    w = np.stack([t[1] for t in traced])
    assert ids.min() >= 0 and ids.max() < 32
    assert all(len(set(row)) == 8 for row in ids.reshape(-1, 8).tolist())  # distinct experts per token
    assert np.allclose(w.sum(-1), 1.0, atol=1e-5) and np.all(np.diff(w, axis=-1) <= 0)  # rank order
    freq = np.bincount(ids.reshape(-1), minlength=32) / ids.reshape(-1, 8).shape[0]
    want = zipf_inclusion(32, 8, 1.1, 20000, np.random.default_rng(0))
    assert np.max(np.abs(freq - want)) < 0.15, (freq, want)
    assert freq[0] > 0.8 and freq[31] < 0.35
    # the same seed routes the same way; another seed does not
    again = np.stack([t[0] for t in run(1.1, 7)])
    assert np.array_equal(again, ids)
    other = np.stack([t[0] for t in run(1.1, 8)])
    assert not np.array_equal(other, ids)
    # back on the model's own router: routes are the router's (distinct, weights summing to one)
    own = run(0.0, 0)
    oi = np.stack([t[0] for t in own])
    assert all(len(set(row)) == 8 for row in oi.reshape(-1, 8).tolist())
    model.close()
