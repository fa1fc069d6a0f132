"""Mixture-of-experts decode step (spm-granite-moe/src/model.rs:330-411) on the
GPU against the oracle's or_moe_model_step.

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
from emufpga_amd.serve import GRANITE_MOE_Q6K, DenseConfig, Model, Session

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
                             kv_f16=int(kv_f16), qk_norm=int(c.qk_norm))
    w = model.host_weights()
    assert w["layers"].size == c.layers * oracle.moe_layer_bytes(cfg)
    return oracle.MoeModelOracle(cfg, w, n_clients)


def rel_inf(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("expert_encoding,n_clients", [(_lib.Q6_K, 1), (_lib.Q6_K, 3), (_lib.Q2_K, 2)],
                         ids=["q6k-1", "q6k-3", "q2k-2"])
def test_moe_decode_steps_match_oracle(ctx, expert_encoding, n_clients):
    model = Model(ctx, small_granite(expert_encoding))
    model.synth(2024 + expert_encoding)
    context = 80  # two attention chunks: the split merge
    sess = Session(model, n_clients, context, kv_f16=True)
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


def test_moe_config_rejects_untied_and_oversized_routes(ctx):
    with pytest.raises(_lib.EmuError):
        Model(ctx, DenseConfig(**{**small_granite().__dict__, "tied": False}))
    with pytest.raises(_lib.EmuError):
        Model(ctx, DenseConfig(**{**small_granite().__dict__, "experts_used": 9, "n_experts": 16}))
