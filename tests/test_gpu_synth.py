"""The device synthesis writes the bytes the oracle's CPU twin computes.

emu_model_synth draws every weight on the device; oracle/synth.c computes the
same draws and quantization on the CPU, so that oracle runs too long for a GPU
test can be done without a GPU and committed (tests/golden/).  Here every
tensor of small dense models (Q6_K, Q8_0) and mixture-of-experts layers (the
f32 router, Q2_K experts, Q5_K fused gate|up experts with Q8_0 downs, the
Gemma form's scales and shared FFN) is compared byte for byte.
"""
import numpy as np
import pytest

import oracle
from emufpga_amd import _lib
from emufpga_amd.serve import DenseConfig, Model

pytestmark = pytest.mark.gpu

DENSE = [
    DenseConfig(hidden=512, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, layers=2, rope_theta=1e6,
                eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K, tied=False, qk_norm=True),
    DenseConfig(hidden=576, heads=9, kv_heads=3, head_dim=64, ffn=1536, vocab=2048, layers=2, rope_theta=1e5,
                eps=1e-5, style=_lib.EMU_STYLE_SMOL, encoding=_lib.Q8_0, tied=True, qk_norm=False),
]
MOE = [
    DenseConfig(512, 4, 4, 128, 0, 1000, 2, 1e4, 1e-5, _lib.EMU_STYLE_GRANITE, _lib.Q6_K, False, True,
                n_experts=8, experts_used=2, expert_ff=256, expert_encoding=_lib.Q2_K, score_mul=0.088388,
                rope_neox=True),
    DenseConfig(512, 4, 2, 256, 0, 1000, 2, 1e4, 1e-6, _lib.EMU_STYLE_GRANITE, _lib.Q6_K, True, True,
                n_experts=8, experts_used=2, expert_ff=256, expert_encoding=_lib.Q5_K, embed_scale=22.6,
                score_mul=1.0 / 16, rope_neox=True, gemma=True, expert_down_encoding=_lib.Q8_0, shared_ff=256,
                window=64, global_every=2, rope_theta_global=1e6, logit_softcap=30.0),
]


def ocfg(c: DenseConfig) -> oracle.DenseCfg:
    return oracle.DenseCfg(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim, ffn=c.ffn,
                           vocab=c.vocab, layers=c.layers, context=4, rope_theta=c.rope_theta, eps=c.eps,
                           style=c.style, dtype=c.encoding, kv_f16=1, tied=int(c.tied), qk_norm=int(c.qk_norm))


@pytest.mark.parametrize("cfg", DENSE, ids=["q6k", "q8_0"])
def test_dense_synthesis_equals_the_cpu_twin(ctx, cfg):
    model = Model(ctx, cfg)
    model.synth(77)
    got = model.host_weights()
    want = oracle.synth_dense_weights(ocfg(cfg), 77)
    for k in want:
        assert np.array_equal(got[k].view(np.uint8), want[k].view(np.uint8)), k
    model.close()


@pytest.mark.parametrize("cfg", MOE, ids=["q2k_experts", "gemma_q5k_q8_0"])
def test_moe_synthesis_equals_the_cpu_twin(ctx, cfg):
    model = Model(ctx, cfg)
    model.synth(78)
    for layer in range(cfg.layers):
        blob = model.read_tensor(_lib.EMU_T_LAYER, layer)
        for off, want in oracle.synth_moe_layer(cfg, 78, layer):
            assert np.array_equal(blob[off:off + want.size], want), (layer, off)
    be, bb = oracle.BLOCK[cfg.encoding]
    embed = oracle.synth_blocks(cfg.encoding, cfg.vocab * (cfg.hidden // be) * bb, 78, 1)
    assert np.array_equal(model.read_tensor(_lib.EMU_T_EMBED), embed)
    model.close()
