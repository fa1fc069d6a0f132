"""Planted mistakes in the oracle must fail its pinning tests (CPU only).

Each case copies oracle/oracle.c, changes one expression the way a plausible
slip would (a RoPE exponent, a score scale, the SwiGLU operand order, the k
QK-norm, the post-attention residual), builds the copy with the oracle's own
flags and reruns the pinning tests against it in a child process
(ORACLE_LIB).  The case passes only if that run fails: the float64
compositions and closed forms in tests/test_oracle.py can see the mistake.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "oracle" / "oracle.c"

# (name, original text, replacement, which occurrence (0-based))
MUTATIONS = [
    ("neox_rope_exponent", "float exponent = 2.0f * index_f / width;", "float exponent = index_f / width;", 0),
    ("fma_rope_exponent", "powf(base, -2.0f * index / width)", "powf(base, -1.0f * index / width)", 0),
    ("interleaved_rope_exponent", "float exponent = (float)pair / (float)dim;",
     "float exponent = (float)pair / (float)dim / 2.0f;", 0),
    ("score_div_becomes_mul", "scores[p] = dot / c;", "scores[p] = dot * c;", 0),
    ("score_inv_sqrt_dropped", "scores[p] = dot * inv;", "scores[p] = dot;", 0),
    ("granite_score_scale_dropped", "scores[p] = dot * c;", "scores[p] = dot;", 0),
    ("swiglu_operands_swapped", "gate[i] = or_silu(gate[i]) * up[i];", "gate[i] = or_silu(up[i]) * gate[i];", 0),
    ("k_qk_norm_skipped", "or_rms_norm(kh, w->k_norm", "(void)0; if (0) or_rms_norm(kh, w->k_norm", 0),
    ("attention_residual_dropped", "state[i] = state[i] + proj[i];", "state[i] = state[i];", 0),
    ("ffn_residual_dropped", "state[i] = state[i] + proj[i];", "state[i] = state[i];", 1),
    ("final_norm_gain_dropped", "or_rms_norm(cs, w->out_norm, H, cfg->eps, cx);",
     "{ float one_[8192]; for (uint32_t i_ = 0; i_ < H; ++i_) one_[i_] = 1.0f; "
     "or_rms_norm(cs, one_, H, cfg->eps, cx); }", 0),
    ("tied_output_ignored", "const uint8_t *out_w = cfg->tied ? w->embed : w->output;",
     "const uint8_t *out_w = w->output;", 0),
    # mixture-of-experts forms (Granite, OLMoE, Gemma-4)
    ("moe_neox_rope_as_interleaved", "if (c->rope_neox)\n                    or_rope_qwen3(q + h * hd",
     "if (0)\n                    or_rope_qwen3(q + h * hd", 0),
    ("moe_untied_output_ignored", "c->untied ? w->output : w->embed", "w->embed", 0),
    ("window_off_by_one", "pos + 1 - c->window", "pos - c->window", 0),
    ("global_layers_swapped", "(layer + 1) % c->global_every == 0", "layer % c->global_every == 0", 0),
    ("global_theta_unused", "c->gemma && global ? c->rope_theta_global : c->rope_theta", "c->rope_theta", 0),
    ("softcap_dropped", "lg[i] = c->softcap * tanhf(t);", "lg[i] = lg[i];", 0),
    ("router_input_sqrt_width_dropped", "r = r / sqrtf(w);", "r = r;", 0),
    ("expert_down_scale_dropped", "d.down_scale = dscale;", "d.down_scale = NULL;", 0),
    ("shared_ffn_gelu_as_silu", "sg[i] = or_gelu_tanh(sg[i]) * su[i];", "sg[i] = or_silu(sg[i]) * su[i];", 0),
    ("experts_read_normed_router_input", "or_moe_ffn(&d, xe, 1, ids, rw, moe)", "or_moe_ffn(&d, rin, 1, ids, rw, moe)", 0),
    ("embed_scale_dropped", "state[i] = state[i] * c->embed_scale;", "state[i] = state[i];", 0),
    ("gemma_router_eps", "sqrtf(mean + 1e-6f)", "sqrtf(mean + 1e-5f)", 0),
]

PINNING = ("test_rope_matches_float64 or test_attend_with_nonzero or test_dense_step_matches or test_moe_model_step"
           " or test_moe_model_forms or test_moe_model_gemma_router_eps")


def _replace_nth(text: str, old: str, new: str, n: int) -> str:
    start = -1
    for _ in range(n + 1):
        start = text.index(old, start + 1)
    return text[:start] + new + text[start + len(old):]


@pytest.mark.parametrize("name,old,new,nth", MUTATIONS, ids=[m[0] for m in MUTATIONS])
def test_planted_mistake_fails_pinning(tmp_path, name, old, new, nth):
    src = SRC.read_text()
    assert src.count(old) > nth, f"mutation site for {name} not found"
    mutated = tmp_path / "oracle.c"
    mutated.write_text(_replace_nth(src, old, new, nth))
    (tmp_path / "oracle.h").write_text((ROOT / "oracle" / "oracle.h").read_text())
    lib = tmp_path / "liboracle.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-shared", "-o",
                    str(lib), str(mutated), "-lm"], check=True, capture_output=True)
    env = dict(os.environ, ORACLE_LIB=str(lib))
    run = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                          str(ROOT / "tests" / "test_oracle.py"), "-k", PINNING],
                         cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=300)
    assert run.returncode == 1, f"{name}: pinning tests did not fail\n{run.stdout[-2000:]}"


def test_unmutated_copy_passes_pinning(tmp_path):
    """Control: the same harness on an unchanged copy passes, so the failures
    above come from the planted mistakes and not from the harness."""
    (tmp_path / "oracle.c").write_text(SRC.read_text())
    (tmp_path / "oracle.h").write_text((ROOT / "oracle" / "oracle.h").read_text())
    lib = tmp_path / "liboracle.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-shared", "-o",
                    str(lib), str(tmp_path / "oracle.c"), "-lm"], check=True, capture_output=True)
    env = dict(os.environ, ORACLE_LIB=str(lib))
    run = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                          str(ROOT / "tests" / "test_oracle.py"), "-k", PINNING],
                         cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout[-2000:]
