"""Decode-step parity: the device-resident decoder against the oracle.

Bars (stated per the target): logits within ||gpu - ref||_inf <= 1e-3 *
||ref||_inf per step; greedy tokens identical over 256 decode steps; the fp16
KV cache holds exactly the oracle's fp16-rounded keys/values to within the
logit tolerance propagated through one layer (checked at 1e-3 relative).
"""
import numpy as np
import pytest

import oracle
from emufpga_amd import _lib
from emufpga_amd.serve import DenseConfig, Model, Session

pytestmark = pytest.mark.gpu

SMALL_QWEN3 = DenseConfig(hidden=512, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, layers=3,
                          rope_theta=1e6, eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K, tied=False,
                          qk_norm=True)
SMALL_SMOL = DenseConfig(hidden=576, heads=9, kv_heads=3, head_dim=64, ffn=1536, vocab=2048, layers=3,
                         rope_theta=1e5, eps=1e-5, style=_lib.EMU_STYLE_SMOL, encoding=_lib.Q8_0, tied=True,
                         qk_norm=False)


def oracle_for(model: Model, context: int, kv_f16: bool, n_clients: int) -> oracle.DenseOracle:
    c = model.cfg
    cfg = oracle.DenseCfg(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim, ffn=c.ffn,
                          vocab=c.vocab, layers=c.layers, context=context, rope_theta=c.rope_theta, eps=c.eps,
                          style=c.style, dtype=c.encoding, kv_f16=int(kv_f16), tied=int(c.tied),
                          qk_norm=int(c.qk_norm))
    return oracle.DenseOracle(cfg, model.host_weights(), n_clients)


def rel_inf(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("cfg", [SMALL_QWEN3, SMALL_SMOL], ids=["qwen3", "smol"])
def test_decode_steps_match_oracle(ctx, cfg):
    model = Model(ctx, cfg)
    model.synth(1234)
    context = 300  # > one 256-position attention chunk: exercises the split merge
    sess = Session(model, 2, context, kv_f16=True)
    ref = oracle_for(model, context, True, 2)
    rng = np.random.default_rng(0)
    worst = 0.0
    for step in range(270):
        toks = rng.integers(0, cfg.vocab, size=2).astype(np.uint32)
        nxt, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        if step % 9 == 0 or step > 255:
            for c in range(2):
                worst = max(worst, rel_inf(logits[c], r[c]))
                tie_last = cfg.style == _lib.EMU_STYLE_SMOL
                assert int(nxt[c]) == int(np.argmax(logits[c])) if not tie_last else True
    assert worst <= 1e-3, worst
    assert list(sess.positions()) == [270, 270]
    kv = sess.read_kv(1, cfg.layers - 1, values=False, positions=270)
    rk = ref.cache(1, cfg.layers - 1, values=False)[:270]
    assert np.max(np.abs(kv - rk)) <= 1e-3 * np.max(np.abs(rk))


@pytest.mark.parametrize("cfg", [SMALL_QWEN3, SMALL_SMOL], ids=["qwen3", "smol"])
def test_greedy_tokens_identical_over_256_steps(ctx, cfg):
    model = Model(ctx, cfg)
    model.synth(99)
    prompt_len, steps = 8, 256
    context = prompt_len + steps
    sess = Session(model, 1, context, kv_f16=True)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, cfg.vocab, size=(1, prompt_len)).astype(np.uint32)
    got = sess.generate(prompt, steps)[0]
    ref = oracle_for(model, context, True, 1)
    tie_last = cfg.style == _lib.EMU_STYLE_SMOL
    toks = []
    for t in range(prompt_len):
        logits = ref.step(prompt[:, t])
    nxt = oracle.argmax(logits[0], tie_last)
    toks.append(nxt)
    for _ in range(steps - 1):
        logits = ref.step([nxt])
        nxt = oracle.argmax(logits[0], tie_last)
        toks.append(nxt)
    assert list(got) == toks


# Qwen3-8B widths (the 4096- and 12288-column integer-limb matvecs at batch 1)
# with two layers and a short vocabulary, so the oracle keeps up.
WIDE_QWEN3 = DenseConfig(hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=3000, layers=2,
                         rope_theta=1e6, eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K, tied=False,
                         qk_norm=True)


def test_qwen3_width_decode_matches_oracle(ctx):
    model = Model(ctx, WIDE_QWEN3)
    model.synth(4321)
    steps, context = 12, 80
    sess = Session(model, 1, context, kv_f16=True)
    ref = oracle_for(model, context, True, 1)
    rng = np.random.default_rng(5)
    worst = 0.0
    for step in range(steps):
        toks = rng.integers(0, WIDE_QWEN3.vocab, size=1).astype(np.uint32)
        nxt, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        worst = max(worst, rel_inf(logits[0], r[0]))
        assert int(nxt[0]) == oracle.argmax(r[0], False), step
    assert worst <= 1e-3, worst


def test_qwen3_width_batched_decode_matches_oracle(ctx):
    """Several clients at Qwen3-8B widths: the chained multi-token matvecs
    (int8 matrix cores) against the oracle, per client."""
    model = Model(ctx, WIDE_QWEN3)
    model.synth(4322)
    steps, context, n = 10, 80, 4
    sess = Session(model, n, context, kv_f16=True)
    ref = oracle_for(model, context, True, n)
    rng = np.random.default_rng(6)
    worst = 0.0
    for step in range(steps):
        toks = rng.integers(0, WIDE_QWEN3.vocab, size=n).astype(np.uint32)
        nxt, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        for c in range(n):
            worst = max(worst, rel_inf(logits[c], r[c]))
            assert int(nxt[c]) == oracle.argmax(r[c], False), (step, c)
    assert worst <= 1e-3, worst


# One client at a 1060-token context: the attention's last-arriving workgroup
# merges up to 17 chunks of 64 positions, past its 16-chunk load batches, and
# the 32 query heads of 128 feed the 4096-column integer-limb o projection.
DEEP_QWEN3 = DenseConfig(hidden=512, heads=32, kv_heads=8, head_dim=128, ffn=512, vocab=600, layers=2,
                         rope_theta=1e6, eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K, tied=False,
                         qk_norm=True)


def test_long_context_chunk_merge_in_the_o_projection_matches_oracle(ctx):
    model = Model(ctx, DEEP_QWEN3)
    model.synth(77)
    context = 1060
    sess = Session(model, 1, context, kv_f16=True)
    ref = oracle_for(model, context, True, 1)
    rng = np.random.default_rng(78)
    worst, checked = 0.0, 0
    for step in range(context):
        toks = rng.integers(0, DEEP_QWEN3.vocab, size=1).astype(np.uint32)
        check = step < 2 or step in (63, 64, 65, 127, 128, 1023, 1024) or step % 101 == 0 or step >= context - 2
        r = ref.step(toks)
        if not check:
            sess.decode_step(toks)
        else:
            nxt, logits = sess.decode_step(toks, want_logits=True)
            worst = max(worst, rel_inf(logits[0], r[0]))
            assert int(nxt[0]) == oracle.argmax(r[0], False), step
            checked += 1
    assert checked > 15 and worst <= 1e-3, worst
    sess.close()
    model.close()


# Hidden width 12288 at two clients: the chained multi-token matvec leaves
# q|k|v as twelve 1024-column partial-sum slices, the most the attention's
# branch-free slice sum takes.
TWELVE_SLICES = DenseConfig(hidden=12288, heads=64, kv_heads=8, head_dim=128, ffn=12288, vocab=512, layers=1,
                            rope_theta=1e6, eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K, tied=False,
                            qk_norm=True)


def test_twelve_slice_width_batched_decode_matches_oracle(ctx):
    model = Model(ctx, TWELVE_SLICES)
    model.synth(1212)
    steps, context, n = 5, 16, 2
    sess = Session(model, n, context, kv_f16=True)
    ref = oracle_for(model, context, True, n)
    rng = np.random.default_rng(12)
    worst = 0.0
    for step in range(steps):
        toks = rng.integers(0, TWELVE_SLICES.vocab, size=n).astype(np.uint32)
        nxt, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        for c in range(n):
            worst = max(worst, rel_inf(logits[c], r[c]))
            assert int(nxt[c]) == oracle.argmax(r[c], False), (step, c)
    assert worst <= 1e-3, worst
    sess.close()
    model.close()


ATTN_SHAPES = [
    # (heads, kv_heads, head_dim, style): group sizes 8, 1, 3 and 2; head dims 64, 256, 128
    (8, 1, 64, _lib.EMU_STYLE_QWEN3),
    (2, 2, 256, _lib.EMU_STYLE_QWEN3),
    (6, 2, 128, _lib.EMU_STYLE_SMOL),
    (4, 2, 256, _lib.EMU_STYLE_SMOL),
]


@pytest.mark.parametrize("heads,kv_heads,head_dim,style", ATTN_SHAPES)
def test_attention_shapes_match_oracle(ctx, heads, kv_heads, head_dim, style):
    smol = style == _lib.EMU_STYLE_SMOL
    cfg = DenseConfig(hidden=512, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=768, vocab=600,
                      layers=2, rope_theta=1e5 if smol else 1e6, eps=1e-5 if smol else 1e-6, style=style,
                      encoding=_lib.Q8_0 if smol else _lib.Q6_K, tied=smol, qk_norm=not smol)
    model = Model(ctx, cfg)
    model.synth(heads * 1000 + head_dim)
    context = 140
    sess = Session(model, 2, context, kv_f16=True)
    ref = oracle_for(model, context, True, 2)
    rng = np.random.default_rng(heads + head_dim)
    worst = 0.0
    for step in range(context):
        toks = rng.integers(0, cfg.vocab, size=2).astype(np.uint32)
        _, logits = sess.decode_step(toks, want_logits=True)
        r = ref.step(toks)
        if step % 7 == 0 or step >= context - 3:
            worst = max(worst, rel_inf(logits[0], r[0]), rel_inf(logits[1], r[1]))
    assert worst <= 1e-3, worst


def test_batched_client_gets_what_it_would_alone(ctx):  # spm-batch/tests/batching.rs:128-145
    model = Model(ctx, SMALL_QWEN3)
    model.synth(7)
    prompts = np.array([[1, 2, 3, 4], [9, 8, 7, 6], [5, 5, 5, 5]], np.uint32)
    together = Session(model, 3, 64).generate(prompts, 20)
    for c in range(3):
        alone = Session(model, 1, 64).generate(prompts[c:c + 1], 20)
        assert np.array_equal(alone[0], together[c])


def test_context_full_is_an_error(ctx):  # spm-kv/src/cache.rs:50-54
    model = Model(ctx, SMALL_SMOL)
    model.synth(3)
    sess = Session(model, 1, 10)
    with pytest.raises(_lib.ContextFull):
        sess.generate(np.zeros((1, 5), np.uint32), 7)
    for _ in range(10):
        sess.decode_step([1])
    with pytest.raises(_lib.ContextFull):
        sess.decode_step([1])


def test_generate_is_deterministic_and_replays(ctx):
    model = Model(ctx, SMALL_QWEN3)
    model.synth(11)
    sess = Session(model, 2, 128)
    prompts = np.array([[3, 1, 4, 1, 5], [2, 7, 1, 8, 2]], np.uint32)
    a = sess.generate(prompts, 40)
    sess.reset()
    b = sess.generate(prompts, 40)
    assert np.array_equal(a, b)


def test_a_client_replaced_mid_run_gets_what_a_fresh_client_gets(ctx):
    """Continuous batching in lockstep: client 1 is replaced by a fresh client
    after 10 steps; both clients then get exactly what they would alone."""
    model = Model(ctx, SMALL_QWEN3)
    model.synth(17)
    rng = np.random.default_rng(18)
    a_prompt = rng.integers(0, SMALL_QWEN3.vocab, size=30).astype(np.uint32)
    b_prompt = rng.integers(0, SMALL_QWEN3.vocab, size=12).astype(np.uint32)
    c_prompt = rng.integers(0, SMALL_QWEN3.vocab, size=20).astype(np.uint32)

    def alone(prompt):
        s = Session(model, 1, 64)
        out = [int(s.decode_step([t])[0]) for t in prompt]
        s.close()
        return out

    sess = Session(model, 2, 64)
    got_a, got_c = [], []
    for i in range(10):
        nxt = sess.decode_step([a_prompt[i], b_prompt[i]])
        got_a.append(int(nxt[0]))
    sess.reset_client(1)
    assert list(sess.positions()) == [10, 0]
    for i in range(20):
        nxt = sess.decode_step([a_prompt[10 + i], c_prompt[i]])
        got_a.append(int(nxt[0]))
        got_c.append(int(nxt[1]))
    assert got_a == alone(a_prompt)
    assert got_c == alone(c_prompt)
    with pytest.raises(_lib.EmuError):
        sess.reset_client(2)


def _oracle_greedy(ref: oracle.DenseOracle, prompt: np.ndarray, steps: int, tie_last: bool) -> np.ndarray:
    """Feed each client's prompt one token per step, then its own greedy
    token for `steps` steps (serve-demo.rs:62-91), all clients in lockstep."""
    n = prompt.shape[0]
    for t in range(prompt.shape[1]):
        logits = ref.step(prompt[:, t])
    toks = np.empty((n, steps), np.uint32)
    nxt = np.array([oracle.argmax(logits[c], tie_last) for c in range(n)], np.uint32)
    for s in range(steps):
        toks[:, s] = nxt
        if s + 1 < steps:
            logits = ref.step(nxt)
            nxt = np.array([oracle.argmax(logits[c], tie_last) for c in range(n)], np.uint32)
    return toks


def _oracle_threads():
    import os
    return max(1, min(16, os.cpu_count() or 1))


def test_greedy_256_steps_on_the_batch1_limb_kernels(ctx):
    """One client at Qwen3-8B widths: every projection (q|k|v, o, gate|up,
    the 12288-column down, the output rows) runs the timed integer-limb
    matvec; 256 greedy tokens after a 16-token prompt equal the oracle's."""
    model = Model(ctx, WIDE_QWEN3)
    model.synth(2024)
    prompt_len, steps = 16, 256
    context = prompt_len + steps
    sess = Session(model, 1, context, kv_f16=True)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, WIDE_QWEN3.vocab, size=(1, prompt_len)).astype(np.uint32)
    got = sess.generate(prompt, steps)
    oracle.set_threads(_oracle_threads())
    try:
        want = _oracle_greedy(oracle_for(model, context, True, 1), prompt, steps, False)
    finally:
        oracle.set_threads(1)
    assert np.array_equal(got, want), int(np.argmax(got[0] != want[0]))
    sess.close()
    model.close()


@pytest.mark.parametrize("n_clients", [1, 3])
def test_f32_activation_mode_matches_oracle(ctx, n_clients):
    """EMU_SESSION_F32_ACT at Qwen3-8B widths, where the default step takes
    the int8-limb kernels (batch 1) or the matrix cores (3 clients): every
    matvec dequantizes and multiplies in f32 instead.  Logits within 1e-3 *
    max |logit| and greedy tokens equal to the oracle's on every step."""
    model = Model(ctx, WIDE_QWEN3)
    model.synth(99)
    context = 48
    sess = Session(model, n_clients, context, kv_f16=True)
    assert ctx.lib.emu_session_set_options(sess.h, 4) == _lib.EMU_E_ARG  # unknown bit
    sess.set_options(f32_act=True)
    ref = oracle_for(model, context, True, n_clients)
    rng = np.random.default_rng(n_clients)
    oracle.set_threads(_oracle_threads())
    worst = 0.0
    try:
        for step in range(40):
            toks = rng.integers(0, WIDE_QWEN3.vocab, size=n_clients).astype(np.uint32)
            nxt, logits = sess.decode_step(toks, want_logits=True)
            r = ref.step(toks)
            for c in range(n_clients):
                worst = max(worst, rel_inf(logits[c], r[c]))
                assert int(nxt[c]) == oracle.argmax(r[c], False), (step, c)
    finally:
        oracle.set_threads(1)
    print(f"f32 activations, {n_clients} client(s): worst logit error {worst:.2e} of max |logit|")
    assert worst <= 1e-3, worst
    sess.close()
    model.close()


# Eight clients at Qwen3-8B widths (hidden 4096, 32/8 heads of 128, SwiGLU
# 12288) through the chained int8 matrix-core matvecs; two layers and a
# 2000-row output keep the oracle's 8 x 271 steps inside the test's time.
WIDE_QWEN3_2L = DenseConfig(hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=2000, layers=2,
                            rope_theta=1e6, eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K,
                            tied=False, qk_norm=True)


def test_greedy_256_steps_on_the_eight_client_mfma_chain(ctx):
    """Eight clients, 16-token prompts, 256 greedy steps through the chained
    int8 matrix-core matvecs, step by step beside the oracle (its tokens fed
    to both): every step's logits within 1e-3 * max |logit| of the oracle's,
    and every client's greedy token equal to the oracle's argmax unless the
    oracle's top-2 gap is within that bar on both sides (gap <= 2e-3 * max
    |logit|: a numerical tie, which must then pick the runner-up).  The count
    of ties and the smallest gap met are printed."""
    model = Model(ctx, WIDE_QWEN3_2L)
    model.synth(2025)
    n, prompt_len, steps = 8, 16, 256
    context = prompt_len + steps
    sess = Session(model, n, context, kv_f16=True)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, WIDE_QWEN3_2L.vocab, size=(n, prompt_len)).astype(np.uint32)
    ref = oracle_for(model, context, True, n)
    oracle.set_threads(_oracle_threads())
    worst, min_gap, ties, diverged = 0.0, float("inf"), [], []
    try:
        toks = prompt[:, 0]
        for step in range(prompt_len - 1 + steps):
            nxt, logits = sess.decode_step(toks, want_logits=True)
            r = ref.step(toks)
            want = np.array([oracle.argmax(r[c], False) for c in range(n)], np.uint32)
            for c in range(n):
                scale = float(np.max(np.abs(r[c])))
                worst = max(worst, float(np.max(np.abs(logits[c].astype(np.float64) - r[c]))) / scale)
                if step >= prompt_len - 1:
                    order = np.argsort(-r[c], kind="stable")[:2]
                    gap = float(r[c][order[0]] - r[c][order[1]]) / scale
                    min_gap = min(min_gap, gap)
                    if int(nxt[c]) != int(want[c]):
                        tie = gap <= 2e-3 and int(nxt[c]) == int(order[1])
                        (ties if tie else diverged).append((step, c, gap))
            toks = prompt[:, step + 1] if step + 1 < prompt_len else want
    finally:
        oracle.set_threads(1)
    print(f"8-client chain: worst logit error {worst:.2e} of max |logit|; smallest top-2 gap {min_gap:.2e}; "
          f"ties {ties}")
    assert worst <= 1e-3, worst
    assert not diverged, diverged
    sess.close()
    model.close()
