"""Mixture-of-experts decoders at their workload shapes against the oracle's
decode steps, committed as golden files (tests/golden/make_moe_goldens.py):
the oracle needs minutes for these shapes, a GPU test has seconds.

  gemma6     the Gemma-4-style decoder with 6 of its 30 layers, so that the
             global layer (5) runs beside five 1024-position sliding-window
             layers, 2 clients, 1040-token prompts (past the window), 8
             checked steps;
  granite24  the Granite decoder at all 24 layers, 4 clients, 256-token
             prompts, 16 checked steps.

The device synthesis first gives the golden run's weights (SHA-256 of every
layer's pieces).  The prompts are fed token by token; then each checked step
feeds the oracle's tokens (teacher forcing).  Bars per step and client: the
logits at the oracle's 8 largest entries within 1e-3 * max |logit| of the
oracle's, and the greedy token the oracle's unless its top-2 gap is within
that bar on both sides (a numerical tie, which must then pick the
runner-up).  Both activation forms: the int8 limbs of the timed path and f32
(EMU_SESSION_F32_ACT).  The worst error and any ties are printed.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from emufpga_amd import _lib
from emufpga_amd.serve import GEMMA4_MOE, GRANITE_MOE_Q6K, DenseConfig, Model, Session

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
SHAPES = {"gemma6": DenseConfig(**{**GEMMA4_MOE.__dict__, "layers": 6}), "granite24": GRANITE_MOE_Q6K}
TOL = 1e-3


@pytest.fixture(scope="module", params=sorted(SHAPES))
def case(request, ctx):
    path = GOLDEN / f"{request.param}.json"
    if not path.exists():
        pytest.skip(f"{path.name} not written (tests/golden/make_moe_goldens.py)")
    with open(path) as f:
        doc = json.load(f)
    cfg = SHAPES[request.param]
    model = Model(ctx, cfg)
    model.synth(doc["weights"]["synth_seed"])
    yield request.param, cfg, model, doc
    model.close()


def test_device_weights_are_the_golden_runs(case):
    name, cfg, model, doc = case
    for layer in range(cfg.layers):
        blob = model.read_tensor(_lib.EMU_T_LAYER, layer)
        h = hashlib.sha256()
        for off, n, *_ in oracle.moe_layer_pieces(cfg, layer):
            h.update(blob[off:off + n].tobytes())
        assert h.hexdigest() == doc["weights"]["layer_piece_sha256"][layer], (name, layer)


@pytest.mark.parametrize("mode", ["int8", "f32"])
def test_checked_steps_match_the_oracle(case, mode):
    name, cfg, model, doc = case
    prompts = np.array(doc["prompts"], np.uint32)
    n, plen = prompts.shape
    steps = doc["steps"]
    sess = Session(model, n, plen + len(steps), kv_f16=True)
    sess.set_options(f32_act=(mode == "f32"))
    for t in range(plen - 1):
        sess.decode_step(prompts[:, t])
    feed = prompts[:, -1]
    worst, ties, wrong = 0.0, [], []
    for i, rec in enumerate(steps):
        nxt, lg = sess.decode_step(feed, want_logits=True)
        for c, r in enumerate(rec):
            lc = lg[c].astype(np.float64)
            err = float(np.max(np.abs(lc[np.array(r["top_ids"])] - np.array(r["top_vals"]))))
            worst = max(worst, err / r["max_abs"], abs(float(np.max(np.abs(lc))) - r["max_abs"]) / r["max_abs"])
            if int(nxt[c]) != r["token"]:
                tie = r["gap"] <= 2 * TOL * r["max_abs"] and int(nxt[c]) == r["top_ids"][1]
                (ties if tie else wrong).append((i, c, r["gap"] / r["max_abs"]))
        feed = np.array([r["token"] for r in rec], np.uint32)
    sess.close()
    print(f"{name} {mode}: worst logit error {worst:.3e} of max |logit| over {len(steps)} steps x {n} clients; "
          f"ties {ties}")
    assert worst <= TOL, worst
    assert not wrong, wrong
