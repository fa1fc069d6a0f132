#!/usr/bin/env python3
"""Golden decode steps of two mixture-of-experts decoders at their real
shapes, from the oracle (too slow for a GPU test's time limit):

  gemma6_window.json  the Gemma-4-style decoder cut to 6 layers (local
                      layers 0-4 with the 1024-position window at RoPE 1e4,
                      global layer 5 at RoPE 1e6), 2 clients, 1040-token
                      prompts (past the window), then 8 checked steps;
  granite24.json      the Granite decoder at all 24 layers, 4 clients,
                      256-token prompts, then 16 checked steps.

Weights: the bytes the library's device synthesis writes (oracle.
synth_moe_weights, synth.c), with SHA-256 digests of every layer's pieces for
the GPU test to check first.  Prompts: numpy default_rng, uniform ids.  The
router is the model's own (no injected routing).  Each checked step feeds the
oracle's own greedy token (ties to the lowest index, math.rs:35-40) and
records per client the token, the 8 largest logits with their indices, the
top-2 gap and the largest |logit|.

Usage: python tests/golden/make_moe_goldens.py [--only gemma6|granite24] [--threads N]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from emufpga_amd.serve import GEMMA4_MOE, GRANITE_MOE_Q6K, DenseConfig  # noqa: E402

CASES = {
    # name: (shape, synthesis seed, clients, prompt length, checked steps, prompt seed)
    "gemma6": (DenseConfig(**{**GEMMA4_MOE.__dict__, "layers": 6}), 606, 2, 1040, 8, 61),
    "granite24": (GRANITE_MOE_Q6K, 2424, 4, 256, 16, 62),
}


def moe_cfg(c: DenseConfig, context: int) -> oracle.MoeModelCfg:
    return oracle.MoeModelCfg(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                              vocab=c.vocab, layers=c.layers, context=context, n_experts=c.n_experts,
                              experts_used=c.experts_used, expert_ff=c.expert_ff, rope_theta=c.rope_theta,
                              eps=c.eps, embed_scale=c.embed_scale, residual_scale=c.residual_scale,
                              logit_div=c.logit_div, score_mul=c.score_mul, dtype=c.encoding,
                              expert_dtype=c.expert_encoding, kv_f16=1, qk_norm=int(c.qk_norm),
                              rope_neox=int(c.rope_neox), untied=int(not c.tied), gemma=int(c.gemma),
                              expert_down_dtype=c.expert_down_encoding, shared_ff=c.shared_ff, window=c.window,
                              global_every=c.global_every, rope_theta_global=c.rope_theta_global,
                              softcap=c.logit_softcap)


def piece_digest(blob: np.ndarray, pieces) -> str:
    h = hashlib.sha256()
    for off, n, *_ in pieces:
        h.update(blob[off:off + n].tobytes())
    return h.hexdigest()


def run(name: str) -> dict:
    c, seed, n, prompt_len, steps, pseed = CASES[name]
    mcfg = moe_cfg(c, prompt_len + steps)
    t0 = time.time()
    w = oracle.synth_moe_weights(c, mcfg, seed)
    lb = oracle.moe_layer_bytes(mcfg)
    digests = [piece_digest(w["layers"][l * lb:(l + 1) * lb], oracle.moe_layer_pieces(c, l)) for l in range(c.layers)]
    print(f"{name}: synthesised {w['layers'].nbytes / 1e9:.2f} GB of layers in {time.time() - t0:.0f} s", flush=True)
    prompts = np.random.default_rng(pseed).integers(0, c.vocab, size=(n, prompt_len)).astype(np.uint32)
    orc = oracle.MoeModelOracle(mcfg, w, n)
    t0 = time.time()
    for t in range(prompt_len - 1):
        orc.step(prompts[:, t], want_logits=False)
        if t % 128 == 0:
            print(f"{name}: prompt position {t}, {time.time() - t0:.0f} s", flush=True)
    feed = prompts[:, -1]
    out = []
    for i in range(steps):
        lg = orc.step(feed)
        rec = []
        for ci in range(n):
            top = np.argsort(-lg[ci], kind="stable")[:8]
            tok = oracle.argmax(lg[ci], False)
            assert tok == int(top[0])
            rec.append({"token": tok, "top_ids": [int(v) for v in top], "top_vals": [float(lg[ci][v]) for v in top],
                        "gap": float(lg[ci][top[0]] - lg[ci][top[1]]), "max_abs": float(np.max(np.abs(lg[ci])))})
        out.append(rec)
        feed = np.array([r["token"] for r in rec], np.uint32)
        print(f"{name}: step {i}: tokens {[r['token'] for r in rec]}, {time.time() - t0:.0f} s", flush=True)
    return {"what": f"{name}: decode steps of the oracle at the workload's shape (see make_moe_goldens.py)",
            "layers": c.layers, "clients": n, "weights": {"synth_seed": seed, "layer_piece_sha256": digests},
            "prompts": prompts.tolist(), "steps": out, "oracle_seconds": round(time.time() - t0, 1)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=sorted(CASES))
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    args = ap.parse_args()
    oracle.set_threads(args.threads)
    for name in [args.only] if args.only else sorted(CASES):
        doc = run(name)
        path = os.path.join(ROOT, "tests", "golden", f"{name}.json")
        with open(path, "w") as f:
            json.dump(doc, f, indent=0)
            f.write("\n")
        print(f"wrote {path}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
