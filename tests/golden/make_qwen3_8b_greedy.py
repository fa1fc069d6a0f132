#!/usr/bin/env python3
"""Golden greedy decode of the Qwen3-8B-shaped Q6_K decoder, from the oracle.

The oracle needs about 9 s per token on one core for this shape (36 layers,
width 4096, 151936-row output), far beyond a GPU test's time limit, so the
tokens are computed here, once, and committed:

  * the weights are the bytes the library's device synthesis writes for
    QWEN3_8B_Q6K with seed 8 (oracle.synth_dense_weights, synth.c); the
    GPU test first checks that, tensor by tensor, through SHA-256 digests;
  * a 16-token prompt (numpy default_rng(2026), uniform ids), then 256
    greedy steps, fp16 KV cache, ties to the lowest index (top_k,
    spm-qwen3-slice/src/math.rs:38-48);
  * per step: the token, the logits' 8 largest values with their indices,
    the gap between the two largest and the largest |logit|.

Usage: python tests/golden/make_qwen3_8b_greedy.py [--threads N] [--steps 256]
Writes tests/golden/qwen3_8b_greedy.json.
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

SEED = 8
PROMPT_SEED = 2026
PROMPT_LEN = 16
OUT = os.path.join(ROOT, "tests", "golden", "qwen3_8b_greedy.json")


def qwen3_cfg(context: int) -> oracle.DenseCfg:
    return oracle.DenseCfg(hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936, layers=36,
                           context=context, rope_theta=1e6, eps=1e-6, style=0, dtype=oracle.OR_Q6_K, kv_f16=1,
                           tied=0, qk_norm=1)


def digests(w: dict, layers: int) -> dict:
    per = w["layers"].size // layers
    return {
        "layers": [hashlib.sha256(w["layers"][l * per:(l + 1) * per].tobytes()).hexdigest() for l in range(layers)],
        "embed": hashlib.sha256(w["embed"].tobytes()).hexdigest(),
        "output": hashlib.sha256(w["output"].tobytes()).hexdigest(),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--out", default=OUT)
    args = ap.parse_args()
    oracle.set_threads(args.threads)
    cfg = qwen3_cfg(PROMPT_LEN + args.steps)
    t0 = time.time()
    w = oracle.synth_dense_weights(cfg, SEED)
    print(f"synthesised {sum(v.nbytes for v in w.values()) / 1e9:.2f} GB in {time.time() - t0:.0f} s", flush=True)
    dig = digests(w, cfg.layers)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg.vocab, size=PROMPT_LEN).astype(np.uint32)
    orc = oracle.DenseOracle(cfg, w, 1)
    t0 = time.time()
    for t in range(PROMPT_LEN - 1):
        orc.step([int(prompt[t])])
    feed = int(prompt[-1])
    steps = []
    for i in range(args.steps):
        lg = orc.step([feed])[0]
        top = np.argsort(-lg, kind="stable")[:8]
        tok = oracle.argmax(lg, False)
        assert tok == int(top[0])
        steps.append({"token": tok, "top_ids": [int(v) for v in top], "top_vals": [float(lg[v]) for v in top],
                      "gap": float(lg[top[0]] - lg[top[1]]), "max_abs": float(np.max(np.abs(lg)))})
        feed = tok
        if i % 16 == 0:
            print(f"step {i}: token {tok}, gap {steps[-1]['gap']:.4g}, {time.time() - t0:.0f} s", flush=True)
    doc = {
        "what": "greedy decode of the Qwen3-8B-shaped Q6_K decoder (36 layers, width 4096, 32/8 heads of 128, "
                "QK-norm, SwiGLU 12288, untied 151936-row output, RoPE 1e6, eps 1e-6), fp16 KV, batch 1, "
                "computed by the oracle (single precision, the reference CPU path's arithmetic)",
        "weights": {"synth_seed": SEED, "sha256": dig},
        "prompt": [int(v) for v in prompt],
        "steps": steps,
        "oracle_seconds": round(time.time() - t0, 1),
        "threads": args.threads,
    }
    with open(args.out, "w") as f:
        json.dump(doc, f, indent=0)
        f.write("\n")
    print(f"wrote {args.out}: {len(steps)} steps, min gap {min(s['gap'] for s in steps):.4g}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
