#!/usr/bin/env python3
"""Decode throughput of the Qwen3-8B-shaped Q6_K decoder on one MI355X.

One step = one greedy decode step of every client through the whole model
(embedding, 36 layers, 151936-row output, greedy select), weights and KV cache
resident in HBM.  Prints one JSON line (see the repository's bench contract).

  value     batch-1 decode tokens/s after a 512-token prompt (fp16 KV)
  batch8    the same model with 8 clients (aggregate tokens/s); its matvecs
            run on the int8 matrix cores (activation limbs as the A operand)
  roofline  the dominant kernel: the fused gate|up Q6_K matvec (RMSNorm +
            SwiGLU epilogue, integer-limb dot products), 2 x 12288 x 4096
            weights = 82,575,360 B per launch, timed with HIP events on the
            library's stream while it walks all 36 layers (6.2 GB of distinct
            weights, so nothing is served from the 256 MB Infinity Cache);
            `traffic` is the HBM bytes per launch that the committed PMC
            summary (profiles/qmv_limb_gate_up_qwen3_8b_pmc.txt) measured
  cpu_baseline  the oracle (C restatement of the reference CPU path), one
            thread, one token through 1 and 4 layers + output, extrapolated
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import shutil
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from emufpga_amd import _lib  # noqa: E402
from emufpga_amd.device import Context  # noqa: E402
from emufpga_amd.gguf import GgufFile, row_bytes  # noqa: E402
from emufpga_amd.serve import (GRANITE_MOE_Q6K, QWEN3_8B_Q6K, SMOLLM2_135M_Q8, DenseConfig, Model,  # noqa: E402
                               Session)

METRIC = "decode tok/s at batch 1 and 8; achieved HBM GB/s vs 8 TB/s peak"
HBM_PEAK_GBS = 8000.0
KERNEL = "qmv_limb_kernel<LimbQ6KLM, S=1, D=1, dual, norm> (fused gate|up, 2 x 12288 x 4096 Q6_K, lane-major)"
PMC_SUMMARY = os.path.join(ROOT, "profiles", "qmv_limb_gate_up_qwen3_8b_pmc.txt")
COPY_BYTES = 256 << 20  # calibration copy for the PMC byte counters


def measured_traffic():
    """HBM bytes per gate|up launch from the committed PMC summary, if any."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_offsets(cfg):
    rb_h = row_bytes(cfg.encoding, cfg.hidden)
    rb_q = row_bytes(cfg.encoding, cfg.q_width)
    off_g = cfg.q_width * rb_h + 2 * cfg.kv_width * rb_h + cfg.hidden * rb_q
    off_u = off_g + cfg.ffn * rb_h
    return rb_h, off_g, off_u


def time_gate_up(ctx: Context, model: Model, rounds: int) -> tuple[float, int, int]:
    """Average duration (ms) of the fused gate|up matvec over all layers."""
    cfg = model.cfg
    rb_h, off_g, off_u = layer_offsets(cfg)
    rng = np.random.default_rng(0)
    x = ctx.upload(rng.normal(size=cfg.hidden).astype(np.float32))
    gain = ctx.upload(np.ones(cfg.hidden, np.float32))
    y = ctx.alloc(cfg.ffn * 4)
    # the copy the batch-1 decode step reads (the lane-major Q6_K layout)
    bases = [model.tensor_lane_major(_lib.EMU_T_LAYER, l)[0] for l in range(cfg.layers)]

    def launch(base):
        ctx.check(ctx.lib.emu_qmatvec_fused(ctx.h, cfg.encoding, C.c_void_p(base + off_g),
                                            C.c_void_p(base + off_u), cfg.ffn, cfg.hidden, x.ptr, 1,
                                            gain.ptr, cfg.eps, y.ptr, _lib.EMU_MV_LANE_MAJOR), "gate_up")

    for base in bases:  # warm
        launch(base)
    ctx.sync()
    ctx.event_record(0)
    for _ in range(rounds):
        for base in bases:
            launch(base)
    ctx.event_record(1)
    ms = ctx.event_elapsed(0, 1) / (rounds * len(bases))
    algo = 2 * cfg.ffn * rb_h
    return ms, algo, rounds * len(bases)


def cpu_baseline(model: Model, budget_s: float = 40.0) -> dict:
    """One batch-1 token through the oracle (single-threaded C restatement of
    the reference CPU path): the whole model when a one-layer probe says it
    fits the time budget, else 1 and 4 layers extrapolated."""
    import oracle

    cfg = model.cfg

    def weights(n_layers):
        return {
            "layers": np.concatenate([model.read_tensor(_lib.EMU_T_LAYER, l) for l in range(n_layers)]),
            "embed": model.read_tensor(_lib.EMU_T_EMBED),
            "output": model.read_tensor(_lib.EMU_T_OUTPUT),
            "attn_norm": model.read_tensor(_lib.EMU_T_ATTN_NORM, dtype=np.float32),
            "ffn_norm": model.read_tensor(_lib.EMU_T_FFN_NORM, dtype=np.float32),
            "q_norm": model.read_tensor(_lib.EMU_T_Q_NORM, dtype=np.float32),
            "k_norm": model.read_tensor(_lib.EMU_T_K_NORM, dtype=np.float32),
            "out_norm": model.read_tensor(_lib.EMU_T_OUT_NORM, dtype=np.float32),
        }

    ocfg = oracle.DenseCfg(hidden=cfg.hidden, heads=cfg.heads, kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                           ffn=cfg.ffn, vocab=cfg.vocab, layers=cfg.layers, context=4, rope_theta=cfg.rope_theta,
                           eps=cfg.eps, style=cfg.style, dtype=cfg.encoding, kv_f16=1, tied=0, qk_norm=1)

    def timed(w, limit):
        orc = oracle.DenseOracle(ocfg, w, 1)
        t0 = time.perf_counter()
        orc.step([17], layers_limit=limit)
        dt = time.perf_counter() - t0
        log(f"cpu oracle: {limit} layer(s) + output in {dt:.2f} s")
        return dt

    w4 = weights(4)
    t1, t4 = timed(w4, 1), timed(w4, 4)
    per_layer = (t4 - t1) / 3
    estimate = t1 + (cfg.layers - 1) * per_layer
    if estimate <= budget_s:
        del w4
        full = timed(weights(cfg.layers), cfg.layers)
        how = f"the whole {cfg.layers}-layer model timed: {full:.2f} s/token"
    else:
        full = estimate
        how = f"1 and 4 layers timed, per-layer {per_layer:.3f} s extrapolated to {cfg.layers} layers: {full:.2f} s/token"
    return {
        "value": round(1.0 / full, 5),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": ("one batch-1 token at position 0 through the embedding, the layers and the 151936-row output on "
                   "the single-threaded C restatement of the reference CPU path; " + how),
        "algorithmic_gbs": round(model.weight_bytes() / full / 1e9, 3),
    }


def load_leg(ctx) -> dict:
    """GGUF file -> HBM: a Qwen3-8B-width decoder cut to 4 layers (plus its
    full 151936-row embedding and output) written to a GGUF file, then every
    tensor placed by emu_model_load_gguf.  The file was just written, so its
    pages come from the page cache: this is the read + PCIe placement rate,
    not a cold-disk rate."""
    cfg = DenseConfig(**{**QWEN3_8B_Q6K.__dict__, "layers": 4})
    tmp = tempfile.mkdtemp(prefix="emu_gguf_")
    try:
        path = os.path.join(tmp, "qwen3_8b_4layers_q6k.gguf")
        src = Model(ctx, cfg)
        src.synth(4242)
        nbytes = src.save_gguf(path)
        src.close()
        with GgufFile(path) as f:
            dst = Model(ctx, cfg)
            t0 = time.perf_counter()
            dst.load_gguf(f)
            ctx.sync()
            dt = time.perf_counter() - t0
            tensor_bytes = sum(t.len for t in f.content.tensors)
        dst.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    gbs = tensor_bytes / dt / 1e9
    log(f"GGUF load: {tensor_bytes / 1e9:.2f} GB of tensors in {dt * 1e3:.1f} ms -> {gbs:.2f} GB/s")
    return {"value": round(gbs, 2), "unit": "GB/s", "tensor_bytes": tensor_bytes, "file_bytes": nbytes,
            "seconds": round(dt, 4),
            "workload": "Qwen3-8B-width Q6_K decoder cut to 4 layers, GGUF file in the page cache -> HBM"}


def smol_leg(ctx, rng, with_cpu: bool) -> dict:
    """The SmolLM2-135M-shaped Q8_0 decoder (30 layers, width 576, tied 49152-row
    output): batch 1, 32-token prompt, 256 timed greedy steps; beside it the
    oracle's single-threaded CPU decode of the same model."""
    cfg = SMOLLM2_135M_Q8
    model = Model(ctx, cfg)
    model.synth(135)
    sess = Session(model, 1, 512, kv_f16=True)
    prompt = rng.integers(0, cfg.vocab, size=(1, 32)).astype(np.uint32)
    sess.generate(prompt, 1 + 8)
    ctx.sync()
    steps = 256
    ms = sess.time_decode(steps)
    pos = int(sess.positions()[0])
    tok_s = steps / (ms / 1e3)
    log(f"SmolLM2 batch 1: {steps} steps in {ms:.2f} ms -> {tok_s:.1f} tok/s (context {pos - steps}..{pos})")
    out = {"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms / steps, 4),
           "context_at_timing": [pos - steps, pos],
           "workload": ("SmolLM2-135M-shaped decoder, Q8_0 linears and tied embedding (seeded synthetic), batch 1, "
                        "32-token prompt, 256 greedy decode steps, fp16 KV cache")}
    if with_cpu:
        import oracle

        ocfg = oracle.DenseCfg(hidden=cfg.hidden, heads=cfg.heads, kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                               ffn=cfg.ffn, vocab=cfg.vocab, layers=cfg.layers, context=16,
                               rope_theta=cfg.rope_theta, eps=cfg.eps, style=cfg.style, dtype=cfg.encoding,
                               kv_f16=1, tied=1, qk_norm=0)
        orc = oracle.DenseOracle(ocfg, model.host_weights(), 1)
        t0 = time.perf_counter()
        n = 8
        for i in range(n):
            orc.step([int(prompt[0, i])])
        dt = (time.perf_counter() - t0) / n
        log(f"SmolLM2 cpu oracle: {dt * 1e3:.1f} ms/token")
        out["cpu_baseline"] = {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": 1, "kind": "port",
                               "sample": f"{n} batch-1 decode steps at positions 0..{n - 1} on the single-threaded "
                                         "C restatement of the reference CPU path"}
    sess.close()
    model.close()
    return out


def moe_leg(ctx, rng) -> dict:
    """Granite-shaped MoE decode, 4 clients, 256-token prompts, 128 timed steps.
    The routing is the model's own router on seeded synthetic weights (close to
    uniform: about 21 distinct experts per layer for 4 x 8 routes, against
    about 18 under the Zipf(1.1) injection the MoE workload describes)."""
    cfg = GRANITE_MOE_Q6K
    model = Model(ctx, cfg)
    model.synth(20260202)
    sess = Session(model, 4, 1024, kv_f16=True)
    prompt = rng.integers(0, cfg.vocab, size=(4, 256)).astype(np.uint32)
    sess.generate(prompt, 1 + 8)
    ctx.sync()
    steps = 128
    ms = sess.time_decode(steps)
    ctx.sync()
    pos = int(sess.positions()[0])
    tok_s = 4 * steps / (ms / 1e3)
    log(f"granite MoE batch 4: {steps} steps in {ms:.2f} ms -> {tok_s:.1f} tok/s (context {pos - steps}..{pos})")
    sess.close()
    model.close()
    return {"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms / steps, 4),
            "context_at_timing": [pos - steps, pos], "clients": 4,
            "workload": ("Granite-shaped MoE decoder (24 layers, width 1024, 32 Q6_K SwiGLU experts of 512, "
                         "8 routed, tied 49155-row output), seeded synthetic weights, 256-token prompts, "
                         "routing by the model's own router")}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--context", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-batch8", action="store_true")
    ap.add_argument("--no-moe", action="store_true", help="skip the Granite MoE decode leg")
    ap.add_argument("--no-load", action="store_true", help="skip the GGUF -> HBM load leg")
    ap.add_argument("--no-smol", action="store_true", help="skip the SmolLM2 decode leg")
    ap.add_argument("--batch8-only", action="store_true",
                    help="only the 8-client decode, logged without the JSON line; for profiling")
    ap.add_argument("--moe-only", action="store_true",
                    help="only the Granite MoE decode leg, logged without the JSON line; for profiling")
    ap.add_argument("--roofline-rounds", type=int, default=8)
    ap.add_argument("--kernel-only", action="store_true",
                    help="only time the dominant kernel (the fused gate|up matvec over all layers); for profiling")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: this decode path runs "
              "on one GPU, whose share of a sharded model is the same kernels at their real shapes",
              file=sys.stderr)
        return 2

    cfg = QWEN3_8B_Q6K
    ctx = Context(0)
    cus, arch = ctx.device_info()
    log(f"device: {arch}, {cus} CUs")
    if args.moe_only:
        log(json.dumps(moe_leg(ctx, np.random.default_rng(43))))
        ctx.close()
        return 0
    t0 = time.perf_counter()
    model = Model(ctx, cfg)
    model.synth(20260101)
    weight_bytes = model.weight_bytes()
    log(f"synthesised {weight_bytes / 1e9:.3f} GB of Q6_K weights in {time.perf_counter() - t0:.1f} s")

    if args.kernel_only:
        ku_ms, ku_bytes, launches = time_gate_up(ctx, model, args.roofline_rounds)
        achieved = ku_bytes / (ku_ms / 1e3) / 1e9
        # One device-to-device copy of known size: its counter readings
        # calibrate the PMC byte counters (reads COPY_BYTES, writes COPY_BYTES).
        src, dst = ctx.alloc(COPY_BYTES), ctx.alloc(COPY_BYTES)
        ctx.check(ctx.lib.emu_memcpy_dtod(ctx.h, dst.ptr, src.ptr, COPY_BYTES), "calibration copy")
        ctx.sync()
        print(json.dumps({"kernel": KERNEL, "avg_launch_us": round(ku_ms * 1e3, 3), "launches": launches,
                          "achieved_gbs": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                          "calibration_copy_bytes": COPY_BYTES}), flush=True)
        return 0

    rng = np.random.default_rng(42)
    results = {}
    for batch in ([8] if args.batch8_only else [1] if args.no_batch8 else [1, 8]):
        sess = Session(model, batch, args.context, kv_f16=True)
        prompt = rng.integers(0, cfg.vocab, size=(batch, args.prompt)).astype(np.uint32)
        t0 = time.perf_counter()
        sess.generate(prompt, 1 + args.warmup)  # prefill + warmup decode steps, untimed
        log(f"batch {batch}: prompt {args.prompt} + {args.warmup} warmup steps in {time.perf_counter() - t0:.1f} s")
        ctx.sync()
        ms = sess.time_decode(args.steps)
        ctx.sync()
        pos = int(sess.positions()[0])
        results[batch] = (ms, pos)
        log(f"batch {batch}: {args.steps} steps in {ms:.2f} ms -> {batch * args.steps / (ms / 1e3):.1f} tok/s "
            f"(context {pos - args.steps}..{pos})")
        sess.close()

    if args.batch8_only:
        model.close()
        ctx.close()
        return 0
    ms1, pos1 = results[1]
    step_ms = ms1 / args.steps
    tok_s = args.steps / (ms1 / 1e3)
    ctx_mid = pos1 - args.steps // 2
    kv_bytes = cfg.layers * 2 * cfg.kv_width * 2 * ctx_mid  # fp16 K and V read per token
    step_gbs = (weight_bytes + kv_bytes) / (step_ms / 1e3) / 1e9

    ku_ms, ku_bytes, launches = time_gate_up(ctx, model, args.roofline_rounds)
    achieved = ku_bytes / (ku_ms / 1e3) / 1e9
    log(f"gate|up matvec: {ku_ms * 1e3:.2f} us avg over {launches} launches -> {achieved:.0f} GB/s")

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi8->i32 dots + f32",
        "data": "synthetic",
        "config": {
            "workload": (f"Qwen3-8B-shaped dense decoder, Q6_K weights (seeded N(0,0.02) synthetic), batch 1, "
                         f"{args.prompt}-token prompt then greedy decode, fp16 KV cache sized {args.context}"),
            "hidden": cfg.hidden, "layers": cfg.layers, "heads": cfg.heads, "kv_heads": cfg.kv_heads,
            "head_dim": cfg.head_dim, "ffn": cfg.ffn, "vocab": cfg.vocab, "encoding": "Q6_K",
            "context_at_timing": [pos1 - args.steps, pos1],
        },
        "step_hbm_gbs": round(step_gbs, 1),
        "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "weight_bytes_per_step": weight_bytes,
        "roofline": {
            "kernel": KERNEL,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "avg_launch_us": round(ku_ms * 1e3, 3),
            "algorithmic_bytes_per_launch": ku_bytes,
        },
    }
    if 8 in results:
        ms8, pos8 = results[8]
        kv8 = 8 * cfg.layers * 2 * cfg.kv_width * 2 * (pos8 - args.steps // 2)
        gbs8 = (weight_bytes + kv8) / (ms8 / args.steps / 1e3) / 1e9
        out["batch8"] = {"value": round(8 * args.steps / (ms8 / 1e3), 2), "unit": "tok/s",
                         "ms_per_step": round(ms8 / args.steps, 4), "context_at_timing": [pos8 - args.steps, pos8],
                         "step_hbm_gbs": round(gbs8, 1), "step_hbm_frac": round(gbs8 / HBM_PEAK_GBS, 4),
                         "matvec": "int8 MFMA (v_mfma_i32_32x32x16_i8), activation limbs as the A operand"}
    if not args.no_smol:
        out["smollm2_b1"] = smol_leg(ctx, rng, not args.no_cpu)
    if not args.no_moe:
        out["moe_granite_b4"] = moe_leg(ctx, rng)
    if not args.no_load:
        out["gguf_load"] = load_leg(ctx)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(model)
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
