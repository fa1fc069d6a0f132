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

from emufpga_amd import _lib, metrics  # noqa: E402
from emufpga_amd.device import Context  # noqa: E402
from emufpga_amd.gguf import GgufFile, row_bytes  # noqa: E402
from emufpga_amd.serve import (GEMMA4_MOE, GRANITE_MOE_Q6K, OLMOE_1B_7B, QWEN3_8B_Q6K, SMOLLM2_135M_Q8,  # noqa: E402
                               DenseConfig, Model, Session)

METRIC = "decode tok/s at batch 1 and 8; achieved HBM GB/s vs 8 TB/s peak"
HBM_PEAK_GBS = 8000.0
KERNEL = "qmv_limb_kernel<LimbQ6KLM, S=1, D=1, dual, norm> (fused gate|up, 2 x 12288 x 4096 Q6_K, lane-major)"
PMC_SUMMARY = os.path.join(ROOT, "profiles", "qmv_limb_gate_up_qwen3_8b_pmc.txt")
COPY_BYTES = 256 << 20  # calibration copy for the PMC byte counters
TRACE_DIR = ""  # --trace-dir
DIRECT = False  # --direct: every step launched kernel by kernel
DIRECT_TIMED = False  # --direct-timed: prompt and warmup from the graph, timed steps kernel by kernel
NO_ROOFLINE = False  # --no-roofline: skip the kernels' back-to-back roofline timings (profiling runs)
HBM_READ_BPS = None  # bytes/s a read-only stream gets from HBM on this device, measured once per run


def layer_times(sess: Session, reps: int = 5) -> np.ndarray:
    """Median over `reps` decode steps of each interval of a step (us): the
    embedding, every layer, the output matvec and selection."""
    return np.median(np.stack([sess.time_layers() for _ in range(reps)]), axis=0)


def layer_summary(us: np.ndarray) -> dict:
    layers = us[1:-1]
    return {"embed_us": round(float(us[0]), 2), "layer_mean_us": round(float(layers.mean()), 2),
            "layer_min_us": round(float(layers.min()), 2), "layer_max_us": round(float(layers.max()), 2),
            "output_us": round(float(us[-1]), 2),
            "how": "HIP events between each layer's kernels of one directly launched step, median of 5 steps"}


def session(model: Model, n: int, context: int) -> Session:
    """A decode session with an fp16 KV cache; with --direct its steps are
    launched kernel by kernel instead of replayed from a captured graph."""
    sess = Session(model, n, context, kv_f16=True)
    if DIRECT:
        sess.set_options(direct=True)
    return sess


def before_timing(sess: Session) -> None:
    """With --direct-timed, the steps from here on are launched kernel by
    kernel (a kernel tracer then sees the timed steps, at their context)."""
    if DIRECT_TIMED:
        sess.set_options(direct=True)


def calibration_copy(ctx) -> None:
    """One device-to-device copy of COPY_BYTES: its PMC byte-counter readings
    calibrate the counters (it reads and writes COPY_BYTES)."""
    src, dst = ctx.alloc(COPY_BYTES), ctx.alloc(COPY_BYTES)
    ctx.check(ctx.lib.emu_memcpy_dtod(ctx.h, dst.ptr, src.ptr, COPY_BYTES), "calibration copy")
    ctx.sync()
    src.free()
    dst.free()


STEP_PMC_SUMMARY = os.path.join(ROOT, "profiles", "decode_step_qwen3_8b_q6k_b1_pmc.txt")


def measured_step_bytes():
    """HBM bytes per batch-1 decode step from the committed FETCH_SIZE
    summary of a whole step, if any."""
    try:
        with open(STEP_PMC_SUMMARY) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_step:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


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
    # A run of large fills ahead of the first event keeps the GPU busy while
    # the host queues the timed launches, so the events time the kernels back
    # to back and not the host's launch rate (a ctypes call per launch).
    spacer = ctx.alloc(1 << 30)
    ctx.sync()
    for _ in range(8 + rounds * len(bases) // 16):
        spacer.zero()
    ctx.event_record(0)
    for _ in range(rounds):
        for base in bases:
            launch(base)
    ctx.event_record(1)
    ms = ctx.event_elapsed(0, 1) / (rounds * len(bases))
    algo = 2 * cfg.ffn * rb_h
    return ms, algo, rounds * len(bases)


def time_all_matvecs(ctx: Context, model: Model, rounds: int) -> tuple[float, int]:
    """Every batch-1 matvec of a decode step -- per layer q|k|v (RMSNorm
    fused), o (+ residual), gate|up (RMSNorm + SwiGLU fused), down
    (+ residual), then the 151936-row output (final RMSNorm fused) -- launched
    back to back over all 36 layers on the lane-major copies, as the step
    launches them: average time per step (ms) and algorithmic bytes per step."""
    cfg = model.cfg
    H, QW, KW, F = cfg.hidden, cfg.q_width, cfg.kv_width, cfg.ffn
    rb_h, rb_q, rb_f = row_bytes(cfg.encoding, H), row_bytes(cfg.encoding, QW), row_bytes(cfg.encoding, F)
    off_o = (QW + 2 * KW) * rb_h
    off_g = off_o + H * rb_q
    off_u = off_g + F * rb_h
    off_d = off_u + F * rb_h
    rng = np.random.default_rng(1)
    x = ctx.upload(rng.normal(size=H).astype(np.float32))
    xq = ctx.upload(rng.normal(size=QW).astype(np.float32))
    xf = ctx.upload(rng.normal(size=F).astype(np.float32) * 0.1)
    gain = ctx.upload(np.ones(H, np.float32))
    yqkv, ystate, yact, ylog = ctx.alloc((QW + 2 * KW) * 4), ctx.alloc(H * 4), ctx.alloc(F * 4), ctx.alloc(cfg.vocab * 4)
    ystate.zero()
    bases = [model.tensor_lane_major(_lib.EMU_T_LAYER, l)[0] for l in range(cfg.layers)]
    out_w = model.tensor_lane_major(_lib.EMU_T_OUTPUT)[0]
    lm, acc = _lib.EMU_MV_LANE_MAJOR, _lib.EMU_MV_LANE_MAJOR | _lib.EMU_MV_ACCUMULATE
    f = ctx.lib.emu_qmatvec_fused

    def step():
        for b in bases:
            ctx.check(f(ctx.h, cfg.encoding, C.c_void_p(b), None, QW + 2 * KW, H, x.ptr, 1, gain.ptr, cfg.eps,
                        yqkv.ptr, lm), "qkv")
            ctx.check(f(ctx.h, cfg.encoding, C.c_void_p(b + off_o), None, H, QW, xq.ptr, 1, None, 0.0, ystate.ptr,
                        acc), "o")
            ctx.check(f(ctx.h, cfg.encoding, C.c_void_p(b + off_g), C.c_void_p(b + off_u), F, H, x.ptr, 1, gain.ptr,
                        cfg.eps, yact.ptr, lm), "gate_up")
            ctx.check(f(ctx.h, cfg.encoding, C.c_void_p(b + off_d), None, H, F, xf.ptr, 1, None, 0.0, ystate.ptr,
                        acc), "down")
        ctx.check(f(ctx.h, cfg.encoding, C.c_void_p(out_w), None, cfg.vocab, H, x.ptr, 1, gain.ptr, cfg.eps,
                    ylog.ptr, lm), "output")

    step()  # warm
    spacer = ctx.alloc(1 << 30)
    ctx.sync()
    for _ in range(8 + rounds * (4 * cfg.layers + 1) // 12):
        spacer.zero()
    ctx.event_record(0)
    for _ in range(rounds):
        step()
    ctx.event_record(1)
    ms = ctx.event_elapsed(0, 1) / rounds
    per_step = cfg.layers * (off_d + H * rb_f) + cfg.vocab * rb_h
    return ms, per_step


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
    sess = session(model, 1, 512)
    prompt = rng.integers(0, cfg.vocab, size=(1, 32)).astype(np.uint32)
    sess.generate(prompt, 1 + 8)
    ctx.sync()
    steps = 256
    before_timing(sess)
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


def moe_layer_bytes(cfg, experts: float) -> float:
    """Algorithmic weight bytes one MoE layer reads in a step that routes to
    `experts` distinct experts: q|k|v and o, the f32 router, the Gemma form's
    scales and shared FFN, and the routed experts' gate, up and down rows."""
    H, QW, KW = cfg.hidden, cfg.q_width, cfg.kv_width
    attn = (QW + 2 * KW) * row_bytes(cfg.encoding, H) + H * row_bytes(cfg.encoding, QW)
    router = 4 * cfg.n_experts * H
    down_enc = cfg.expert_down_encoding if cfg.gemma else cfg.expert_encoding
    per_expert = 2 * cfg.expert_ff * row_bytes(cfg.expert_encoding, H) + H * row_bytes(down_enc, cfg.expert_ff)
    extra = 0
    if cfg.gemma:
        extra = 4 * (H + cfg.n_experts)
        if cfg.shared_ff:
            extra += 2 * cfg.shared_ff * row_bytes(cfg.encoding, H) + H * row_bytes(cfg.encoding, cfg.shared_ff)
    return attn + router + extra + experts * per_expert


def moe_cpu_baseline(model: Model, budget_layers: int = 2) -> dict:
    """One batch-1 token through the oracle's MoE decoder (single-threaded C
    restatement of the reference CPU path): 1 and 2 layers + the output
    timed, the per-layer cost extrapolated to the whole model."""
    import oracle

    c = model.cfg
    w = {"layers": np.concatenate([model.read_tensor(_lib.EMU_T_LAYER, l) for l in range(budget_layers)]),
         "embed": model.read_tensor(_lib.EMU_T_EMBED),
         "attn_norm": model.read_tensor(_lib.EMU_T_ATTN_NORM, dtype=np.float32),
         "ffn_norm": model.read_tensor(_lib.EMU_T_FFN_NORM, dtype=np.float32),
         "q_norm": model.read_tensor(_lib.EMU_T_Q_NORM, dtype=np.float32),
         "k_norm": model.read_tensor(_lib.EMU_T_K_NORM, dtype=np.float32),
         "out_norm": model.read_tensor(_lib.EMU_T_OUT_NORM, dtype=np.float32)}
    if not c.tied:
        w["output"] = model.read_tensor(_lib.EMU_T_OUTPUT)
    if c.gemma:
        w["ffn_norm2"] = model.read_tensor(_lib.EMU_T_FFN_NORM2, dtype=np.float32)
    ocfg = oracle.MoeModelCfg(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                              vocab=c.vocab, layers=c.layers, context=4, n_experts=c.n_experts,
                              experts_used=c.experts_used, expert_ff=c.expert_ff, rope_theta=c.rope_theta,
                              eps=c.eps, embed_scale=c.embed_scale, residual_scale=c.residual_scale,
                              logit_div=c.logit_div, score_mul=c.score_mul, dtype=c.encoding,
                              expert_dtype=c.expert_encoding, kv_f16=1, qk_norm=int(c.qk_norm),
                              rope_neox=int(c.rope_neox), untied=int(not c.tied), gemma=int(c.gemma),
                              expert_down_dtype=c.expert_down_encoding, shared_ff=c.shared_ff, window=c.window,
                              global_every=c.global_every, rope_theta_global=c.rope_theta_global,
                              softcap=c.logit_softcap)
    oracle.set_threads(1)

    def timed(limit):
        orc = oracle.MoeModelOracle(ocfg, w, 1)
        t0 = time.perf_counter()
        orc.step([17], layers_limit=limit)
        return time.perf_counter() - t0

    t1, t2 = timed(1), timed(2)
    per_layer = max(t2 - t1, 0.0)
    full = t1 + (c.layers - 1) * per_layer
    log(f"cpu oracle ({c.layers}-layer MoE): 1 layer + output {t1:.2f} s, 2 layers {t2:.2f} s -> {full:.2f} s/token")
    return {"value": round(1.0 / full, 5), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": (f"one batch-1 token at position 0 on the single-threaded C restatement of the reference "
                       f"CPU path with the model's own router: 1 and 2 layers + the output timed "
                       f"({t1:.2f} s, {t2:.2f} s), per-layer cost extrapolated to {c.layers} layers")}


# The expert layers of the three MoE workloads: (gate|up encoding, down encoding,
# experts, width, expert ff, routes per token, tokens, gate and up fused per
# expert, activation, Zipf exponent).
MOE_LAYERS = {
    "granite": (_lib.Q6_K, _lib.Q6_K, 32, 1024, 512, 8, 4, False, _lib.EMU_ACT_SILU, 1.1),
    "olmoe": (_lib.Q2_K, _lib.Q2_K, 64, 2048, 1024, 8, 8, False, _lib.EMU_ACT_SILU, 1.0),
    "gemma": (_lib.Q5_K, _lib.Q8_0, 128, 2816, 704, 8, 8, True, _lib.EMU_ACT_GELU_TANH, 1.2),
}
BLOCK = {_lib.Q6_K: (256, 210, (208,)), _lib.Q5_K: (256, 176, (0, 2)), _lib.Q2_K: (256, 84, (80, 82)),
         _lib.Q8_0: (32, 34, (0,))}


def random_blocks(enc: int, nblocks: int, rng) -> np.ndarray:
    """Random block bytes with moderate f16 scales at the format's scale offsets."""
    _, bb, scales = BLOCK[enc]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    for off in scales:
        raw[:, off:off + 2] = (rng.uniform(0.5, 1.0, nblocks) * 2.0 ** -10).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw


def moe_layer_leg(ctx, name: str, reps: int) -> dict:
    """One selected-expert FFN layer (emu_moe_ffn) of a MoE workload at its shape,
    with Zipf routes, called back to back: the expert kernels alone, for counters."""
    enc_in, enc_down, E, W, FF, K, T, fused, act, s = MOE_LAYERS[name]
    rng = np.random.default_rng(7)
    be_in, bb_in, _ = BLOCK[enc_in]
    be_ff, bb_ff, _ = BLOCK[enc_down]
    n_in = E * (2 if fused else 1) * FF * W // be_in
    bufs = [ctx.upload(random_blocks(enc_in, n_in, rng)),
            None if fused else ctx.upload(random_blocks(enc_in, n_in, rng)),
            ctx.upload(random_blocks(enc_down, E * W * FF // be_ff, rng))]
    bs = ctx.upload(rng.uniform(0.5, 2.0, E).astype(np.float32)) if fused else None
    desc = _lib.MoeDesc(enc_in, enc_down, bufs[0].addr, bufs[1].addr if bufs[1] else None, bufs[2].addr,
                        bs.addr if bs else None, E, W, FF, K, act)
    rank = rng.permutation(E) + 1
    logits = -s * np.log(rank)[None, :] - np.log(-np.log(rng.uniform(1e-9, 1.0, size=(T, E))))
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :K].astype(np.int32)
    wts = np.full((T, K), 1.0 / K, np.float32)
    distinct = len(set(ids.reshape(-1).tolist()))
    bx, bi, bw = ctx.upload(rng.normal(size=(T, W)).astype(np.float32)), ctx.upload(ids), ctx.upload(wts)
    ws_bytes = ctx.lib.emu_moe_workspace_bytes(T, K, W, FF)
    ws, out = ctx.alloc(ws_bytes), ctx.alloc(T * W * 4)

    def call():
        ctx.check(ctx.lib.emu_moe_ffn(ctx.h, C.byref(desc), bx.ptr, T, bi.ptr, bw.ptr, ws.ptr, ws_bytes, out.ptr),
                  "emu_moe_ffn")

    for _ in range(5):
        call()
    # queued behind fills so the events time the GPU, not the host's ctypes calls
    spacer = ctx.alloc(1 << 30)
    ctx.sync()
    for _ in range(4 + reps // 8):
        spacer.zero()
    ctx.event_record(0)
    for _ in range(reps):
        call()
    ctx.event_record(1)
    us = ctx.event_elapsed(0, 1) / reps * 1e3
    spacer.free()
    expert_bytes = 2 * FF * (W // be_in) * bb_in + W * (FF // be_ff) * bb_ff
    gbs = distinct * expert_bytes / (us * 1e-6) / 1e9
    log(f"{name} expert layer: {T} tokens x {K} routes, {distinct} distinct experts of {expert_bytes} B: "
        f"{us:.1f} us per call ({reps} calls) -> {gbs:.0f} GB/s")
    return {"layer": name, "us_per_call": round(us, 2), "distinct_experts": distinct,
            "expert_bytes": expert_bytes, "algorithmic_bytes": distinct * expert_bytes, "achieved_gbs": round(gbs, 1)}


# Matrix-pipe busy fraction of the expert kernels, from the committed counter
# summary (SQ_VALU_MFMA_BUSY_CYCLES over SQ_BUSY_CYCLES per SIMD).
MFMA_BUSY = {"granite": (0.056, 0.037), "olmoe": (0.169, 0.149), "gemma": (0.133, 0.086)}
MFMA_SOURCE = "profiles/moe_experts_layer_counters.txt"


def expert_roofline(ctx, name: str) -> dict:
    """The leg's selected-expert FFN layer (one emu_moe_ffn call: limbs, gate|up,
    limbs, down, combine) at the workload's shape and skew, called back to
    back, timed with HIP events: the experts' algorithmic bytes over the
    call's time, and the matrix pipe's busy fraction from the counters."""
    r = moe_layer_leg(ctx, name, 40)
    gu, dn = MFMA_BUSY[name]
    return {"kernel": "emu_moe_ffn (moe_mma_kernel gate|up and down on v_mfma_i32_32x32x16_i8, limbs, combine)",
            "bound": "hbm", "achieved": r["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4), "us_per_call": r["us_per_call"],
            "algorithmic_bytes_per_call": r["algorithmic_bytes"], "distinct_experts": r["distinct_experts"],
            "mfma_busy_gate_up": gu, "mfma_busy_down": dn, "mfma_busy_source": MFMA_SOURCE,
            "note": "layer called back to back: its experts' rows stay in the 256 MB Infinity Cache between calls"}


def moe_leg(ctx, rng, name: str, cfg, n_clients: int, prompt_len: int, steps: int, zipf_s: float,
            with_cpu: bool, seed: int) -> dict:
    """A mixture-of-experts decoder: n_clients concurrent sequences after
    prompt_len-token prompts, `steps` timed greedy steps with Zipf(zipf_s)
    routing (the workload's skew; the router is still read), the number of
    distinct experts per layer measured from the device route trace of a
    further untimed stretch, and the step's algorithmic HBM rate from it."""
    model = Model(ctx, cfg)
    t0 = time.perf_counter()
    model.synth(seed)
    ctx.sync()
    log(f"{name}: synthesised in {time.perf_counter() - t0:.1f} s")
    sess = session(model, n_clients, prompt_len + steps + 64 + 16)
    sess.route_zipf(zipf_s, seed)
    prompt = rng.integers(0, cfg.vocab, size=(n_clients, prompt_len)).astype(np.uint32)
    t0 = time.perf_counter()
    sess.generate(prompt, 1 + 8)
    ctx.sync()
    log(f"{name}: {prompt_len}-token prompts + 8 warmup steps in {time.perf_counter() - t0:.1f} s")
    before_timing(sess)
    ms = sess.time_decode(steps)
    ctx.sync()
    pos = int(sess.positions()[0])
    # distinct experts per (step, layer), from the routes of 32 further steps
    trace_steps = 32
    sess.route_trace(trace_steps)
    sess.time_decode(trace_steps)
    ctx.sync()
    us, traced = [], []
    for slot in range(trace_steps):
        ids, _ = sess.read_routes(slot)
        traced.append(ids)
        us += [len(set(ids[layer].reshape(-1).tolist())) for layer in range(cfg.layers)]
    mean_u = float(np.mean(us))
    lt = layer_times(sess)
    sess.close()
    if TRACE_DIR:
        os.makedirs(TRACE_DIR, exist_ok=True)
        with open(os.path.join(TRACE_DIR, f"{name}_routes.json"), "w") as f:
            f.write(metrics.routing_trace(name, traced, n_clients, cfg.n_experts).to_json())
        with open(os.path.join(TRACE_DIR, f"{name}_experts.json"), "w") as f:
            f.write(metrics.expert_trace(name, cfg, traced[0], lt[1:-1]).to_json())
    tok_s = n_clients * steps / (ms / 1e3)
    ctx_mid = pos - steps // 2
    kv_ctx = [min(ctx_mid, cfg.window) if cfg.gemma and cfg.window and (l + 1) % cfg.global_every else ctx_mid
              for l in range(cfg.layers)]
    kv_bytes = n_clients * sum(2 * cfg.kv_width * 2 * k for k in kv_ctx)
    step_bytes = cfg.layers * moe_layer_bytes(cfg, mean_u) + cfg.vocab * row_bytes(cfg.encoding, cfg.hidden) + kv_bytes
    gbs = step_bytes / (ms / steps / 1e3) / 1e9
    log(f"{name}: {steps} steps in {ms:.2f} ms -> {tok_s:.1f} tok/s, {mean_u:.1f} distinct experts per layer, "
        f"{step_bytes / 1e9:.3f} GB/step -> {gbs:.0f} GB/s (context {pos - steps}..{pos})")
    out = {"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms / steps, 4), "clients": n_clients,
           "context_at_timing": [pos - steps, pos], "routing": f"Zipf(s={zipf_s}) Gumbel-top-k, seed {seed}",
           "distinct_experts_per_layer": round(mean_u, 2), "algorithmic_bytes_per_step": int(step_bytes),
           "step_hbm_gbs": round(gbs, 1), "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           # Ps / Rp / eta of one traced step (its own routes) at the timed step time
           "layer_times": layer_summary(lt),
           "scan_metrics": metrics.step_metrics(cfg, n_clients, ms / steps / 1e3, traced[0],
                                                resident_bytes=model.resident_bytes(),
                                                hbm_bytes_per_s=HBM_READ_BPS).report(),
           "roofline": None if NO_ROOFLINE else expert_roofline(ctx, name)}
    if with_cpu:
        out["cpu_baseline"] = moe_cpu_baseline(model)
    model.close()
    return out


def moe_cached_leg(ctx, rng, cfg, n_clients: int, prompt_len: int, warm: int, steps: int, zipf_s: float,
                   seed: int, n_slots: int) -> dict:
    """The Gemma-4-style decoder with its experts behind the expert cache:
    every expert (layers x experts x expert bytes) in pinned host memory,
    n_slots of them in HBM, the cache's policy (admit on second use, the
    least recently used victim of the incoming expert's own layer first, as
    mmid-cache does: plain LRU over all layers evicts every expert before its
    next use once a step's ~1,000 distinct experts outnumber the slots) run
    on the device inside the captured step, admissions copied into their
    slots, other misses read by the expert kernels over PCIe.  The prompts
    run resident; the cache is attached after them, warmed for `warm` steps,
    then `steps` steps are timed with its counters read on either side."""
    from emufpga_amd.expert_cache import ExpertCache

    model = Model(ctx, cfg)
    model.synth(seed)
    down_enc = cfg.expert_down_encoding if cfg.gemma else cfg.expert_encoding
    eb = 2 * cfg.expert_ff * row_bytes(cfg.expert_encoding, cfg.hidden) + cfg.hidden * row_bytes(down_enc, cfg.expert_ff)
    cache = ExpertCache(ctx, cfg.layers, cfg.n_experts, eb, n_slots=n_slots, n_transient=1, layer_aware=True)
    t0 = time.perf_counter()
    cache.load_model(model)
    log(f"cached: {cfg.layers * cfg.n_experts} experts ({cfg.layers * cfg.n_experts * eb / 1e9:.1f} GB) into pinned "
        f"host memory in {time.perf_counter() - t0:.1f} s; {n_slots} HBM slots")
    host_gbs = ctx.host_read_rate()
    sess = session(model, n_clients, prompt_len + warm + steps + 16)
    sess.route_zipf(zipf_s, seed)
    prompt = rng.integers(0, cfg.vocab, size=(n_clients, prompt_len)).astype(np.uint32)
    sess.generate(prompt, 1)
    sess.attach_cache(cache)
    sess.time_decode(warm)
    s0 = cache.stats()
    before_timing(sess)
    ms = sess.time_decode(steps)
    s1 = cache.stats()
    sess.route_trace(2)
    sess.time_decode(2)
    routes = sess.read_routes(0)[0]
    pos = int(sess.positions()[0])
    sess.close()
    d = {k: s1[k] - s0[k] for k in ("hits", "misses", "loads", "evictions", "streamed", "bytes_uploaded",
                                     "bytes_streamed")}
    step_s = ms / steps / 1e3
    total = metrics.model_parameter_bytes(cfg)
    resident = total - cfg.layers * cfg.n_experts * eb + n_slots * eb
    sm = metrics.step_metrics(cfg, n_clients, step_s, routes, resident_bytes=resident, hbm_bytes_per_s=HBM_READ_BPS)
    streamed = d["bytes_streamed"] / steps
    if HBM_READ_BPS and host_gbs > 0:  # the misses come from host memory, the rest from HBM
        sm.storage_time = (sm.parameter_bytes_read - streamed) / HBM_READ_BPS + streamed / (host_gbs * 1e9)
    tok_s = n_clients * steps / (ms / 1e3)
    hit = d["hits"] / max(1, d["hits"] + d["misses"])
    log(f"cached: {steps} steps in {ms:.1f} ms -> {tok_s:.1f} tok/s; hit rate {hit:.3f}; per step "
        f"{d['bytes_uploaded'] / steps / 1e6:.1f} MB copied into slots, {streamed / 1e6:.1f} MB read from host "
        f"memory; host stream {host_gbs:.1f} GB/s")
    cache.close()
    model.close()
    return {"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms / steps, 4), "clients": n_clients,
            "context_at_timing": [pos - steps - 2, pos - 2], "hbm_slots": n_slots, "expert_bytes": eb,
            "Rp": round(resident / total, 4), "hit_rate": round(hit, 4),
            "bytes_copied_into_slots_per_step": int(d["bytes_uploaded"] / steps),
            "bytes_read_from_host_per_step": int(streamed), "host_read_gbs": round(host_gbs, 1),
            "cache_counters": d, "routing": f"Zipf(s={zipf_s}) Gumbel-top-k, seed {seed}",
            "note": ("Rp counts what the step reads from HBM: every non-expert parameter and the slots; the "
                     "synthetic model's own expert tensors, the source of the pinned host copies, also stay "
                     "in HBM here but the cached step reads none of them"),
            "scan_metrics": sm.report(),
            "workload": (f"Gemma-4-style MoE decoder as moe_gemma_b8, {n_clients} clients after {prompt_len}-token "
                         f"prompts; its {cfg.layers * cfg.n_experts} experts in pinned host memory behind "
                         f"{n_slots} HBM slots (admit on second use, layer-aware LRU), the policy on the device in the step; "
                         f"{warm} warm-up steps, then {steps} timed")}


def decode_256(ctx, model: Model, rng, batch: int, prompt: int, context: int) -> dict:
    """The workload's full decode: a `prompt`-token prompt, then 256 timed
    greedy steps (context prompt -> prompt + 256)."""
    sess = session(model, batch, context)
    toks = rng.integers(0, model.cfg.vocab, size=(batch, prompt)).astype(np.uint32)
    sess.generate(toks, 1)
    ctx.sync()
    ms = sess.time_decode(256)
    ctx.sync()
    pos = int(sess.positions()[0])
    sess.close()
    tok_s = batch * 256 / (ms / 1e3)
    log(f"batch {batch}: 256 steps from context {pos - 256} to {pos} in {ms:.1f} ms -> {tok_s:.1f} tok/s")
    return {"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms / 256, 4),
            "context_at_timing": [pos - 256, pos]}


def trace_summary(trace_dir: str, steps: int, by_grid: bool = False) -> str:
    """Kernel statistics of the last `steps` decode steps of a rocprofv3
    kernel trace (the steps counted by their embed_kernel dispatches from the
    end), so a profile of a run covers the timed steps at their context and
    not its prompt.  With by_grid each launch shape (grid size in threads)
    of a kernel is a line of its own."""
    import csv
    import glob
    from collections import defaultdict

    rows = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"]
                if by_grid:
                    grid = "x".join(r.get(f"Grid_Size_{a}", "") or "1" for a in "XYZ")
                    name = f"[grid {grid}] {name}"
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), name))
    rows.sort()
    embeds = [i for i, r in enumerate(rows) if "embed_kernel<" in r[2]]
    sel = rows[embeds[-steps]:]
    agg = defaultdict(list)
    for s0, e0, name in sel:
        agg[name].append((e0 - s0) / 1e3)
    tot = sum(sum(v) for v in agg.values())
    span = (sel[-1][1] - sel[0][0]) / 1e3
    out = [f"last {steps} decode steps: {len(sel)} dispatches, kernel time {tot:.1f} us, wall {span:.1f} us "
           f"({span / steps:.1f} us per step, launched one by one)",
           " share    calls    avg_us    min_us    max_us  kernel"]
    for name, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{100 * sum(v) / tot:5.1f}%  {len(v):7d}  {sum(v) / len(v):8.2f}  {min(v):8.2f}  {max(v):8.2f}  "
                   f"{name}")
    return "\n".join(out)


def pmc_summary(pmc_dir: str, match: str) -> str:
    """Median counter values per dispatch of the kernels whose name contains
    `match` in a rocprofv3 --pmc run, one line per (kernel, grid size)."""
    import csv
    import glob
    import statistics
    from collections import defaultdict

    per = defaultdict(lambda: defaultdict(float))  # (kernel, grid) -> (dispatch, counter) -> value
    for f in glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if match not in r["Kernel_Name"]:
                    continue
                grid = r.get("Grid_Size") or "x".join(r.get(f"Grid_Size_{a}", "") or "1" for a in "XYZ")
                per[(r["Kernel_Name"], grid)][(r["Dispatch_Id"], r["Counter_Name"])] += float(r["Counter_Value"])
    out = []
    for (name, grid), vals in sorted(per.items(), key=lambda kv: kv[0][1]):
        by_counter = defaultdict(list)
        for (_, counter), v in vals.items():
            by_counter[counter].append(v)
        n = max(len(v) for v in by_counter.values())
        cs = ", ".join(f"{c} {statistics.median(v):.0f}" for c, v in sorted(by_counter.items()))
        out.append(f"[grid {grid}] {n} dispatches: {cs}  {name}")
    return "\n".join(out)


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
    ap.add_argument("--no-gemma", action="store_true", help="skip the Gemma-4-style MoE leg")
    ap.add_argument("--no-cached", action="store_true", help="skip the Gemma-4-style leg behind the expert cache")
    ap.add_argument("--cached-only", action="store_true",
                    help="only the Gemma-4-style leg behind the expert cache, logged without the JSON line")
    ap.add_argument("--cache-slots", type=int, default=1536, help="HBM slots of the expert-cache leg")
    ap.add_argument("--trace-dir", default="",
                    help="write each MoE leg's routing trace (emufpga.moe-routing.v1) and one step's expert "
                         "trace (emufpga.serial-moe.v1) as JSON files here")
    ap.add_argument("--moe-prompt", type=int, default=0,
                    help="prompt length of the OLMoE / Gemma legs (default: the workloads' 1024 / 2048)")
    ap.add_argument("--batch8-only", action="store_true",
                    help="only the 8-client decode, logged without the JSON line; for profiling")
    ap.add_argument("--moe-only", nargs="?", const="granite", choices=["granite", "olmoe", "gemma"],
                    help="only one MoE decode leg (default granite), logged without the JSON line; for profiling")
    ap.add_argument("--moe-layer", choices=sorted(MOE_LAYERS),
                    help="only one MoE workload's selected-expert FFN layer, called back to back; for counters")
    ap.add_argument("--smol-only", action="store_true",
                    help="only the SmolLM2 decode leg, logged without the JSON line; for profiling")
    ap.add_argument("--roofline-rounds", type=int, default=8)
    ap.add_argument("--direct", action="store_true",
                    help="launch each decode step's kernels one by one instead of replaying a captured graph "
                         "(same kernels and results); for counter passes, which fail on graph launches")
    ap.add_argument("--trace-summary", nargs=2, metavar=("TRACE_DIR", "STEPS"),
                    help="print the kernel statistics of the last STEPS decode steps of a rocprofv3 kernel trace "
                         "(no GPU used)")
    ap.add_argument("--by-grid", action="store_true", help="--trace-summary: a line per launch shape")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("PMC_DIR", "MATCH"),
                    help="print median counters per dispatch of the kernels matching MATCH in a rocprofv3 --pmc run "
                         "(no GPU used)")
    ap.add_argument("--no-roofline", action="store_true",
                    help="skip the back-to-back kernel timings (gate|up, all matvecs, expert layers), so a kernel "
                         "trace holds the decode steps only")
    ap.add_argument("--direct-timed", action="store_true",
                    help="replay the prompt and warmup steps from the captured graph, launch the timed steps "
                         "kernel by kernel; for kernel traces of the timed steps at their context")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only time the dominant kernel (the fused gate|up matvec over all layers); for profiling")
    args = ap.parse_args()
    if args.trace_summary:
        print(trace_summary(args.trace_summary[0], int(args.trace_summary[1]), args.by_grid))
        return 0
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary[0], args.pmc_summary[1]))
        return 0
    global TRACE_DIR, DIRECT, DIRECT_TIMED, HBM_READ_BPS, NO_ROOFLINE
    TRACE_DIR = args.trace_dir
    DIRECT = args.direct
    DIRECT_TIMED = args.direct_timed
    NO_ROOFLINE = args.no_roofline
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: this decode path runs "
              "on one GPU, whose share of a sharded model is the same kernels at their real shapes",
              file=sys.stderr)
        return 2

    cfg = QWEN3_8B_Q6K
    ctx = Context(0)
    cus, arch = ctx.device_info()
    log(f"device: {arch}, {cus} CUs")
    if args.moe_layer:
        log(json.dumps(moe_layer_leg(ctx, args.moe_layer, args.steps)))
        ctx.close()
        return 0
    if args.cached_only:
        HBM_READ_BPS = ctx.hbm_read_rate() * 1e9
        log(json.dumps(moe_cached_leg(ctx, np.random.default_rng(44), GEMMA4_MOE, 8, args.moe_prompt or 2048, 32,
                                      args.steps, 1.2, 20260404, args.cache_slots)))
        ctx.close()
        return 0
    if args.smol_only:
        calibration_copy(ctx)
        log(json.dumps(smol_leg(ctx, np.random.default_rng(42), False)))
        ctx.close()
        return 0
    if args.moe_only:
        leg = {"granite": (GRANITE_MOE_Q6K, 4, 256, 128, 1.1, 20260202),
               "olmoe": (OLMOE_1B_7B, 8, args.moe_prompt or 1024, args.steps, 1.0, 20260303),
               "gemma": (GEMMA4_MOE, 8, args.moe_prompt or 2048, args.steps, 1.2, 20260404)}[args.moe_only]
        m_cfg, n, prompt, steps, zs, seed = leg
        calibration_copy(ctx)
        log(json.dumps(moe_leg(ctx, np.random.default_rng(43), args.moe_only, m_cfg, n, prompt, steps, zs, False,
                               seed)))
        ctx.close()
        return 0
    t0 = time.perf_counter()
    model = Model(ctx, cfg)
    model.synth(20260101)
    weight_bytes = model.weight_bytes()
    resident_bytes = model.resident_bytes()
    log(f"synthesised {weight_bytes / 1e9:.3f} GB of Q6_K weights in {time.perf_counter() - t0:.1f} s")
    HBM_READ_BPS = ctx.hbm_read_rate() * 1e9
    log(f"HBM read stream (2 GiB, non-temporal): {HBM_READ_BPS / 1e9:.0f} GB/s")

    if args.kernel_only:
        ku_ms, ku_bytes, launches = time_gate_up(ctx, model, args.roofline_rounds)
        achieved = ku_bytes / (ku_ms / 1e3) / 1e9
        calibration_copy(ctx)
        print(json.dumps({"kernel": KERNEL, "avg_launch_us": round(ku_ms * 1e3, 3), "launches": launches,
                          "achieved_gbs": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                          "calibration_copy_bytes": COPY_BYTES}), flush=True)
        return 0

    rng = np.random.default_rng(42)
    results = {}
    for batch in ([8] if args.batch8_only else [1] if args.no_batch8 else [1, 8]):
        sess = session(model, batch, args.context)
        prompt = rng.integers(0, cfg.vocab, size=(batch, args.prompt)).astype(np.uint32)
        t0 = time.perf_counter()
        sess.generate(prompt, 1 + args.warmup)  # prefill + warmup decode steps, untimed
        log(f"batch {batch}: prompt {args.prompt} + {args.warmup} warmup steps in {time.perf_counter() - t0:.1f} s")
        ctx.sync()
        before_timing(sess)
        ms = sess.time_decode(args.steps)
        ctx.sync()
        pos = int(sess.positions()[0])
        results[batch] = (ms, pos, layer_times(sess))
        log(f"batch {batch}: {args.steps} steps in {ms:.2f} ms -> {batch * args.steps / (ms / 1e3):.1f} tok/s "
            f"(context {pos - args.steps}..{pos})")
        sess.close()

    if args.batch8_only:
        model.close()
        ctx.close()
        return 0
    ms1, pos1, lt1 = results[1]
    step_ms = ms1 / args.steps
    tok_s = args.steps / (ms1 / 1e3)
    ctx_mid = pos1 - args.steps // 2
    kv_bytes = cfg.layers * 2 * cfg.kv_width * 2 * ctx_mid  # fp16 K and V read per token
    step_gbs = (weight_bytes + kv_bytes) / (step_ms / 1e3) / 1e9

    if args.no_roofline:
        log(f"batch 1: {tok_s:.1f} tok/s (no roofline timings: profiling run)")
        model.close()
        ctx.close()
        return 0
    ku_ms, ku_bytes, launches = time_gate_up(ctx, model, args.roofline_rounds)
    achieved = ku_bytes / (ku_ms / 1e3) / 1e9
    log(f"gate|up matvec: {ku_ms * 1e3:.2f} us avg over {launches} launches -> {achieved:.0f} GB/s")
    am_ms, am_bytes = time_all_matvecs(ctx, model, 4)
    am_gbs = am_bytes / (am_ms / 1e3) / 1e9
    log(f"all batch-1 matvecs of a step back to back: {am_ms * 1e3:.1f} us for {am_bytes / 1e9:.3f} GB -> "
        f"{am_gbs:.0f} GB/s")

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
        "hbm_read_gbs": round(HBM_READ_BPS / 1e9, 1),
        "layer_times": layer_summary(lt1),
        # resident: every HBM copy of the weights (GGUF order, lane-major, operand order)
        "scan_metrics": {**metrics.step_metrics(cfg, 1, step_ms / 1e3, resident_bytes=resident_bytes,
                                                hbm_bytes_per_s=HBM_READ_BPS, read_bytes=measured_step_bytes()
                                                ).report(),
                         "parameter_bytes_read_source": os.path.relpath(STEP_PMC_SUMMARY, ROOT)
                         if measured_step_bytes() else "algorithmic", "algorithmic_bytes_read": weight_bytes},
        "weight_bytes_per_step": weight_bytes,
        "roofline": {
            "kernel": KERNEL,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            # not measured in this run: the committed counter summary's figure
            "traffic_source": f"{os.path.relpath(PMC_SUMMARY, os.path.dirname(os.path.abspath(__file__)))} "
                              "(rocprofv3 FETCH_SIZE + WRITE_SIZE passes, each scaled by a 256 MiB copy's reading)",
            "avg_launch_us": round(ku_ms * 1e3, 3),
            "algorithmic_bytes_per_launch": ku_bytes,
            # every matvec of a batch-1 step (145 launches), bytes over their summed time
            "all_matvecs_b1": {"achieved": round(am_gbs, 1), "frac": round(am_gbs / HBM_PEAK_GBS, 4),
                               "bytes_per_step": am_bytes, "us_per_step": round(am_ms * 1e3, 1),
                               "how": "q|k|v, o, gate|up, down of 36 layers and the output matvec launched back "
                                      "to back on the lane-major copies, HIP events over 4 rounds"},
        },
    }
    if 8 in results:
        ms8, pos8, lt8 = results[8]
        kv8 = 8 * cfg.layers * 2 * cfg.kv_width * 2 * (pos8 - args.steps // 2)
        gbs8 = (weight_bytes + kv8) / (ms8 / args.steps / 1e3) / 1e9
        out["batch8"] = {"value": round(8 * args.steps / (ms8 / 1e3), 2), "unit": "tok/s",
                         "ms_per_step": round(ms8 / args.steps, 4), "context_at_timing": [pos8 - args.steps, pos8],
                         "step_hbm_gbs": round(gbs8, 1), "step_hbm_frac": round(gbs8 / HBM_PEAK_GBS, 4),
                         "layer_times": layer_summary(lt8),
                         "scan_metrics": metrics.step_metrics(cfg, 8, ms8 / args.steps / 1e3,
                                                              resident_bytes=resident_bytes,
                                                              hbm_bytes_per_s=HBM_READ_BPS).report(),
                         "matvec": "int8 MFMA (v_mfma_i32_32x32x16_i8), activation limbs as the A operand"}
    if not args.no_smol:
        out["smollm2_b1"] = smol_leg(ctx, rng, not args.no_cpu)
    out["decode_256_steps_b1"] = decode_256(ctx, model, rng, 1, args.prompt, args.context)
    if not args.no_batch8:
        out["decode_256_steps_b8"] = decode_256(ctx, model, rng, 8, args.prompt, args.context)
    if not args.no_moe:
        wl = "seeded synthetic weights; routing Zipf(s) injected (Gumbel-top-k), the router still read"
        leg = moe_leg(ctx, rng, "granite", GRANITE_MOE_Q6K, 4, 256, 128, 1.1, not args.no_cpu, 20260202)
        leg["workload"] = ("Granite-shaped MoE decoder (24 layers, width 1024, 16/8 heads of 64, 32 Q6_K SwiGLU "
                           "experts of 512, 8 routed, tied 49155-row output), 4 clients, 256-token prompts; " + wl)
        out["moe_granite_b4"] = leg
        leg = moe_leg(ctx, rng, "olmoe", OLMOE_1B_7B, 8, args.moe_prompt or 1024, args.steps, 1.0,
                      not args.no_cpu, 20260303)
        leg["workload"] = ("OLMoE-1B-7B-shaped decoder (16 layers, width 2048, 16 heads of 128 with QK-norm, "
                           "Q6_K attention and untied 50304-row output, 64 Q2_K SwiGLU experts of 1024, 8 "
                           "routed), 8 clients; " + wl)
        out["moe_olmoe_b8"] = leg
        if not args.no_gemma:
            leg = moe_leg(ctx, rng, "gemma", GEMMA4_MOE, 8, args.moe_prompt or 2048, args.steps, 1.2,
                          not args.no_cpu, 20260404)
            leg["workload"] = ("Gemma-4-style MoE decoder (30 layers, width 2816, 16/8 heads of 256 with QK-norm, "
                               "5 sliding-window (1024) : 1 global layers, 128 Q5_K GeGLU experts of 704 with Q8_0 "
                               "downs and per-expert scales, 8 routed, shared GeGLU FFN of 2048, Q6_K attention "
                               "and tied 262144-row output soft-capped at 30), 8 clients; " + wl)
            out["moe_gemma_b8"] = leg
            if not args.no_cached:
                out["moe_gemma_cached_b8"] = moe_cached_leg(ctx, rng, GEMMA4_MOE, 8, args.moe_prompt or 2048, 32,
                                                            32, 1.2, 20260404, args.cache_slots)
    if not args.no_load:
        out["gguf_load"] = load_leg(ctx)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(model)
        # vs_baseline stays null: it is reserved for a published number of this metric
        out["vs_cpu_baseline"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
