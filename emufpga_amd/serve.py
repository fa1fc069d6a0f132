"""Serve API: a dense decoder resident in HBM and client sessions.

Mirrors components/serve/crates/spm-batch: ``Session.decode_step`` is
decode_step (src/step.rs:19-39) for every client at once, each client at its
own position with its own KV cache (Client, src/session.rs:13-38), and
``Session.generate`` is the caller loop of examples/serve-demo.rs:62-91
(prefill one prompt token per step, then greedy decode), run device-resident.

``Model.from_gguf`` builds the model from a GGUF file: the configuration from
the file's llama.cpp metadata keys and tensor shapes, every tensor uploaded to
its place in the model's HBM residency (emu_model_load_gguf).
"""
from __future__ import annotations

import ctypes as C
import sys
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import (EMU_STYLE_GRANITE, EMU_STYLE_QWEN3, EMU_STYLE_SMOL, EMU_T_ATTN_NORM, EMU_T_EMBED, EMU_T_FFN_NORM,
                   EMU_T_FFN_NORM2, EMU_T_K_NORM, EMU_T_LAYER, EMU_T_OUT_NORM, EMU_T_OUTPUT, EMU_T_Q_NORM, Q6_K,
                   Q8_0, ModelConfig)
from .device import Context
from .gguf import F32, MT_F32, MT_STR, MT_U32, GgufFile, row_bytes, write


@dataclass(frozen=True)
class DenseConfig:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    layers: int
    rope_theta: float
    eps: float
    style: int
    encoding: int
    tied: bool
    qk_norm: bool
    # mixture-of-experts layers (EMU_STYLE_GRANITE); zero keeps the dense forms
    n_experts: int = 0
    experts_used: int = 0
    expert_ff: int = 0
    expert_encoding: int = 0
    embed_scale: float = 0.0
    residual_scale: float = 0.0
    logit_div: float = 0.0
    score_mul: float = 0.0
    # OLMoE / Gemma-4 forms of the mixture-of-experts decoder (emu_model_config)
    rope_neox: bool = False
    gemma: bool = False
    expert_down_encoding: int = 0
    shared_ff: int = 0
    window: int = 0
    global_every: int = 0
    rope_theta_global: float = 0.0
    logit_softcap: float = 0.0

    def native(self) -> ModelConfig:
        return ModelConfig(self.hidden, self.heads, self.kv_heads, self.head_dim, self.ffn, self.vocab,
                           self.layers, self.rope_theta, self.eps, self.style, self.encoding,
                           int(self.tied), int(self.qk_norm), self.n_experts, self.experts_used, self.expert_ff,
                           self.expert_encoding, self.embed_scale, self.residual_scale, self.logit_div,
                           self.score_mul, int(self.rope_neox), int(self.gemma), self.expert_down_encoding,
                           self.shared_ff, self.window, self.global_every, self.rope_theta_global,
                           self.logit_softcap)

    @property
    def q_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim


# Qwen3-8B shape (spm-qwen3-slice/src/model.rs:10-12, attention.rs:1-3, math.rs:4, attention.rs:18)
QWEN3_8B_Q6K = DenseConfig(4096, 32, 8, 128, 12288, 151936, 36, 1e6, 1e-6, EMU_STYLE_QWEN3, Q6_K, False, True)
# SmolLM2-135M shape (spm-smol/src/config.rs:24-45), linears + tied embedding in Q8_0
SMOLLM2_135M_Q8 = DenseConfig(576, 9, 3, 64, 1536, 49152, 30, 1e5, 1e-5, EMU_STYLE_SMOL, Q8_0, True, False)
# Granite MoE shape (spm-granite-moe/src/model.rs:16-17, attention.rs:8-10, shape.rs:16-21): 24 layers of
# width 1024, 16/8 heads of 64, 32 Q6_K SwiGLU experts of width 512 with 8 routed, f32 router,
# tied 49155-row output; x12 embeddings, x0.22 residuals, logits / 6, scores x 1/64, theta 1.5e6.
GRANITE_MOE_Q6K = DenseConfig(1024, 16, 8, 64, 0, 49155, 24, 1.5e6, 1e-6, EMU_STYLE_GRANITE, Q6_K, True, False,
                              n_experts=32, experts_used=8, expert_ff=512, expert_encoding=Q6_K, embed_scale=12.0,
                              residual_scale=0.22, logit_div=6.0, score_mul=0.015625)


# OLMoE-1B-7B shape (spm-granite-moe/src/shape.rs:16-21: width 2048, FF 1024, 64 experts, top 8): 16 layers,
# 16 heads of 128 (no GQA), per-head QK-norm, half-split RoPE at 1e4, Q6_K attention and untied 50304-row
# output, Q2_K SwiGLU experts, f32 router, scores x 1/sqrt(128).
OLMOE_1B_7B = DenseConfig(2048, 16, 16, 128, 0, 50304, 16, 1e4, 1e-5, EMU_STYLE_GRANITE, Q6_K, False, True,
                          n_experts=64, experts_used=8, expert_ff=1024, expert_encoding=_lib.Q2_K,
                          score_mul=float(np.float32(1.0 / np.sqrt(128.0))), rope_neox=True)
# Gemma-4-style MoE shape (gemma_smoke.rs:13-20: width 2816, FF 704, 8 routed, Q5_K gate|up, Q8_0 down): 30
# layers, 16 heads / 8 KV heads of 256, per-head QK-norm, five sliding-window (1024) layers to one global,
# RoPE 1e4 local / 1e6 global, 128 experts plus a shared dense GeGLU FFN of 2048 (a size chosen here: the
# workload leaves it open), Q6_K attention, shared FFN and tied 262144-row output, embeddings x sqrt(2816),
# scores x 1/16, logits soft-capped at 30.
GEMMA4_MOE = DenseConfig(2816, 16, 8, 256, 0, 262144, 30, 1e4, 1e-6, EMU_STYLE_GRANITE, Q6_K, True, True,
                         n_experts=128, experts_used=8, expert_ff=704, expert_encoding=_lib.Q5_K,
                         embed_scale=float(np.float32(np.sqrt(2816.0))), score_mul=1.0 / 16, rope_neox=True,
                         gemma=True, expert_down_encoding=Q8_0, shared_ff=2048, window=1024, global_every=6,
                         rope_theta_global=1e6, logit_softcap=30.0)

_STYLES = {"qwen3": EMU_STYLE_QWEN3, "llama": EMU_STYLE_SMOL, "granitemoe": EMU_STYLE_GRANITE}


def config_from_gguf(f: GgufFile) -> DenseConfig:
    """The decoder shape a GGUF file declares: general.architecture picks the
    style (qwen3, llama for the SmolLM2 path, granitemoe), {arch}.* keys give
    the sizes and constants, token_embd gives the vocabulary and encoding,
    and the presence of output / attn_q_norm tensors decides tied and qk_norm."""
    meta = f.content.metadata
    arch = meta.get("general.architecture", "")
    if arch not in _STYLES:
        raise ValueError(f"unsupported architecture {arch!r}")
    names = {t.name for t in f.content.tensors}

    def num(key, default=None):
        try:
            return f.number(f"{arch}.{key}")
        except KeyError:
            if default is None:
                raise ValueError(f"GGUF metadata {arch}.{key} is missing") from None
            return default

    embd = f.tensor("token_embd.weight")
    hidden, heads = int(num("embedding_length")), int(num("attention.head_count"))
    style = _STYLES[arch]
    moe = style == EMU_STYLE_GRANITE
    kw = {}
    if moe:
        kw = dict(n_experts=int(num("expert_count")), experts_used=int(num("expert_used_count")),
                  expert_ff=int(num("expert_feed_forward_length", num("feed_forward_length", 0))),
                  expert_encoding=f.tensor("blk.0.ffn_gate_exps.weight").dtype,
                  embed_scale=float(num("embedding_scale", 1.0)), residual_scale=float(num("residual_scale", 1.0)),
                  logit_div=float(num("logit_scale", 1.0)), score_mul=float(num("attention.scale", 0.0)))
    return DenseConfig(hidden=hidden, heads=heads, kv_heads=int(num("attention.head_count_kv", heads)),
                       head_dim=int(num("attention.key_length", hidden // heads)),
                       ffn=0 if moe else int(num("feed_forward_length")), vocab=int(embd.dims[1]),
                       layers=int(num("block_count")), rope_theta=float(num("rope.freq_base", 10000.0)),
                       eps=float(num("attention.layer_norm_rms_epsilon")), style=style, encoding=embd.dtype,
                       tied="output.weight" not in names, qk_norm="blk.0.attn_q_norm.weight" in names, **kw)


def gguf_tensors(cfg: DenseConfig, w: dict):
    """A model's weights (Model.host_weights()) as GGUF (metadata, tensors)
    under llama.cpp's names, shapes in GGML order (row length first): the
    inverse of config_from_gguf and emu_model_load_gguf."""
    H, QW, KW = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    enc, moe = cfg.encoding, cfg.style == _lib.EMU_STYLE_GRANITE
    rb_h, rb_q = row_bytes(enc, H), row_bytes(enc, QW)
    t = [("token_embd.weight", (H, cfg.vocab), enc, w["embed"].data)]
    if not cfg.tied:
        t.append(("output.weight", (H, cfg.vocab), enc, w["output"].data))
    t.append(("output_norm.weight", (H,), F32, w["out_norm"].data))
    layers = w["layers"]
    if moe:
        rb_he, rb_fe = row_bytes(cfg.expert_encoding, H), row_bytes(cfg.expert_encoding, cfg.expert_ff)
        off_o = (QW + 2 * KW) * rb_h
        off_r = (off_o + H * rb_q + 15) // 16 * 16
        ge = cfg.n_experts * cfg.expert_ff * rb_he
        de = cfg.n_experts * H * rb_fe
        lb = (off_r + 4 * cfg.n_experts * H + 2 * ge + de + 15) // 16 * 16
    else:
        rb_f = row_bytes(enc, cfg.ffn)
        lb = (QW + 2 * KW) * rb_h + H * rb_q + 2 * cfg.ffn * rb_h + H * rb_f
    assert layers.size == lb * cfg.layers
    for l in range(cfg.layers):
        blob = layers[l * lb:(l + 1) * lb]
        at = 0

        def take(name, dims, dtype, n):
            nonlocal at
            t.append((f"blk.{l}.{name}.weight", dims, dtype, blob[at:at + n].data))
            at += n

        t.append((f"blk.{l}.attn_norm.weight", (H,), F32, w["attn_norm"][l * H:(l + 1) * H].data))
        t.append((f"blk.{l}.ffn_norm.weight", (H,), F32, w["ffn_norm"][l * H:(l + 1) * H].data))
        if cfg.qk_norm:
            d = cfg.head_dim
            t.append((f"blk.{l}.attn_q_norm.weight", (d,), F32, w["q_norm"][l * d:(l + 1) * d].data))
            t.append((f"blk.{l}.attn_k_norm.weight", (d,), F32, w["k_norm"][l * d:(l + 1) * d].data))
        take("attn_q", (H, QW), enc, QW * rb_h)
        take("attn_k", (H, KW), enc, KW * rb_h)
        take("attn_v", (H, KW), enc, KW * rb_h)
        take("attn_output", (QW, H), enc, H * rb_q)
        if moe:
            at = off_r
            take("ffn_gate_inp", (H, cfg.n_experts), F32, 4 * cfg.n_experts * H)
            take("ffn_gate_exps", (H, cfg.expert_ff, cfg.n_experts), cfg.expert_encoding, ge)
            take("ffn_up_exps", (H, cfg.expert_ff, cfg.n_experts), cfg.expert_encoding, ge)
            take("ffn_down_exps", (cfg.expert_ff, H, cfg.n_experts), cfg.expert_encoding, de)
        else:
            take("ffn_gate", (H, cfg.ffn), enc, cfg.ffn * rb_h)
            take("ffn_up", (H, cfg.ffn), enc, cfg.ffn * rb_h)
            take("ffn_down", (cfg.ffn, H), enc, H * row_bytes(enc, cfg.ffn))
    arch = {v: k for k, v in _STYLES.items()}[cfg.style]
    u32 = [("embedding_length", H), ("block_count", cfg.layers), ("attention.head_count", cfg.heads),
           ("attention.head_count_kv", cfg.kv_heads), ("attention.key_length", cfg.head_dim)]
    f32 = [("rope.freq_base", cfg.rope_theta), ("attention.layer_norm_rms_epsilon", cfg.eps)]
    if moe:
        u32 += [("expert_count", cfg.n_experts), ("expert_used_count", cfg.experts_used),
                ("expert_feed_forward_length", cfg.expert_ff)]
        f32 += [("embedding_scale", cfg.embed_scale), ("residual_scale", cfg.residual_scale),
                ("logit_scale", cfg.logit_div), ("attention.scale", cfg.score_mul)]
    else:
        u32.append(("feed_forward_length", cfg.ffn))
    meta = [("general.architecture", MT_STR, arch), ("general.alignment", MT_U32, 64)]
    meta += [(f"{arch}.{k}", MT_U32, v) for k, v in u32] + [(f"{arch}.{k}", MT_F32, v) for k, v in f32]
    return meta, t


class Model:
    """Weights of a dense decoder in one HBM allocation (emu_model)."""

    def __init__(self, ctx: Context, cfg: DenseConfig):
        self.ctx, self.cfg = ctx, cfg
        h = C.c_void_p()
        native = cfg.native()
        ctx.check(ctx.lib.emu_model_create(ctx.h, C.byref(native), C.byref(h)), "emu_model_create")
        self.h = h

    def close(self) -> None:
        if self.h is not None and self.ctx.live:
            self.ctx.lib.emu_model_destroy(self.h)
        self.h = None

    def __del__(self):  # pragma: no cover
        if not sys.is_finalizing():
            try:
                self.close()
            except Exception:
                pass

    def synth(self, seed: int) -> None:
        self.ctx.check(self.ctx.lib.emu_model_synth(self.h, seed), "emu_model_synth")

    def load_gguf(self, f: GgufFile) -> None:
        """Every tensor from an open GGUF file, by name, into HBM."""
        st = self.ctx.lib.emu_model_load_gguf(self.h, f.h)
        self.ctx.check(st, "emu_model_load_gguf")

    def save_gguf(self, path) -> int:
        """Write every tensor to a GGUF file that from_gguf reads back."""
        meta, tensors = gguf_tensors(self.cfg, self.host_weights())
        return write(path, meta, tensors, align=64)

    @classmethod
    def from_gguf(cls, ctx: Context, path, cfg: DenseConfig | None = None) -> "Model":
        with GgufFile(path) as f:
            m = cls(ctx, cfg or config_from_gguf(f))
            m.load_gguf(f)
        return m

    def tensor(self, kind: int, layer: int = 0) -> tuple[int, int]:
        p, n = C.c_void_p(), C.c_size_t()
        self.ctx.check(self.ctx.lib.emu_model_tensor(self.h, kind, layer, C.byref(p), C.byref(n)),
                       "emu_model_tensor")
        return p.value, n.value

    def tensor_lane_major(self, kind: int, layer: int = 0) -> tuple[int, int]:
        """Address and size of the lane-major copy the batch-1 matvec reads."""
        p, n = C.c_void_p(), C.c_size_t()
        self.ctx.check(self.ctx.lib.emu_model_tensor_lane_major(self.h, kind, layer, C.byref(p), C.byref(n)),
                       "emu_model_tensor_lane_major")
        return p.value, n.value

    def read_tensor(self, kind: int, layer: int = 0, dtype=np.uint8) -> np.ndarray:
        addr, n = self.tensor(kind, layer)
        out = np.empty(n, np.uint8)
        self.ctx.check(self.ctx.lib.emu_memcpy_dtoh(self.ctx.h, out.ctypes.data_as(C.c_void_p),
                                                    C.c_void_p(addr), n), "emu_memcpy_dtoh")
        return out.view(dtype)

    def write_tensor(self, kind: int, data: np.ndarray, layer: int = 0) -> None:
        addr, n = self.tensor(kind, layer)
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        if data.size != n:
            raise ValueError(f"tensor holds {n} bytes, got {data.size}")
        self.ctx.check(self.ctx.lib.emu_memcpy_htod(self.ctx.h, C.c_void_p(addr),
                                                    data.ctypes.data_as(C.c_void_p), n), "emu_memcpy_htod")

    def weight_bytes(self) -> int:
        v = C.c_uint64()
        self.ctx.check(self.ctx.lib.emu_model_weight_bytes(self.h, C.byref(v)), "emu_model_weight_bytes")
        return v.value

    def resident_bytes(self) -> int:
        """HBM held by the parameters: GGUF order plus the derived copies."""
        v = C.c_uint64()
        self.ctx.check(self.ctx.lib.emu_model_resident_bytes(self.h, C.byref(v)), "emu_model_resident_bytes")
        return v.value

    def host_weights(self) -> dict:
        """Every tensor copied to host memory (for the checker)."""
        c = self.cfg
        layers = np.concatenate([self.read_tensor(EMU_T_LAYER, l) for l in range(c.layers)])
        out = {
            "layers": layers,
            "embed": self.read_tensor(EMU_T_EMBED),
            "attn_norm": self.read_tensor(EMU_T_ATTN_NORM, dtype=np.float32),
            "ffn_norm": self.read_tensor(EMU_T_FFN_NORM, dtype=np.float32),
            "q_norm": self.read_tensor(EMU_T_Q_NORM, dtype=np.float32),
            "k_norm": self.read_tensor(EMU_T_K_NORM, dtype=np.float32),
            "out_norm": self.read_tensor(EMU_T_OUT_NORM, dtype=np.float32),
        }
        out["output"] = out["embed"] if c.tied else self.read_tensor(EMU_T_OUTPUT)
        if c.gemma:
            out["ffn_norm2"] = self.read_tensor(EMU_T_FFN_NORM2, dtype=np.float32)
        return out


class Session:
    """A set of clients decoding in lockstep (emu_session)."""

    def __init__(self, model: Model, n_clients: int, context: int, kv_f16: bool = True):
        self.model, self.ctx = model, model.ctx
        self.n, self.context, self.kv_f16 = n_clients, context, kv_f16
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.emu_session_create(model.h, n_clients, context, int(kv_f16), C.byref(h)),
                       "emu_session_create")
        self.h = h

    def close(self) -> None:
        if self.h is not None and self.ctx.live:
            self.ctx.lib.emu_session_destroy(self.h)
        self.h = None

    def __del__(self):  # pragma: no cover
        if not sys.is_finalizing():
            try:
                self.close()
            except Exception:
                pass

    def reset(self) -> None:
        self.ctx.check(self.ctx.lib.emu_session_reset(self.h), "emu_session_reset")

    def reset_client(self, client: int) -> None:
        """Replace one client by a fresh one; the others keep their state."""
        self.ctx.check(self.ctx.lib.emu_session_reset_client(self.h, client), "emu_session_reset_client")

    def decode_step(self, tokens, want_logits: bool = False):
        toks = np.ascontiguousarray(tokens, np.uint32)
        nxt = np.empty(self.n, np.uint32)
        logits_buf = self.ctx.alloc(self.n * self.model.cfg.vocab * 4) if want_logits else None
        self.ctx.check(self.ctx.lib.emu_decode_step(self.h, toks.ctypes.data_as(C.c_void_p),
                                                    nxt.ctypes.data_as(C.c_void_p),
                                                    logits_buf.ptr if logits_buf else None), "emu_decode_step")
        if want_logits:
            return nxt, logits_buf.read(np.float32).reshape(self.n, self.model.cfg.vocab)
        return nxt

    def generate(self, prompts: np.ndarray, steps: int) -> np.ndarray:
        prompts = np.ascontiguousarray(prompts, np.uint32).reshape(self.n, -1)
        out = np.empty((self.n, steps), np.uint32)
        self.ctx.check(self.ctx.lib.emu_generate(self.h, prompts.ctypes.data_as(C.c_void_p), prompts.shape[1],
                                                 steps, out.ctypes.data_as(C.c_void_p)), "emu_generate")
        return out

    def time_decode(self, steps: int) -> float:
        ms = C.c_float()
        self.ctx.check(self.ctx.lib.emu_time_decode(self.h, steps, C.byref(ms)), "emu_time_decode")
        return ms.value

    def set_options(self, f32_act: bool = False, direct: bool = False) -> None:
        """f32_act: f32 activations in every matvec and expert (the int8-limb
        kernels otherwise); direct: launch the step's kernels one by one
        instead of replaying a captured graph."""
        flags = (_lib.EMU_SESSION_F32_ACT if f32_act else 0) | (_lib.EMU_SESSION_DIRECT if direct else 0)
        self.ctx.check(self.ctx.lib.emu_session_set_options(self.h, flags), "emu_session_set_options")

    def attach_cache(self, cache) -> None:
        """Read the experts through an ExpertCache (its policy then runs on
        the device, inside the step); None detaches."""
        self.ctx.check(self.ctx.lib.emu_session_attach_expert_cache(self.h, cache.h if cache else None),
                       "emu_session_attach_expert_cache")

    def time_layers(self) -> np.ndarray:
        """One decode step timed interval by interval (microseconds): the
        embedding, each layer, then the output matvec and selection."""
        out = np.zeros(self.model.cfg.layers + 2, np.float32)
        self.ctx.check(self.ctx.lib.emu_session_time_layers(self.h, out.ctypes.data_as(C.c_void_p), out.size),
                       "emu_session_time_layers")
        return out

    def route_zipf(self, s: float, seed: int = 0) -> None:
        """Zipf(s) routing for throughput runs (0: the model's own router)."""
        self.ctx.check(self.ctx.lib.emu_session_route_zipf(self.h, float(s), int(seed)), "emu_session_route_zipf")

    def route_trace(self, capacity: int) -> None:
        """Record the routes of every step on the device (capacity steps)."""
        self.ctx.check(self.ctx.lib.emu_session_route_trace(self.h, int(capacity)), "emu_session_route_trace")
        self._trace_cap = int(capacity)

    def read_routes(self, slot: int) -> tuple[np.ndarray, np.ndarray]:
        """(ids, weights) of one trace slot: layers x clients x k."""
        c = self.model.cfg
        ids = np.empty((c.layers, self.n, c.experts_used), np.int32)
        w = np.empty((c.layers, self.n, c.experts_used), np.float32)
        self.ctx.check(self.ctx.lib.emu_session_read_routes(self.h, int(slot), ids.ctypes.data_as(C.c_void_p),
                                                            w.ctypes.data_as(C.c_void_p)), "emu_session_read_routes")
        return ids, w

    def positions(self) -> np.ndarray:
        out = np.empty(self.n, np.uint32)
        self.ctx.check(self.ctx.lib.emu_session_positions(self.h, out.ctypes.data_as(C.c_void_p)),
                       "emu_session_positions")
        return out

    def read_kv(self, client: int, layer: int, values: bool, positions: int) -> np.ndarray:
        out = np.empty(positions * self.model.cfg.kv_width, np.float32)
        self.ctx.check(self.ctx.lib.emu_session_read_kv(self.h, client, layer, int(values),
                                                        out.ctypes.data_as(C.c_void_p), positions),
                       "emu_session_read_kv")
        return out.reshape(positions, -1)


__all__ = ["DenseConfig", "Model", "Session", "QWEN3_8B_Q6K", "SMOLLM2_135M_Q8", "GRANITE_MOE_Q6K", "OLMOE_1B_7B",
           "GEMMA4_MOE", "_lib"]
